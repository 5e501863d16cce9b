"""Shared helpers for the GPU parity tests (host-side only)."""
import sys

import numpy as np

import grxcp_amd as g


def say(msg: str) -> None:
    """Name the case before a GPU step, flushed, so a crash log names it."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()


def col_major(mat: np.ndarray, ld: int) -> np.ndarray:
    rows, cols = mat.shape
    buf = np.zeros(ld * cols, mat.dtype)
    view = buf.reshape(cols, ld)
    view[:, :rows] = mat.T
    return buf


def from_col_major(buf: np.ndarray, rows: int, cols: int, ld: int) -> np.ndarray:
    return buf[: ld * cols].reshape(cols, ld)[:, :rows].T


def window_mask(rows: int, cols: int, ld: int) -> np.ndarray:
    """True inside the rows x cols window of a column-major ld buffer."""
    m = np.zeros((cols, ld), bool)
    m[:, :rows] = True
    return m.reshape(-1)


def normwise_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref|: the relative error the gates bound."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


def to_dev(a: np.ndarray) -> g.DeviceBuffer:
    return g.DeviceBuffer.from_array(a)


GUARD = 4096
POISON = 0xA5


class Guarded:
    """A device buffer holding `init`'s bytes between two 4 KB guard bands
    filled with POISON: a kernel that writes outside its output changes
    a guard band."""

    def __init__(self, init: np.ndarray):
        init = np.ascontiguousarray(init)
        self.n = init.nbytes
        self.buf = g.DeviceBuffer(self.n + 2 * GUARD)
        self.buf.upload(np.full(self.n + 2 * GUARD, POISON, np.uint8))
        self.buf.upload(init, offset=GUARD)
        self.p = self.buf.ptr.value + GUARD

    def download(self, dtype, count=None) -> np.ndarray:
        if count is None:
            count = self.n // np.dtype(dtype).itemsize
        return self.buf.download(dtype, count, offset=GUARD)

    def guards_intact(self) -> bool:
        lo = self.buf.download(np.uint8, GUARD, offset=0)
        hi = self.buf.download(np.uint8, GUARD, offset=GUARD + self.n)
        return bool((lo == POISON).all() and (hi == POISON).all())
