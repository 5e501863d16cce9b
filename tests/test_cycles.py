"""grxCycleSummarize (include/grx/grx_cycles.h), host only.

The summary semantics follow the reference's header
(ref include/grx/grx_cycles.h:67-99): slots left all-zero were never written
and are skipped; the span (last end - first start) is only reported when every
written slot came from one core (one clock domain), otherwise spanIsValid = 0
and cores = 2 ("more than one"); busy = end - start per slot, min / median
(element n/2 of the sorted list) / max. The expected values below are worked
out by hand from those rules.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def summarize(tmp_path_factory):
    gxx = shutil.which("g++")
    assert gxx, "g++ is part of this image"
    exe = str(tmp_path_factory.mktemp("cycles") / "cycle_summary")
    subprocess.run([gxx, "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cycle_summary_main.cpp"), "-o", exe], check=True)

    def run(slots):
        text = "".join(f"{a} {b} {c} {w}\n" for a, b, c, w in slots)
        out = subprocess.run([exe], input=text, capture_output=True, text=True, check=True).stdout
        keys = ["warps", "cores", "span_valid", "span", "busy_min", "busy_median", "busy_max"]
        return dict(zip(keys, map(int, out.split())))
    return run


def test_empty_and_unwritten(summarize):
    zero = dict(warps=0, cores=0, span_valid=0, span=0, busy_min=0, busy_median=0, busy_max=0)
    assert summarize([]) == zero
    assert summarize([(0, 0, 0, 0)] * 5) == zero


def test_one_core(summarize):
    # busy = 100, 40, 280 -> sorted 40, 100, 280; span = 400 - 100
    slots = [(100, 200, 7, 0), (0, 0, 0, 0), (110, 150, 7, 1), (120, 400, 7, 2)]
    assert summarize(slots) == dict(warps=3, cores=1, span_valid=1, span=300,
                                    busy_min=40, busy_median=100, busy_max=280)


def test_even_count_median_is_upper_middle(summarize):
    slots = [(0, 10, 1, 0), (0, 30, 1, 1), (0, 20, 1, 2), (0, 40, 1, 3)]
    s = summarize(slots)
    assert (s["busy_min"], s["busy_median"], s["busy_max"]) == (10, 30, 40)


def test_two_cores_invalidate_the_span(summarize):
    slots = [(100, 200, 1, 0), (100, 300, 2, 0)]
    assert summarize(slots) == dict(warps=2, cores=2, span_valid=0, span=0,
                                    busy_min=100, busy_median=200, busy_max=200)


def test_slot_starting_at_zero_counts_when_written(summarize):
    # only the all-zero slot is "unwritten"; start 0 with end > 0 is a record
    s = summarize([(0, 50, 3, 0), (10, 20, 3, 1)])
    assert s["warps"] == 2 and s["span"] == 50
