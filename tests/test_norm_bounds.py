"""The GPU norm checks can fail: planted mistakes, on the CPU.

tests/test_gpu_dnn.py holds every norm output to `norm_bound` (half an output
ulp plus fp32 arithmetic) and pins eps with `eps_rows` at `EPS_CASES`. Here a
kernel that dropped eps is stood in for by the oracle with eps dropped
(oracle mutation 4), and a kernel with a 1 % scale error by the correct
result times 1.01, each rounded to bf16 as the kernel's output would be: the
GPU tests' own check must reject both, on the same inputs. The correct
result, rounded to bf16, must pass (the bound is not too tight).
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_dnn import BF16, EPS_CASES, eps_rows, norm_violations


@pytest.fixture(autouse=True)
def _no_mutation():
    O.set_mutation(0)
    yield
    O.set_mutation(0)


def _inputs(hidden):
    r = np.random.default_rng(hidden + 1)
    x = O.bf16_to_f32(O.f32_to_bf16(eps_rows(hidden)))
    gamma = O.bf16_to_f32(O.f32_to_bf16((1 + 0.02 * r.standard_normal(hidden)).astype(np.float32)))
    beta = O.bf16_to_f32(O.f32_to_bf16((0.02 * r.standard_normal(hidden)).astype(np.float32)))
    return x, gamma, beta


def _norm(layer, x, gamma, beta, eps):
    return O.layernorm(x, gamma, beta, eps) if layer else O.rmsnorm(x, gamma, eps)


def _as_kernel_output(y):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(y, np.float32)))


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("eps,hidden", EPS_CASES)
def test_correct_result_passes_and_dropped_eps_fails(layer, eps, hidden):
    x, gamma, beta = _inputs(hidden)
    b = beta if layer else None
    ref = _norm(layer, x, gamma, beta, eps)
    assert norm_violations(_as_kernel_output(ref), ref, b, BF16) == 0
    O.set_mutation(4)                       # the oracle's norms drop eps
    with np.errstate(invalid="ignore", divide="ignore"):
        wrong = _as_kernel_output(_norm(layer, x, gamma, beta, eps))
    O.set_mutation(0)
    assert norm_violations(wrong, ref, b, BF16) > 0


@pytest.mark.parametrize("layer", [False, True])
def test_one_percent_scale_error_fails(layer):
    r = np.random.default_rng(5)
    hidden = 8192
    x = O.bf16_to_f32(O.f32_to_bf16(r.standard_normal((8, hidden)).astype(np.float32)))
    gamma = O.bf16_to_f32(O.f32_to_bf16((1 + 0.02 * r.standard_normal(hidden)).astype(np.float32)))
    beta = O.bf16_to_f32(O.f32_to_bf16((0.02 * r.standard_normal(hidden)).astype(np.float32)))
    ref = _norm(layer, x, gamma, beta, 1e-6)
    b = beta if layer else None
    assert norm_violations(_as_kernel_output(ref), ref, b, BF16) == 0
    assert norm_violations(_as_kernel_output(ref * 1.01), ref, b, BF16) > 0
