"""A transformer inference block end to end through the libraries' C ABI.

The reference's library-breadth exit gate (ref
docs/designs/grxcp_roadmap.md:870-877): "a transformer inference workload
(attention + GEMM + layernorm + softmax) runs end-to-end through GRXCP
libraries with numerical agreement against a PyTorch CPU reference". Here a
pre-LayerNorm block (GPT style) plus the output projection and softmax runs
only through grxblasGemmEx and grxDNN calls on device buffers:

  h  = LayerNorm(x)                      grxdnnLayerNormForward
  qkv = h Wqkv^T                         grxblasGemmEx (T, N): weights [out, in]
  o  = causal attention(q, k, v)         grxdnnAttentionForward, strided
                                         views into qkv, o written as [T, d]
  x2 = x + o Wo^T                        GemmEx with beta = 1 on a copy of x
  u  = GELU_tanh(LayerNorm(x2) W1^T)     LayerNorm, GemmEx, grxdnnGeluForward in place
  x3 = x2 + u W2^T                       GemmEx, beta = 1
  p  = softmax(LayerNorm(x3) Wout^T)     LayerNorm, GemmEx to fp32, grxdnnSoftmaxForward

The reference computes the same graph with torch on the CPU in float32,
rounding to bfloat16 where the library chain stores bfloat16. Agreement:
normwise relative error <= 2e-2 on the residual stream and the logits, and
<= 2e-2 of the largest probability on the probabilities.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import grxcp_amd as g
from helpers import normwise_rel_err, say, to_dev

pytestmark = pytest.mark.gpu

BF16, F32 = g.GRX_R_16BF, g.GRX_R_32F


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, shape) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(shape).float()


def test_transformer_block_matches_torch_cpu(blas, dnn):
    torch.manual_seed(0)
    B, S, H, D = 2, 256, 8, 64
    dm, dff, V, T = H * D, 4 * H * D, 1000, B * S
    eps = 1e-5

    def w(out, inp):
        return (torch.randn(out, inp) / inp ** 0.5).bfloat16()

    x = torch.randn(T, dm).bfloat16()
    ln = [((1 + 0.1 * torch.randn(dm)).bfloat16(), (0.1 * torch.randn(dm)).bfloat16()) for _ in range(3)]
    Wqkv, Wo, W1, W2, Wout = w(3 * dm, dm), w(dm, dm), w(dff, dm), w(dm, dff), w(V, dm)

    # ---- device chain
    dev = {name: to_dev(bits(t)) for name, t in
           [("x", x), ("Wqkv", Wqkv), ("Wo", Wo), ("W1", W1), ("W2", W2), ("Wout", Wout)]}
    lnd = [(to_dev(bits(gm)), to_dev(bits(bt))) for gm, bt in ln]
    buf = {name: g.DeviceBuffer(n * 2) for name, n in
           [("h", T * dm), ("qkv", T * 3 * dm), ("o", T * dm), ("x2", T * dm), ("u", T * dff),
            ("x3", T * dm)]}
    logits = g.DeviceBuffer(T * V * 4)
    probs = g.DeviceBuffer(T * V * 4)
    act = g.TensorDesc(BF16, [T, dm])
    wdesc = g.TensorDesc(BF16, [dm])

    def linear(W, k, n_out, src, dst, ctype=BF16, beta=0.0):
        s = blas.gemm_ex(1, 0, n_out, T, k, 1.0, dev[W].p, BF16, k, src.p, BF16, k, beta, dst.p, ctype, n_out)
        assert s == g.SUCCESS, (W, g.STATUS[s])

    def layernorm(i, src, dst):
        s = dnn.layernorm(act, src.p, wdesc, lnd[i][0].p, lnd[i][1].p, eps, act, dst.p)
        assert s == g.SUCCESS, g.STATUS[s]

    def d2d(dst, src, nbytes):
        g.check_rt(g.load().rt.grxMemcpy(dst.p, src.p, ctypes.c_size_t(nbytes), 3), "grxMemcpy")

    say("transformer block: attention half")
    layernorm(0, dev["x"], buf["h"])
    linear("Wqkv", dm, 3 * dm, buf["h"], buf["qkv"])
    # q/k/v: [B, H, S, D] views of qkv[T, 3*dm]; o written straight into [T, dm]
    qkv_strides = [S * 3 * dm, D, 3 * dm, 1]
    qd = g.TensorDesc(BF16, [B, H, S, D], qkv_strides)
    od = g.TensorDesc(BF16, [B, H, S, D], [S * dm, D, dm, 1])
    ad = g.AttnDesc(True, D ** -0.5)
    base = buf["qkv"].ptr.value
    s = dnn.attention(ad, qd, ctypes.c_void_p(base), qd, ctypes.c_void_p(base + 2 * dm),
                      qd, ctypes.c_void_p(base + 4 * dm), od, buf["o"].p)
    assert s == g.SUCCESS, g.STATUS[s]
    d2d(buf["x2"], dev["x"], T * dm * 2)
    linear("Wo", dm, dm, buf["o"], buf["x2"], beta=1.0)
    say("transformer block: MLP half")
    layernorm(1, buf["x2"], buf["h"])
    linear("W1", dm, dff, buf["h"], buf["u"])
    ud = g.TensorDesc(BF16, [T, dff])
    assert dnn.gelu(g.GELU_TANH, ud, buf["u"].p, ud, buf["u"].p) == g.SUCCESS
    d2d(buf["x3"], buf["x2"], T * dm * 2)
    linear("W2", dff, dm, buf["u"], buf["x3"], beta=1.0)
    say("transformer block: output softmax")
    layernorm(2, buf["x3"], buf["h"])
    linear("Wout", dm, V, buf["h"], logits, ctype=F32)
    ld = g.TensorDesc(F32, [T, V])
    assert dnn.softmax(ld, logits.p, ld, probs.p) == g.SUCCESS
    g.synchronize()
    x3_gpu = from_bits(buf["x3"].download(np.uint16, T * dm), (T, dm))
    logits_gpu = torch.from_numpy(logits.download(np.float32, T * V).reshape(T, V))
    probs_gpu = torch.from_numpy(probs.download(np.float32, T * V).reshape(T, V))

    # ---- torch CPU reference, bf16 where the chain stores bf16
    def lnf(t, i):
        return F.layer_norm(t.float(), (dm,), ln[i][0].float(), ln[i][1].float(), eps).bfloat16()

    h = lnf(x, 0)
    qkv = (h.float() @ Wqkv.float().T).bfloat16()
    q, k, v = qkv.float().view(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=D ** -0.5).bfloat16()
    o = o.float().permute(0, 2, 1, 3).reshape(T, dm)
    x2 = (x.float() + o @ Wo.float().T).bfloat16()
    u = (lnf(x2, 1).float() @ W1.float().T).bfloat16()
    u = F.gelu(u.float(), approximate="tanh").bfloat16()
    x3 = (x2.float() + u.float() @ W2.float().T).bfloat16()
    lg = lnf(x3, 2).float() @ Wout.float().T
    pr = torch.softmax(lg, dim=-1)

    assert normwise_rel_err(x3_gpu.numpy(), x3.float().numpy()) <= 2e-2
    assert normwise_rel_err(logits_gpu.numpy(), lg.numpy()) <= 2e-2
    assert float((probs_gpu - pr).abs().max()) <= 2e-2 * float(pr.max())
    np.testing.assert_allclose(probs_gpu.sum(dim=-1).numpy(), 1.0, rtol=1e-5)
    # the most likely token agrees wherever the reference's top two are not a near tie
    top2 = torch.topk(pr, 2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 1e-3
    assert torch.equal(probs_gpu.argmax(-1)[clear], pr.argmax(-1)[clear])
