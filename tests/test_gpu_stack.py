"""The config-3 decode step (viper_amd.stack) on the GPU: wiring checked
against a CPU oracle chain at small dimensions, and run-to-run determinism.

Each kernel's own parity is pinned in the other GPU test files; here the
point is that every launch reads and writes the right buffers, so the
comparison is loose (5% of the logit scale) and the greedy token must match
unless the oracle's top two logits are closer than that.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (run them on the MI355X box)")
    return torch


def u16(t):
    return t.contiguous().view(__import__("torch").int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("fused", [False, True])
def test_stack_step_wiring_and_determinism(torch_dev, fused):
    torch = torch_dev
    from viper_amd.stack import Stack
    s = Stack(torch, hidden=256, inter=512, n_heads=2, n_kv_heads=1, head_dim=128, layers=2, passes=2,
              vocab=1000, seed=7)
    run = s.step_fused if fused else s.step
    run()
    torch.cuda.synchronize()
    logits = u16(s.logits)
    token = int(s.token.item())
    run()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(s.logits), logits)

    # oracle chain
    H, I, nQ = s.H, s.I, s.nQ
    x = u16(s.x0)
    attn = u16(s.attn)
    W = [[(p.cpu().numpy(), sc.view(torch.int16).cpu().numpy().view(np.uint16), n, k) for (p, sc, n, k) in lw]
         for lw in s.w]
    ln = [u16(t)[None, :][0] for t in s.ln]
    for loop in range(s.passes):
        for l in range(s.layers):
            wq, wk, wv, wo, wg, wu, wd = W[l]
            xn = O.rmsnorm_bf16(x, ln[2 * l], s.eps)
            xq, xs = O.quantize_act(attn, 64)
            y, _, _ = O.qlinear_prequant(O.Q4_G64, wo[0], wo[1], O.SCALE_FP16, H, nQ, xq, xs, residual=x)
            x = y
            xn = O.rmsnorm_bf16(x, ln[2 * l + 1], s.eps)
            g, _, _ = O.qlinear(O.Q4_G64, wg[0], wg[1], O.SCALE_FP16, I, H, xn)
            u, _, _ = O.qlinear(O.Q4_G64, wu[0], wu[1], O.SCALE_FP16, I, H, xn)
            h = O.swiglu_bf16(g, u)
            xq, xs = O.quantize_act(h, 64)
            x, _, _ = O.qlinear_prequant(O.Q4_G64, wd[0], wd[1], O.SCALE_FP16, H, I, xq, xs, residual=x)
    xn = O.rmsnorm_bf16(x, u16(s.final_ln), s.eps)
    ref, _, _ = O.linear_bf16(u16(s.head), xn)
    rf, gf = O.bf16_to_f32(ref[0]).astype(np.float64), O.bf16_to_f32(logits[0]).astype(np.float64)
    scale = np.abs(rf).max()
    assert np.abs(gf - rf).max() <= 0.05 * scale
    top = np.sort(rf)[-2:]
    if top[1] - top[0] > 0.1 * scale:
        assert token == int(np.argmax(rf))
    assert token == int(O.argmax_bf16(logits)[0])
