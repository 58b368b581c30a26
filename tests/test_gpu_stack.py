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


def _close_bits(hd, hr, what):
    """Within 1 bf16 ulp (1 in the bit pattern) outside the flush-to-zero range."""
    tiny = 2.0 ** -100
    small = np.abs(O.bf16_to_f32(hr)) < tiny
    assert (np.abs(O.bf16_to_f32(hd))[small] < tiny).all(), what
    d = np.abs(hd.astype(np.int32) - hr.astype(np.int32))[~small]
    assert int(d.max(initial=0)) <= 1, f"{what}: {int(d.max())} bf16 steps"


@pytest.mark.parametrize("fused", [False, True])
def test_stack_production_size_every_launch(torch_dev, fused):
    """The config-3 step at its real size (hidden 2560, intermediate 10240,
    20/4 heads of 128, 22 layers looped twice, vocab 166144), every launch of
    all 44 slots checked against the oracle on the GPU's own inputs (teacher
    forcing, so each launch is held to the single-kernel bar: GEMV outputs
    within 1 bf16 ulp or 1e-5 of the sum of |terms|, rmsnorm and swiglu rows
    within 1 ulp), then the LM head and the greedy token; finally the same
    step untraced must give the traced run's logits bit for bit."""
    torch = torch_dev
    from viper_amd.stack import Stack
    s = Stack(torch)
    print(f"stack production size fused={fused}", flush=True)
    H, I, nQ, nKV = s.H, s.I, s.nQ, s.nKV
    W = [[(pk.cpu().numpy(), sc.view(torch.int16).cpu().numpy().view(np.uint16), n, k) for (pk, sc, n, k) in lw]
         for lw in s.w]
    ln = [u16(t) for t in s.ln]
    attn = u16(s.attn)
    Q4, F16 = O.Q4_G64, O.SCALE_FP16

    def gemv(w, x, residual=None):
        return O.qlinear_omp(Q4, w[0], w[1], F16, w[2], w[3], x, residual=residual, full=True)

    s.trace = True
    s.x.copy_(s.x0)
    for slot in range(s.layers * s.passes):
        l = slot % s.layers
        wq, wk, wv, wo, wg, wu, wd = W[l]
        x_in = u16(s.x)
        s.attention_half(slot, fused)
        torch.cuda.synchronize()
        xn = u16(s.xn)
        _close_bits(xn[0], O.rmsnorm_bf16(x_in, ln[2 * l], s.eps)[0], f"slot {slot} input rmsnorm")
        for w, out, name in ((wq, s.q, "q"), (wk, s.k, "k"), (wv, s.v, "v")):
            y, _, a = gemv(w, xn)
            O.assert_bf16_close(u16(out), y, a, rel=1e-5, what=f"slot {slot} {name}")
        x_mid = u16(s.x)
        y, _, a = gemv(wo, attn, residual=x_in)
        O.assert_bf16_close(x_mid, y, a, rel=1e-5, what=f"slot {slot} o + residual")

        s.mlp_half(slot, fused)
        torch.cuda.synchronize()
        xn = u16(s.xn)
        _close_bits(xn[0], O.rmsnorm_bf16(x_mid, ln[2 * l + 1], s.eps)[0], f"slot {slot} post rmsnorm")
        g, u, h = u16(s.g), u16(s.ut), u16(s.gt)
        for w, out, name in ((wg, g, "gate"), (wu, u, "up")):
            y, _, a = gemv(w, xn)
            O.assert_bf16_close(out, y, a, rel=1e-5, what=f"slot {slot} {name}")
        _close_bits(h[0], O.swiglu_bf16(g, u)[0], f"slot {slot} swiglu")
        y, _, a = gemv(wd, h, residual=x_mid)
        O.assert_bf16_close(u16(s.x), y, a, rel=1e-5, what=f"slot {slot} down + residual")

    x_fin = u16(s.x)
    s.head_step(fused)
    torch.cuda.synchronize()
    xn = u16(s.xn)
    _close_bits(xn[0], O.rmsnorm_bf16(x_fin, u16(s.final_ln), s.eps)[0], "final rmsnorm")
    logits = u16(s.logits)
    y, _, a = O.linear_bf16(u16(s.head), xn)
    O.assert_bf16_close(logits, y, a, rel=1e-5, what="lm_head")
    token = int(s.token.item())
    assert token == int(O.argmax_bf16(logits)[0])

    s.trace = False
    (s.step_fused if fused else s.step)()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(s.logits), logits)
    assert int(s.token.item()) == token


@pytest.mark.parametrize("fused", [False, True])
def test_stack_step_graph_replays_equal_eager(torch_dev, fused):
    """The decode step captured in one HIP graph (as the bench times it): three replays, with eager
    steps between them, each give the eager step's logits and token bit for bit (the split greedy
    pick's workspace is left zero by every call, so replays need no clearing)."""
    torch = torch_dev
    from viper_amd.stack import Stack
    s = Stack(torch, hidden=512, inter=1024, n_heads=4, n_kv_heads=1, head_dim=128, layers=3, passes=2,
              vocab=20000, seed=11)
    run = s.step_fused if fused else s.step
    run()
    torch.cuda.synchronize()
    logits, token = u16(s.logits), int(s.token.item())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for i in range(3):
        s.logits.zero_()
        s.token.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u16(s.logits), logits, err_msg=f"replay {i}")
        assert int(s.token.item()) == token
        run()   # eager work between the replays
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u16(s.logits), logits)
    assert int(s.greedy_ws.count_nonzero()) == 0


def test_stack_step_prefetch_equals_plain(torch_dev):
    """The fused step with the next slot's weights warmed from a second stream
    (viper_hip_prefetch) gives the plain fused step's logits and token bit for
    bit, eagerly and as graph replays (the warming only reads)."""
    torch = torch_dev
    from viper_amd.stack import Stack
    s = Stack(torch, hidden=512, inter=1024, n_heads=4, n_kv_heads=1, head_dim=128, layers=3, passes=2,
              vocab=20000, seed=13)
    s.step_fused()
    torch.cuda.synchronize()
    logits, token = u16(s.logits), int(s.token.item())
    s.step_fused(prefetch=64)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(s.logits), logits)
    assert int(s.token.item()) == token
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s.step_fused(prefetch=64)
    for i in range(2):
        s.logits.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u16(s.logits), logits, err_msg=f"replay {i}")
        assert int(s.token.item()) == token
    assert int(s.sink.item()) == 0
