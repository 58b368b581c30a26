"""GPU parity of viper_hip_qlinear_m1: producers folded into the M = 1 GEMV
prologue and up to three matrices per launch.

The folded prologues run the same arithmetic as the standalone producer
kernels, so at the engine's shapes (K = 2560 rmsnorm with 320 threads on both
sides, swiglu element-wise) the outputs must equal the two-launch chain bit
for bit; elsewhere they are checked against the oracle chain fed with the
kernel's own normalized row (norm_out), to the usual bar.
"""
import numpy as np
import pytest

import oracle as O
import viper_amd as va

pytestmark = pytest.mark.gpu
P = va.Prologue


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (run them on the MI355X box)")
    return torch


def dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to("cuda")


def u16(t):
    return t.cpu().numpy().view(np.uint16)


def weights(torch, qtype, N, K, seed, senc=O.SCALE_FP16):
    G = O.group_size(qtype)
    p, s = O.gen_weights(qtype, N, K, seed, senc)
    return va.QuantizedWeight(va.QType(qtype), dev(torch, p), dev(torch, s), N, K, G, va.ScaleEnc(senc)), p, s


def bf16(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


def test_rmsnorm_qkv_equals_two_launches(torch_dev):
    # engine shape: q (2560), k and v (512) from rmsnorm(x) in one launch
    torch = torch_dev
    K, eps = 2560, 1e-6
    ws = [weights(torch, O.Q4_G64, n, K, 500 + i)[0] for i, n in enumerate((2560, 512, 512))]
    x = dev(torch, O.gen_act(1, K, 510, outlier_frac=0.02))
    rng = np.random.default_rng(511)
    gamma = dev(torch, bf16(1.0 + 0.1 * rng.standard_normal(K)))
    ys = [torch.zeros((1, w.rows), dtype=torch.int16, device="cuda") for w in ws]
    norm = torch.zeros((1, K), dtype=torch.int16, device="cuda")
    assert va.linear_m1(ws, P.RMSNORM, x, gamma, ys, eps=eps, norm_out=norm).ok()
    # two-launch chain
    xq = torch.zeros((1, K), dtype=torch.int8, device="cuda")
    xs = torch.zeros((1, K // 64), dtype=torch.float32, device="cuda")
    norm2 = torch.zeros_like(norm)
    assert va.rmsnorm_quantize(x, gamma, eps, 64, xq, xs, out=norm2).ok()
    refs = [torch.zeros_like(y) for y in ys]
    for w, r in zip(ws, refs):
        assert va.linear_prequantized(w, xq, xs, r).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(norm), u16(norm2))
    for y, r in zip(ys, refs):
        np.testing.assert_array_equal(u16(y), u16(r))


@pytest.mark.parametrize("K,N", [(10240, 2560), (10752, 3072)])
def test_swiglu_down_residual_equals_two_launches(torch_dev, K, N):
    # engine shapes: down (K=10240, N=2560; the reference's K=10752, N=3072 on
    # the masked tiling) from silu(gate) * up, residual in place
    torch = torch_dev
    w = weights(torch, O.Q4_G64, N, K, 520)[0]
    rng = np.random.default_rng(521)
    g = dev(torch, bf16(3.0 * rng.standard_normal((1, K))))
    u = dev(torch, bf16(rng.standard_normal((1, K))))
    res = O.gen_act(1, N, 522)
    y = dev(torch, res)
    assert va.linear_m1([w], P.SWIGLU, g, u, [y], residual=y).ok()
    xq = torch.zeros((1, K), dtype=torch.int8, device="cuda")
    xs = torch.zeros((1, K // 64), dtype=torch.float32, device="cuda")
    assert va.swiglu_quantize(g, u, 64, xq, xs).ok()
    r = dev(torch, res)
    assert va.linear_prequantized(w, xq, xs, r, residual=r).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(y), u16(r))


# gate/up pair with the swiglu epilogue: equal, bit for bit, to the two GEMVs
# of one viper_hip_qlinear_m1 launch followed by the standalone swiglu kernel;
# the engine shape (rmsnorm prologue, K=2560, N=10240), the bf16 prologue,
# every format, exact and masked tilings, ragged N, optional gate/up outputs.
@pytest.mark.parametrize("qtype,N,K,pro", [
    (O.Q4_G64, 10240, 2560, P.RMSNORM),
    (O.Q4_G64, 1000, 2560, P.BF16),
    (O.Q4_G64, 333, 1536, P.RMSNORM),
    (O.Q5_G64, 2100, 2560, P.BF16),
    (O.Q6_G64, 517, 4096, P.RMSNORM),
    (O.W8_G32, 777, 2560, P.BF16),
    (O.Q4_G64, 2560, 10240, P.BF16),
    (O.Q4_G64, 10752, 3072, P.RMSNORM),   # the reference engine's gate / up (6-slot tiling)
    (O.Q5_G64, 1000, 10752, P.BF16),      # masked tiling
])
def test_gate_up_swiglu_equals_chain(torch_dev, qtype, N, K, pro):
    torch = torch_dev
    print(f"gate_up_swiglu qtype={qtype} N={N} K={K} pro={int(pro)}", flush=True)
    eps = 1e-6
    wg = weights(torch, qtype, N, K, 540 + K)[0]
    wu = weights(torch, qtype, N, K, 541 + K)[0]
    x = dev(torch, O.gen_act(1, K, 542, outlier_frac=0.02))
    rng = np.random.default_rng(543)
    gamma = dev(torch, bf16(1.0 + 0.1 * rng.standard_normal(K))) if pro == P.RMSNORM else None
    z = lambda: torch.zeros((1, N), dtype=torch.int16, device="cuda")
    h, g1, u1, h_only = z(), z(), z(), z()
    assert va.linear_m1_swiglu(wg, wu, pro, x, gamma, h, eps=eps, gate_out=g1, up_out=u1).ok()
    assert va.linear_m1_swiglu(wg, wu, pro, x, gamma, h_only, eps=eps).ok()
    # chain: one launch for both GEMVs, then the standalone swiglu (its int8 output unused here)
    g2, u2, h2 = z(), z(), z()
    assert va.linear_m1([wg, wu], pro, x, gamma, [g2, u2], eps=eps).ok()
    G = O.group_size(qtype)
    xq = torch.zeros((1, N), dtype=torch.int8, device="cuda")
    xs = torch.zeros((1, max(N // G, 1)), dtype=torch.float32, device="cuda")
    if N % G == 0:
        assert va.swiglu_quantize(g2, u2, G, xq, xs, out=h2).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(g1), u16(g2))
    np.testing.assert_array_equal(u16(u1), u16(u2))
    np.testing.assert_array_equal(u16(h), u16(h_only))
    if N % G == 0:
        np.testing.assert_array_equal(u16(h), u16(h2))
    # the product against the oracle's swiglu of the device's own gate/up: within 1 bf16 ulp.
    # Below 2^-100 in magnitude both sides only need to be below 2^-100: for gate < -87 the
    # hardware reciprocal of 1 + exp(-gate) > 2^126 flushes to zero, as the reference's
    # fast-math division does, where the oracle's IEEE divide keeps a denormal-range value.
    h_ref = O.swiglu_bf16(u16(g1), u16(u1))
    hd, hr = u16(h), h_ref
    tiny = 2.0 ** -100
    small = np.abs(O.bf16_to_f32(hr)) < tiny
    assert (np.abs(O.bf16_to_f32(hd))[small] < tiny).all()
    d = np.abs(hd.astype(np.int32) - hr.astype(np.int32))[~small]
    assert int(d.max(initial=0)) <= 1, int(d.max())


def test_gate_up_swiglu_norm_out_combinations(torch_dev):
    # the optional outputs of the rmsnorm pair (normalized row, gate, up) are flagged together:
    # every combination writes exactly the outputs asked for, the same bits each time
    torch = torch_dev
    K, N, eps = 2560, 10240, 1e-6
    wg = weights(torch, O.Q4_G64, N, K, 560)[0]
    wu = weights(torch, O.Q4_G64, N, K, 561)[0]
    x = dev(torch, O.gen_act(1, K, 562, outlier_frac=0.02))
    rng = np.random.default_rng(563)
    gamma = dev(torch, bf16(1.0 + 0.1 * rng.standard_normal(K)))
    ref_norm = torch.zeros((1, K), dtype=torch.int16, device="cuda")
    xq = torch.zeros((1, K), dtype=torch.int8, device="cuda")
    xs = torch.zeros((1, K // 64), dtype=torch.float32, device="cuda")
    assert va.rmsnorm_quantize(x, gamma, eps, 64, xq, xs, out=ref_norm).ok()
    z = lambda n: torch.full((1, n), 0x5555, dtype=torch.int16, device="cuda")
    h_ref = z(N)
    assert va.linear_m1_swiglu(wg, wu, P.RMSNORM, x, gamma, h_ref, eps=eps).ok()
    for want_norm in (False, True):
        for want_g in (False, True):
            for want_u in (False, True):
                h, norm, g, u = z(N), z(K), z(N), z(N)
                print(f"norm={want_norm} gate={want_g} up={want_u}", flush=True)
                assert va.linear_m1_swiglu(wg, wu, P.RMSNORM, x, gamma, h, eps=eps,
                                           norm_out=norm if want_norm else None,
                                           gate_out=g if want_g else None, up_out=u if want_u else None).ok()
                torch.cuda.synchronize()
                np.testing.assert_array_equal(u16(h), u16(h_ref))
                if want_norm:
                    np.testing.assert_array_equal(u16(norm), u16(ref_norm))
                else:
                    assert (u16(norm) == 0x5555).all()
                for want, t in ((want_g, g), (want_u, u)):
                    assert (u16(t) == 0x5555).all() != want


def test_gate_up_swiglu_errors(torch_dev):
    torch = torch_dev
    wg = weights(torch, O.Q4_G64, 64, 256, 550)[0]
    wu = weights(torch, O.Q4_G64, 32, 256, 551)[0]
    x = dev(torch, O.gen_act(1, 256, 552))
    h = torch.zeros((1, 64), dtype=torch.int16, device="cuda")
    assert va.linear_m1_swiglu(wg, wu, P.BF16, x, None, h).code == va.StatusCode.SHAPE_MISMATCH
    assert va.linear_m1_swiglu(wg, wg, P.SWIGLU, x, x, h).code == va.StatusCode.INVALID_ARGUMENT
    assert va.linear_m1_swiglu(wg, wg, P.RMSNORM, x, None, h).code == va.StatusCode.INVALID_ARGUMENT
    assert va.linear_m1_swiglu(wg, wg, P.BF16, x, None, None).code == va.StatusCode.INVALID_ARGUMENT


@pytest.mark.parametrize("K", [4096, 3072, 10752])
@pytest.mark.parametrize("qtype", [O.Q4_G64, O.Q5_G64, O.Q6_G64, O.W8_G32])
def test_rmsnorm_prologue_against_oracle(torch_dev, qtype, K):
    torch = torch_dev
    eps = 1e-5
    trip = [weights(torch, qtype, n, K, 530 + n, O.SCALE_BF16) for n in (300, 64)]
    ws = [t[0] for t in trip]
    x = O.gen_act(1, K, 531, outlier_frac=0.05)
    rng = np.random.default_rng(532)
    gamma = bf16(1.0 + 0.1 * rng.standard_normal(K))
    ys = [torch.zeros((1, w.rows), dtype=torch.int16, device="cuda") for w in ws]
    norm = torch.zeros((1, K), dtype=torch.int16, device="cuda")
    assert va.linear_m1(ws, P.RMSNORM, dev(torch, x), dev(torch, gamma), ys, eps=eps, norm_out=norm).ok()
    torch.cuda.synchronize()
    nv = u16(norm)
    ref = O.rmsnorm_bf16(x, gamma, eps)
    assert (np.abs(O.bf16_to_f32(nv).astype(np.float64) - O.bf16_to_f32(ref)) <= O.bf16_ulp(ref)).all()
    xq, xs = O.quantize_act(nv, O.group_size(qtype))
    for (w, p, s), y in zip(trip, ys):
        y_ref, _, absterm = O.qlinear_prequant(qtype, p, s, O.SCALE_BF16, w.rows, K, xq, xs)
        O.assert_bf16_close(u16(y), y_ref, absterm, rel=1e-5)


@pytest.mark.parametrize("prologue", [P.BF16, P.INT8])
def test_three_matrices_equal_single_calls(torch_dev, prologue):
    torch = torch_dev
    K = 2560
    ws = [weights(torch, O.Q6_G64, n, K, 540 + n)[0] for n in (1000, 77, 256)]
    x = O.gen_act(1, K, 541)
    xq, xs = O.quantize_act(x, 64)
    a, b = (dev(torch, x), None) if prologue == P.BF16 else (dev(torch, xq), dev(torch, xs))
    ys = [torch.zeros((1, w.rows), dtype=torch.int16, device="cuda") for w in ws]
    res = dev(torch, O.gen_act(1, 1000, 542))
    assert va.linear_m1(ws, prologue, a, b, ys, residual=res).ok()
    refs = [torch.zeros_like(y) for y in ys]
    for i, (w, r) in enumerate(zip(ws, refs)):
        rr = res if i == 0 else None
        if prologue == P.BF16:
            assert va.linear(w, a, r, residual=rr).ok()
        else:
            assert va.linear_prequantized(w, a, b, r, residual=rr).ok()
    torch.cuda.synchronize()
    for y, r in zip(ys, refs):
        np.testing.assert_array_equal(u16(y), u16(r))


def test_m1_errors_are_codes(torch_dev):
    torch = torch_dev
    w = weights(torch, O.Q4_G64, 64, 24576, 550)[0]
    x = torch.zeros((1, 24576), dtype=torch.int16, device="cuda")
    y = torch.zeros((1, 64), dtype=torch.int16, device="cuda")
    # the folded prologues hold at most 20480 elements
    assert va.linear_m1([w], P.SWIGLU, x, x, [y]).code == va.StatusCode.INVALID_ARGUMENT
    assert va.linear_m1([w], P.BF16, x, None, [y]).ok()
    assert va.linear_m1([w] * 4, P.BF16, x, None, [y] * 4).code == va.StatusCode.INVALID_ARGUMENT
    assert va.linear_m1([w], P.BF16, x, None, [y], norm_out=x).code == va.StatusCode.INVALID_ARGUMENT
    # n0's high bits carry launch flags: 2^30 rows or more are refused before any launch
    # (the same small buffers: nothing is read)
    big = va.QuantizedWeight(w.qtype, w.data, w.scales, 1 << 30, w.cols, w.group_size, w.scale_enc)
    assert va.linear_m1([big], P.BF16, x, None, [y]).code == va.StatusCode.INVALID_ARGUMENT
    assert va.linear_m1_swiglu(big, big, P.BF16, x, None, y).code == va.StatusCode.INVALID_ARGUMENT
    torch.cuda.synchronize()
