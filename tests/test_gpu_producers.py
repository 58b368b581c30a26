"""GPU parity of the producer-side quantize kernels (rmsnorm / swiglu + int8
quantize) against the CPU oracle, through the C ABI.

Bar: the bf16 producer output within 1 bf16 ulp of the oracle's (the
reference uses rsqrtf / __expf and an fp32 reduction order of its own, so
exact equality is not defined), and the int8 activations and fp32 group
scales bit-exact against the oracle's quantizer applied to the device's own
bf16 output, which pins the quantize step exactly.
"""
import numpy as np
import pytest

import oracle as O
import viper_amd as va

pytestmark = pytest.mark.gpu


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


def host_u16(t):
    return t.cpu().numpy().view(np.uint16)


def check_producer_output(out_gpu, out_ref, xq_gpu, xs_gpu, group):
    diff = np.abs(O.bf16_to_f32(out_gpu).astype(np.float64) - O.bf16_to_f32(out_ref))
    assert (diff <= np.maximum(O.bf16_ulp(out_ref), O.bf16_ulp(out_gpu))).all()
    assert (out_gpu == out_ref).mean() > 0.99
    xq_ref, xs_ref = O.quantize_act(out_gpu, group)
    np.testing.assert_array_equal(xq_gpu, xq_ref)
    np.testing.assert_array_equal(xs_gpu.view(np.uint32), xs_ref.view(np.uint32))


@pytest.mark.parametrize("M,H", [(1, 2560), (3, 4096), (2, 10240), (1, 64)])
@pytest.mark.parametrize("group", [64, 32])
def test_rmsnorm_quantize(torch_dev, M, H, group):
    torch = torch_dev
    print(f"rmsnorm_quantize M={M} H={H} group={group}", flush=True)
    x = O.gen_act(M, H, 700 + H + M, outlier_frac=0.02, outlier_mul=20.0)
    rng = np.random.default_rng(H)
    gamma = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    eps = 1e-6
    out_ref = O.rmsnorm_bf16(x, gamma, eps)
    out = torch.zeros((M, H), dtype=torch.int16, device="cuda")
    xq = torch.zeros((M, H), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, H // group), dtype=torch.float32, device="cuda")
    xd, gd = dev(torch, x), dev(torch, gamma)
    assert va.rmsnorm_quantize(xd, gd, eps, group, xq, xs, out=out).ok()
    xq2 = torch.zeros_like(xq)
    xs2 = torch.zeros_like(xs)
    assert va.rmsnorm_quantize(xd, gd, eps, group, xq2, xs2).ok()   # no bf16 output
    torch.cuda.synchronize()
    check_producer_output(host_u16(out), out_ref, xq.cpu().numpy(), xs.cpu().numpy(), group)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq2.cpu().numpy())
    np.testing.assert_array_equal(xs.cpu().numpy(), xs2.cpu().numpy())


@pytest.mark.parametrize("M,I", [(1, 10240), (2, 2560), (3, 192)])
@pytest.mark.parametrize("group", [64, 32])
@pytest.mark.parametrize("in_place", [False, True])
def test_swiglu_quantize(torch_dev, M, I, group, in_place):
    torch = torch_dev
    print(f"swiglu_quantize M={M} I={I} group={group} in_place={in_place}", flush=True)
    rng = np.random.default_rng(I + M)
    gate = O.f32_to_bf16((3.0 * rng.standard_normal((M, I))).astype(np.float32))
    up = O.f32_to_bf16(rng.standard_normal((M, I)).astype(np.float32))
    out_ref = O.swiglu_bf16(gate, up)
    gd, ud = dev(torch, gate), dev(torch, up)
    out = gd if in_place else torch.zeros((M, I), dtype=torch.int16, device="cuda")
    xq = torch.zeros((M, I), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, I // group), dtype=torch.float32, device="cuda")
    assert va.swiglu_quantize(gd, ud, group, xq, xs, out=out).ok()
    torch.cuda.synchronize()
    check_producer_output(host_u16(out), out_ref, xq.cpu().numpy(), xs.cpu().numpy(), group)


def test_producer_errors_are_codes(torch_dev):
    torch = torch_dev
    x = torch.zeros((1, 96), dtype=torch.int16, device="cuda")
    g = torch.zeros(96, dtype=torch.int16, device="cuda")
    xq = torch.zeros((1, 96), dtype=torch.int8, device="cuda")
    xs = torch.zeros(3, dtype=torch.float32, device="cuda")
    assert va.rmsnorm_quantize(x, g, 1e-6, 64, xq, xs).code == va.StatusCode.INVALID_ARGUMENT  # 96 % 64
    assert va.rmsnorm_quantize(x, g, 1e-6, 48, xq, xs).code == va.StatusCode.INVALID_ARGUMENT
    assert va.swiglu_quantize(x, x, 16, xq, xs).code == va.StatusCode.INVALID_ARGUMENT
    assert va.rmsnorm_quantize(x, g, 1e-6, 32, xq, xs).ok()
    torch.cuda.synchronize()


def test_mlp_pipeline(torch_dev):
    # config 1 at full size: gate+up (fused2, K=2560, N=2x10240) -> swiglu +
    # quantize -> down (K=10240, N=2560) + residual, each stage checked
    # against the oracle fed with the device's previous stage
    torch = torch_dev
    H, I = 2560, 10240
    G = 64
    pg, sg = O.gen_weights(O.Q4_G64, I, H, 0x5EED0001, O.SCALE_FP16)
    pu, su = O.gen_weights(O.Q4_G64, I, H, 0x5EED0011, O.SCALE_FP16)
    pd, sd = O.gen_weights(O.Q4_G64, H, I, 0x5EED0021, O.SCALE_FP16)
    x = O.gen_act(1, H, 0x5EED0031)
    res = O.gen_act(1, H, 0x5EED0041)
    wg = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, pg), dev(torch, sg), I, H, scale_enc=va.ScaleEnc.FP16)
    wu = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, pu), dev(torch, su), I, H, scale_enc=va.ScaleEnc.FP16)
    wd = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, pd), dev(torch, sd), H, I, scale_enc=va.ScaleEnc.FP16)
    g = torch.zeros((1, I), dtype=torch.int16, device="cuda")
    u = torch.zeros((1, I), dtype=torch.int16, device="cuda")
    xq = torch.zeros((1, I), dtype=torch.int8, device="cuda")
    xs = torch.zeros((1, I // G), dtype=torch.float32, device="cuda")
    y = torch.zeros((1, H), dtype=torch.int16, device="cuda")
    assert va.linear_fused2(wg, wu, dev(torch, x), g, u).ok()
    assert va.swiglu_quantize(g, u, G, xq, xs, out=g).ok()       # in place, as the engine
    assert va.linear_prequantized(wd, xq, xs, y, residual=dev(torch, res)).ok()
    torch.cuda.synchronize()
    # stage 1 (g is overwritten in place: compare u, and g through a second call)
    u_ref, _, u_abs = O.qlinear(O.Q4_G64, pu, su, O.SCALE_FP16, I, H, x)
    O.assert_bf16_close(host_u16(u), u_ref, u_abs, rel=1e-5)
    g2 = torch.zeros((1, I), dtype=torch.int16, device="cuda")
    assert va.linear(wg, dev(torch, x), g2).ok()
    torch.cuda.synchronize()
    g_ref, _, g_abs = O.qlinear(O.Q4_G64, pg, sg, O.SCALE_FP16, I, H, x)
    O.assert_bf16_close(host_u16(g2), g_ref, g_abs, rel=1e-5)
    # stage 2 from the device's g, u
    h_ref = O.swiglu_bf16(host_u16(g2), host_u16(u))
    check_producer_output(host_u16(g), h_ref, xq.cpu().numpy(), xs.cpu().numpy(), G)
    # stage 3 from the device's xq, xs
    y_ref, _, y_abs = O.qlinear_prequant(O.Q4_G64, pd, sd, O.SCALE_FP16, H, I, xq.cpu().numpy(),
                                         xs.cpu().numpy(), residual=res)
    O.assert_bf16_close(host_u16(y), y_ref, y_abs, rel=1e-5)
