"""The verify step's one-launch linears: producers writing the int8 rows in
the matrix-core fragment order and the GEMM reading them.

The fragment order is restated here from its description in
include/viper_qlinear.h (to_frag below), so a producer that wrote bytes to the
wrong lane, k-slot or octet half fails against the natural-layout producer.
Bar: fragment bytes and scales bit-exact against the natural-layout producer
(itself pinned against the oracle in test_gpu_producers.py); GEMM outputs
within 1 bf16 ulp or 1e-5 * sum |group terms| of the oracle, and equal bit for
bit to the natural-layout prequantized entry where that runs the same
matrix-core kernel (more than 4 rows).  With a workspace, long K splits over
workgroups: then the output equals the bf16 entry's (which quantizes the same
rows on the device and runs the same split kernel) bit for bit, and the K
split's block counters are whole epochs (multiples of 64) after every call.
"""
import numpy as np
import pytest

import oracle as O
import viper_amd as va

pytestmark = pytest.mark.gpu
REL_TOL = 1e-5


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


def to_frag(xq, xs, G):
    """Natural layout (xq [M][K] int8, xs [M][K/G] fp32) -> fragment order, 16 rows, as the header
    states it; entries of rows M..15 are left at -1 (int8) / NaN (fp32) to mark "never written"."""
    M, K = xq.shape
    frag = np.full(K * 16, -1, dtype=np.int8)
    sf = np.full((K // G) * 16, np.nan, dtype=np.float32)
    for m in range(M):
        for g in range(K // G):
            sf[g * 16 + m] = xs[m, g]
            if G == 64:
                for kb in range(4):
                    qi = ((kb & 1) << 1) | (kb >> 1)
                    v = xq[m, g * 64 + 16 * qi: g * 64 + 16 * qi + 16]
                    word = np.concatenate([v[0:8:2], v[1:8:2], v[8:16:2], v[9:16:2]])
                    L = 16 * kb + m
                    frag[(g * 64 + L) * 16:(g * 64 + L) * 16 + 16] = word
            else:
                for kb in range(4):
                    qi = ((kb & 1) << 1) | (kb >> 1)
                    v = xq[m, g * 32 + 8 * qi: g * 32 + 8 * qi + 8]
                    off = ((g * 4 + kb) * 16 + m) * 8
                    frag[off:off + 8] = v
    return frag, sf


def _frag_buffers(torch, K, G):
    nq, ns = va.frag_bytes(K, G)
    xf = torch.full((nq,), -1, dtype=torch.int8, device="cuda")
    sf = torch.full((ns // 4,), float("nan"), dtype=torch.float32, device="cuda")
    return xf, sf


def _check_frag(xf, sf, want_q, want_s):
    got_q = xf.cpu().numpy()
    got_s = sf.cpu().numpy()
    np.testing.assert_array_equal(got_q, want_q)
    wrote = ~np.isnan(want_s)
    np.testing.assert_array_equal(got_s[wrote].view(np.uint32), want_s[wrote].view(np.uint32))
    assert np.isnan(got_s[~wrote]).all()          # rows M..15: never written


def bf16(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


@pytest.mark.parametrize("G", [64, 32])
@pytest.mark.parametrize("M,H", [(2, 2560), (5, 3072), (16, 2560), (9, 10240)])
def test_rmsnorm_quantize_frag_equals_natural(torch_dev, M, H, G):
    torch = torch_dev
    print(f"rmsnorm frag M={M} H={H} G={G}", flush=True)
    x = dev(torch, O.gen_act(M, H, 700 + M, outlier_frac=0.05))
    rng = np.random.default_rng(701)
    gamma = dev(torch, bf16(1.0 + 0.1 * rng.standard_normal(H)))
    xq = torch.zeros((M, H), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, H // G), dtype=torch.float32, device="cuda")
    out = torch.zeros((M, H), dtype=torch.int16, device="cuda")
    assert va.rmsnorm_quantize(x, gamma, 1e-6, G, xq, xs, out=out).ok()
    xf, sf = _frag_buffers(torch, H, G)
    out2 = torch.zeros_like(out)
    assert va.rmsnorm_quantize_frag(x, gamma, 1e-6, G, xf, sf, out=out2).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(out2), u16(out))
    want_q, want_s = to_frag(xq.cpu().numpy(), xs.cpu().numpy(), G)
    _check_frag(xf, sf, want_q, want_s)


@pytest.mark.parametrize("G", [64, 32])
@pytest.mark.parametrize("M,I", [(3, 10240), (16, 2560), (8, 10752)])
def test_swiglu_quantize_frag_equals_natural(torch_dev, M, I, G):
    torch = torch_dev
    print(f"swiglu frag M={M} I={I} G={G}", flush=True)
    rng = np.random.default_rng(710 + M)
    g = dev(torch, bf16(3.0 * rng.standard_normal((M, I))))
    u = dev(torch, bf16(rng.standard_normal((M, I))))
    xq = torch.zeros((M, I), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, I // G), dtype=torch.float32, device="cuda")
    h = torch.zeros((M, I), dtype=torch.int16, device="cuda")
    assert va.swiglu_quantize(g, u, G, xq, xs, out=h).ok()
    xf, sf = _frag_buffers(torch, I, G)
    h2 = torch.zeros_like(h)
    assert va.swiglu_quantize_frag(g, u, G, xf, sf, out=h2).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(h2), u16(h))
    want_q, want_s = to_frag(xq.cpu().numpy(), xs.cpu().numpy(), G)
    _check_frag(xf, sf, want_q, want_s)


# The GEMM from fragments: every format, single-segment and long-K shapes
# (segment loop without a workspace, K split with one), the north-star
# verify at full size, the reference engine's q and down shapes, residual,
# ragged N.
@pytest.mark.parametrize("qtype,N,K,M", [
    (O.Q4_G64, 10240, 2560, 16),
    (O.Q4_G64, 2560, 10240, 8),
    (O.Q4_G64, 6144, 3072, 16),
    (O.Q4_G64, 3072, 10752, 5),
    (O.Q5_G64, 1000, 2560, 7),
    (O.Q6_G64, 777, 4096, 12),
    (O.W8_G32, 1001, 2560, 16),
    (O.W8_G32, 513, 6144, 3),
])
def test_prequantized_frag_against_oracle(torch_dev, qtype, N, K, M):
    torch = torch_dev
    print(f"frag gemm qtype={qtype} N={N} K={K} M={M}", flush=True)
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, 720 + N, O.SCALE_FP16)
    x = O.gen_act(M, K, 721, outlier_frac=0.05)
    xq, xs = O.quantize_act(x, G)
    res = O.gen_act(M, N, 722) if M % 2 == 1 else None
    y_ref, _, absterm = O.qlinear_prequant(qtype, packed, scales, O.SCALE_FP16, N, K, xq, xs, residual=res)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc.FP16)
    fq, fs = to_frag(np.asarray(xq, dtype=np.int8).reshape(M, K), np.asarray(xs, dtype=np.float32).reshape(M, K // G), G)
    xf, sf = dev(torch, fq), dev(torch, fs)
    rd = None if res is None else dev(torch, res)
    y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear_prequantized_frag(w, xf, sf, y, residual=rd).ok()
    y_nat = torch.zeros_like(y)
    assert va.linear_prequantized(w, dev(torch, np.asarray(xq, dtype=np.int8)), dev(torch, np.asarray(xs, dtype=np.float32)),
                                  y_nat, residual=rd).ok()
    nws = va.frag_workspace_bytes(qtype, N, K, M)
    ys = torch.zeros_like(y)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")
    assert va.linear_prequantized_frag(w, xf, sf, ys, residual=rd, workspace=ws).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(u16(y), y_ref, absterm, rel=REL_TOL)
    O.assert_bf16_close(u16(y_nat), y_ref, absterm, rel=REL_TOL)
    O.assert_bf16_close(u16(ys), y_ref, absterm, rel=REL_TOL)
    if M > 4:   # the natural entry runs the same matrix-core kernel there (2-4 rows: the dot kernel, whose
        np.testing.assert_array_equal(u16(y), u16(y_nat))   # fp32 sums are added in another order)
    if nws == 0:  # no split for this shape: the workspace is not used
        np.testing.assert_array_equal(u16(ys), u16(y))
    else:
        assert split_state_ok(ws)


# Seeded random shapes on the fragment entry: every format, K of 1..72 quads
# of 4 groups (one segment, the segment loop without a workspace, the K split
# of 2..8 parts with one), ragged N, 2..16 rows, both scale encodings,
# residual on odd M.  Each output against the oracle, with and without a
# workspace; above 4 rows equal bit for bit to the natural-layout entry,
# which runs the same kernel.
def _frag_random_shapes(n=12, seed=0xF7A6):
    rng = np.random.default_rng(seed)
    out = []
    formats = [O.Q4_G64, O.Q5_G64, O.Q6_G64, O.W8_G32]
    for i in range(n):
        qtype = formats[i % 4]
        G = O.group_size(qtype)
        nq = int(rng.choice([1, 2, 3, 5, 8, 10, 12, 16, 20, 24, 30, 35, 40, 48, 60, 72]))
        K = nq * 4 * G
        N = int(rng.integers(1, 2200))
        M = int(rng.integers(2, 17))
        out.append((qtype, N, K, M, int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("qtype,N,K,M,senc", _frag_random_shapes())
def test_prequantized_frag_random_shapes(torch_dev, qtype, N, K, M, senc):
    torch = torch_dev
    print(f"frag random qtype={qtype} N={N} K={K} M={M} senc={senc}", flush=True)
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, 7300 + N, senc)
    x = O.gen_act(M, K, 7301 + M, outlier_frac=0.05)
    xq, xs = O.quantize_act(x, G)
    res = O.gen_act(M, N, 7302) if M % 2 == 1 else None
    y_ref, _, absterm = O.qlinear_prequant(qtype, packed, scales, senc, N, K, xq, xs, residual=res)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc(senc))
    fq, fs = to_frag(np.asarray(xq, dtype=np.int8).reshape(M, K), np.asarray(xs, dtype=np.float32).reshape(M, K // G), G)
    xf, sf = dev(torch, fq), dev(torch, fs)
    rd = None if res is None else dev(torch, res)
    nws = va.frag_workspace_bytes(qtype, N, K, M)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")
    y, ys, y_nat = (torch.zeros((M, N), dtype=torch.int16, device="cuda") for _ in range(3))
    assert va.linear_prequantized_frag(w, xf, sf, y, residual=rd).ok()
    assert va.linear_prequantized_frag(w, xf, sf, ys, residual=rd, workspace=ws).ok()
    assert va.linear_prequantized(w, dev(torch, np.asarray(xq, dtype=np.int8)), dev(torch, np.asarray(xs, dtype=np.float32)),
                                  y_nat, residual=rd).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(u16(y), y_ref, absterm, rel=REL_TOL)
    O.assert_bf16_close(u16(ys), y_ref, absterm, rel=REL_TOL)
    if M > 4:
        np.testing.assert_array_equal(u16(y), u16(y_nat))
    if nws == 0:
        np.testing.assert_array_equal(u16(ys), u16(y))
    else:
        assert split_state_ok(ws)


def split_state_ok(ws):
    """After a call: every K-split block counter is a whole epoch (64 * calls) and no sum missed."""
    w = ws[:4352].cpu().numpy().view(np.uint32)
    return int(w[1]) == 0 and bool((w[64:64 + 1024] % 64 == 0).all())


# The K split of the fragment entry keeps its own counters: one zeroed
# workspace serves frag calls of different shapes and part counts (K = 10240:
# 4 parts of 10 quads, K = 6144: 3 of 8, K = 8960: 5 of 7, W8 K = 6144: 6 of
# 8; K = 10752, K = 11264 and Q5 at N = 2560 loop over K instead, their split
# kernels leaving no room for two workgroups per CU), growing and shrinking
# in rows and row blocks, interleaved with the bf16 entry (its own quantize
# launch and split) on the same bytes.  Every output against the
# oracle; the frag output equal to the bf16 entry's bit for bit (same rows,
# same kernel); counters whole epochs after every call; no sum missed.
def test_frag_split_shapes_share_one_workspace(torch_dev):
    torch = torch_dev
    shapes = [(O.Q4_G64, 2560, 10240, 16), (O.Q4_G64, 3072, 10752, 5), (O.Q4_G64, 640, 10240, 16),
              (O.Q4_G64, 2560, 10240, 6), (O.W8_G32, 1000, 6144, 9), (O.Q4_G64, 3072, 6144, 16),
              (O.Q4_G64, 1000, 8960, 7), (O.Q4_G64, 700, 11264, 16), (O.Q5_G64, 2560, 10240, 8),
              (O.Q4_G64, 2560, 10240, 16), (O.Q4_G64, 3072, 10752, 12)]
    nws = max(max(va.workspace_bytes(*sh), va.frag_workspace_bytes(*sh)) for sh in shapes)
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    for i, (qtype, N, K, M) in enumerate(shapes * 2):
        print(f"shared workspace call {i}: qtype={qtype} N={N} K={K} M={M}", flush=True)
        G = O.group_size(qtype)
        seed = 760 + 13 * (i % len(shapes))
        packed, scales = O.gen_weights(qtype, N, K, seed, O.SCALE_FP16)
        x = O.gen_act(M, K, seed + 1)
        res = O.gen_act(M, N, seed + 2) if i % 3 == 1 else None
        y_ref, _, absterm = O.qlinear(qtype, packed, scales, O.SCALE_FP16, N, K, x, residual=res)
        w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc.FP16)
        xq, xs = O.quantize_act(x, G)
        fq, fs = to_frag(np.asarray(xq, dtype=np.int8).reshape(M, K), np.asarray(xs, dtype=np.float32).reshape(M, K // G), G)
        rd = None if res is None else dev(torch, res)
        yf = torch.zeros((M, N), dtype=torch.int16, device="cuda")
        yb = torch.full((M, N), 7, dtype=torch.int16, device="cuda")
        assert va.linear_prequantized_frag(w, dev(torch, fq), dev(torch, fs), yf, residual=rd, workspace=ws).ok()
        torch.cuda.synchronize()
        assert split_state_ok(ws)
        assert va.linear(w, dev(torch, x), yb, residual=rd, workspace=ws).ok()
        torch.cuda.synchronize()
        assert split_state_ok(ws)
        O.assert_bf16_close(u16(yf), y_ref, absterm, rel=REL_TOL)
        np.testing.assert_array_equal(u16(yb), u16(yf))


def test_fused2_frag_equals_two_calls(torch_dev):
    torch = torch_dev
    qtype, N, K, M = O.Q4_G64, 1024, 3072, 16
    ws = []
    for i in range(2):
        p, s = O.gen_weights(qtype, N, K, 730 + i, O.SCALE_BF16)
        ws.append(va.QuantizedWeight(va.QType(qtype), dev(torch, p), dev(torch, s), N, K, 64, va.ScaleEnc.BF16))
    x = dev(torch, O.gen_act(M, K, 732))
    rng = np.random.default_rng(733)
    gamma = dev(torch, bf16(1.0 + 0.1 * rng.standard_normal(K)))
    xf, sf = _frag_buffers(torch, K, 64)
    assert va.rmsnorm_quantize_frag(x, gamma, 1e-6, 64, xf, sf).ok()
    z = lambda: torch.zeros((M, N), dtype=torch.int16, device="cuda")
    y0, y1, r0, r1 = z(), z(), z(), z()
    assert va.linear_fused2_prequantized_frag(ws[0], ws[1], xf, sf, y0, y1).ok()
    assert va.linear_prequantized_frag(ws[0], xf, sf, r0).ok()
    assert va.linear_prequantized_frag(ws[1], xf, sf, r1).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(y0), u16(r0))
    np.testing.assert_array_equal(u16(y1), u16(r1))


def test_frag_entry_errors(torch_dev):
    torch = torch_dev
    L = va.lib()
    p, s = O.gen_weights(O.Q4_G64, 64, 512, 740, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, p), dev(torch, s), 64, 512, 64, va.ScaleEnc.FP16)
    xf, sf = _frag_buffers(torch, 512, 64)
    y1 = torch.zeros((1, 64), dtype=torch.int16, device="cuda")
    assert va.linear_prequantized_frag(w, xf, sf, y1).code == va.StatusCode.INVALID_ARGUMENT     # M = 1
    y = torch.zeros((4, 64), dtype=torch.int16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.viper_hip_qlinear_prequantized_frag(4, w.data.data_ptr(), w.scales.data_ptr(), 0, 64, 64, 512,
                                                 xf.data_ptr() + 8, sf.data_ptr(), 4, y.data_ptr(), None, None, 0,
                                                 st) == 2
    # a long-K shape with a workspace that is too small or misaligned
    p3, s3 = O.gen_weights(O.Q4_G64, 64, 10240, 743, O.SCALE_FP16)
    xf3, sf3 = _frag_buffers(torch, 10240, 64)
    need = va.frag_workspace_bytes(O.Q4_G64, 64, 10240, 4)
    assert need > 0
    ws3 = torch.zeros(need + 16, dtype=torch.uint8, device="cuda")
    args3 = (4, dev(torch, p3).data_ptr(), dev(torch, s3).data_ptr(), 0, 64, 64, 10240, xf3.data_ptr(),
             sf3.data_ptr(), 4, y.data_ptr(), None)
    assert L.viper_hip_qlinear_prequantized_frag(*args3, ws3.data_ptr(), need - 1, st) == 2
    assert L.viper_hip_qlinear_prequantized_frag(*args3, ws3.data_ptr() + 8, need, st) == 2
    p2, s2 = O.gen_weights(O.Q4_G64, 64, 128, 741, O.SCALE_FP16)   # K = 2 groups: not a multiple of 4
    w2 = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, p2), dev(torch, s2), 64, 128, 64, va.ScaleEnc.FP16)
    assert va.linear_prequantized_frag(w2, xf, sf, y).code == va.StatusCode.INVALID_ARGUMENT
    x = dev(torch, O.gen_act(17, 512, 742))
    g = dev(torch, bf16(np.ones(512)))
    assert va.rmsnorm_quantize_frag(x, g, 1e-6, 64, xf, sf).code == va.StatusCode.INVALID_ARGUMENT  # M = 17


@pytest.mark.parametrize("M,K,N", [(16, 2560, 4000), (5, 2560, 4000), (16, 10240, 2560), (7, 6144, 3000)])
def test_frag_timeline_matches_gemm(torch_dev, M, K, N):
    # the measurement entry point runs the production matrix-core GEMM with
    # stamps (long K: the K split, with a workspace): y equal to
    # viper_hip_qlinear_prequantized_frag's bit for bit, 10 non-decreasing
    # readings per wave; long K without a workspace, other formats and short
    # stamp buffers rejected
    import ctypes as C
    torch = torch_dev
    L = va.lib()
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 750 + M, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, 64, va.ScaleEnc.FP16)
    x = dev(torch, O.gen_act(M, K, 751))
    xf, sf = _frag_buffers(torch, K, 64)
    assert va.rmsnorm_quantize_frag(x, dev(torch, bf16(np.ones(K))), 1e-6, 64, xf, sf).ok()
    nws = va.frag_workspace_bytes(O.Q4_G64, N, K, M)
    assert (nws > 0) == (K > 5120)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")
    wsp = ws.data_ptr() if nws else None
    y0 = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    y1 = torch.full((M, N), 7, dtype=torch.int16, device="cuda")
    assert va.linear_prequantized_frag(w, xf, sf, y0, workspace=ws if nws else None).ok()
    stamps = torch.zeros(1 << 19, dtype=torch.int64, device="cuda")
    grid, waves = C.c_int(0), C.c_int(0)
    st = torch.cuda.current_stream().cuda_stream
    args = (w.data.data_ptr(), w.scales.data_ptr(), 0, 64, N, K, xf.data_ptr(), sf.data_ptr(), M, y1.data_ptr())
    assert L.viper_hip_qlinear_frag_timeline(4, *args, stamps.data_ptr(), stamps.numel() * 8, C.byref(grid),
                                             C.byref(waves), wsp, nws, st) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(y1), u16(y0))
    nw = grid.value * waves.value
    assert nw > 0
    t = stamps[: nw * 10].view(nw, 10).cpu().numpy()
    assert (np.diff(t, axis=1) >= 0).all() and (t[:, 0] > 0).all()
    if nws:   # one last part per row block stored y after counting
        last = (t[:, 9] > t[:, 8]).reshape(grid.value, waves.value).any(axis=1)
        assert 0 < last.sum() <= grid.value
        assert split_state_ok(ws)
    else:
        assert (t[:, 9] == t[:, 7]).all() and (t[:, 8] == t[:, 7]).all()
    assert L.viper_hip_qlinear_frag_timeline(4, *args, stamps.data_ptr(), 64, None, None, wsp, nws, st) == 2
    assert L.viper_hip_qlinear_frag_timeline(5, *args, stamps.data_ptr(), stamps.numel() * 8, None, None, wsp, nws,
                                             st) == 2
    if nws:   # the split needs its workspace, and a big enough one
        assert L.viper_hip_qlinear_frag_timeline(4, *args, stamps.data_ptr(), stamps.numel() * 8, None, None, None, 0,
                                                 st) == 2
        assert L.viper_hip_qlinear_frag_timeline(4, *args, stamps.data_ptr(), stamps.numel() * 8, None, None, wsp,
                                                 nws - 16, st) == 2
