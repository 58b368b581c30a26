"""GPU parity of the gfx950 kernels against the CPU oracle, through the C ABI.

Bar: per-group int32 dots D[m,n,g] bit-exact; int8 activations and fp32 group
scales bit-exact; bf16 outputs within 1 bf16 ulp of the oracle's bf16 output
or within 1e-5 * sum|group terms| (the condition-aware bound).  Sizes run from
one group up to the north-star shape (K=2560, N=10240), which the oracle
finishes in well under a second.
"""
import sys

import numpy as np
import pytest

import oracle as O
import viper_amd as va

pytestmark = pytest.mark.gpu

FORMATS = [O.Q4_G64, O.Q5_G64, O.Q6_G64, O.W8_G32]
REL_TOL = 1e-5  # relative to sum |group terms|, plus the 1-bf16-ulp clause


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


def host(t, dtype):
    a = t.cpu().numpy()
    return a.view(dtype) if a.dtype.itemsize == np.dtype(dtype).itemsize else a.astype(dtype)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_case(torch, qtype, N, K, M, seed, scale_enc=O.SCALE_FP16, residual=False, outlier=0.0,
             check_partials=True):
    note(f"case qtype={qtype} N={N} K={K} M={M} seed={seed} senc={scale_enc} res={residual}")
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, seed, scale_enc)
    x = O.gen_act(M, K, seed + 1, outlier_frac=outlier, outlier_mul=20.0)
    res = O.gen_act(M, N, seed + 2) if residual else None
    y_ref, _, absterm = O.qlinear(qtype, packed, scales, scale_enc, N, K, x, residual=res)
    xq, _ = O.quantize_act(x, G)
    D_ref = O.group_dots(qtype, packed, N, K, xq)

    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G,
                           va.ScaleEnc(scale_enc))
    xd = dev(torch, x)
    yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    pd = torch.full((M, N, K // G), -7, dtype=torch.int32, device="cuda")
    rd = None if res is None else dev(torch, res)
    nws = va.workspace_bytes(qtype, N, K, M)
    wsd = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda") if nws else None
    if check_partials:
        st = va.linear_partials(w, xd, yd, pd, residual=rd, workspace=wsd)
    else:
        st = va.linear(w, xd, yd, residual=rd, workspace=wsd)
    assert st.ok(), st
    torch.cuda.synchronize()
    if check_partials:
        np.testing.assert_array_equal(host(pd, np.int32), D_ref)
    O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)
    return host(yd, np.uint16)


def test_device_bf16_rounding_exhaustive(torch_dev):
    # the kernels' fp32 -> bf16 conversion (hardware) equals round-to-nearest-
    # even with quiet NaNs (the oracle's f32_to_bf16) on all 2^32 inputs
    torch = torch_dev
    cnt = torch.zeros(1, dtype=torch.int64, device="cuda")
    assert va.lib().viper_hip_check_bf16_rounding(cnt.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert int(cnt[0]) == 0


def test_device_quantizer_exhaustive(torch_dev):
    torch = torch_dev
    counts = torch.full((255 * 128,), -1, dtype=torch.int32, device="cuda")
    st = va.check_quantizer(0, 254, counts)
    assert st.ok(), st
    torch.cuda.synchronize()
    c = counts.cpu().numpy()
    assert (c == 0).all(), np.nonzero(c)[0][:10]


@pytest.mark.parametrize("group", [64, 32])
def test_quantize_act_bitexact(torch_dev, group):
    torch = torch_dev
    M, K = 5, 2560
    x = O.gen_act(M, K, 11, outlier_frac=0.05, outlier_mul=20.0)
    xf = O.bf16_to_f32(x).copy()
    xf[0, :group] = 0.0                         # zero group -> scale 1e-8
    xf[1, :group] = 0.0                         # amax 127 -> scale 1, exact ties
    xf[1, :6] = [127.0, 2.5, 3.5, -2.5, 0.5, -1.5]
    xf[2, group:2 * group] = np.linspace(-1e-6, 1e-6, group)
    x = O.f32_to_bf16(xf)
    xq_ref, xs_ref = O.quantize_act(x, group)
    xq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, K // group), dtype=torch.float32, device="cuda")
    st = va.quantize_act(dev(torch, x), group, xq, xs)
    assert st.ok(), st
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(xs.cpu().numpy().view(np.uint32), xs_ref.view(np.uint32))
    assert list(xq_ref[1, :6]) == [127, 2, 4, -2, 0, -2]


@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("scale_enc", [O.SCALE_FP16, O.SCALE_BF16])
@pytest.mark.parametrize("N,K", [(1, 64), (37, 128), (100, 640), (256, 2560), (19, 10240)])
def test_m1_fused(torch_dev, qtype, scale_enc, N, K):
    run_case(torch_dev, qtype, N, K, 1, seed=1000 + N + K, scale_enc=scale_enc)


@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 9, 10, 16])
def test_multi_row(torch_dev, qtype, M):
    # (Q4 9 and 10 rows at K = 2560: the one-launch bf16-row path, staged in pairs)
    K = 2048 if M <= 8 else 2560
    run_case(torch_dev, qtype, 77, K, M, seed=2000 + M, residual=(M % 2 == 0))


# M = 2..4 at long K from bf16 x: 2 rows (and 3 rows, M * K <= 32768) staged
# by every workgroup of the M = 1 kernel, 4 rows at K = 10240 and rows past
# the staging bound on the matrix cores after the quantize launch.  (The
# prequantized entry takes 4 rows at K = 10240 through all eight staging
# rounds of a 640-thread workgroup: test_prequantized_entry.)
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("M,K", [(2, 10240), (3, 10240), (4, 10240), (3, 12288), (4, 16384)])
def test_multi_row_long_k(torch_dev, qtype, M, K):
    run_case(torch_dev, qtype, 45, K, M, seed=2100 + M + K, residual=(M == 4))


# M = 2..16 run on the i8 matrix cores when K is a multiple of two groups:
# one load segment per wave (K <= 40 groups per 4 waves), the double-buffered
# loop (long K), two 16-row tiles per wave (N >= 64 tiles per CU), partial
# tiles, and K with an odd group count (the v_dot4 path).
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,M,senc", [
    (16, 128, 2, O.SCALE_FP16),
    (45, 2560, 16, O.SCALE_BF16),
    (50, 10240, 16, O.SCALE_FP16),
    (33, 6144, 7, O.SCALE_BF16),
    (16400, 256, 3, O.SCALE_FP16),
    (29, 192, 4, O.SCALE_FP16),
    (300, 384, 9, O.SCALE_BF16),     # 6 groups (W8: 12): the pair-wise matrix-core kernel
    (70, 640, 12, O.SCALE_FP16),     # 10 groups (W8: 20)
    (1000, 3072, 16, O.SCALE_BF16),  # 12 quads: one per wave of 12 (W8: 24 quads, 3 parts of 8)
    (3000, 2816, 9, O.SCALE_FP16),   # 11 quads on 12 waves, the last one idle; 3000 rows: 48-row blocks
    (10752, 3072, 5, O.SCALE_FP16),  # the reference engine's gate shape on 12 waves (W8: the K split)
])
def test_mfma_shapes(torch_dev, qtype, N, K, M, senc):
    run_case(torch_dev, qtype, N, K, M, seed=3000 + N + M, scale_enc=senc, residual=(M % 2 == 1))


# Long K on the matrix cores (more than 20 quads of 4 groups) splits K in
# 2..8 parts, one workgroup each, where the split kernel leaves room for two
# workgroups per CU (else it loops over K); the last part of a row block to
# finish adds the parts' sums in part order.  The workspace starts zeroed
# (the contract) and serves a second call with another row count; a repeated
# call must give the same bits.
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,M,M2,senc", [
    (2560, 10240, 16, 4, O.SCALE_FP16),   # down shape
    (50, 10240, 7, 3, O.SCALE_BF16),      # ragged last row block
    (1000, 6144, 12, 2, O.SCALE_FP16),    # 6 quads per part; M2 = 2 on the dot path
    (333, 12288, 9, 16, O.SCALE_BF16),    # 6 parts of 8 quads (W8: 8 parts of 12, two quads per wave)
    (777, 8960, 9, 5, O.SCALE_FP16),      # 5 parts of 7 quads (W8: 70 quads, 7 parts of 10)
    (500, 11264, 16, 6, O.SCALE_BF16),    # W8: 8 parts of 11 quads, two quads per wave (Q4/Q5/Q6: the loop)
    (3072, 10752, 12, 16, O.SCALE_FP16),  # the reference engine's down shape (Q4: the loop; W8: 6 parts of 14)
])
def test_k_split(torch_dev, qtype, N, K, M, M2, senc):
    torch = torch_dev
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, 5100 + N, senc)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G,
                           va.ScaleEnc(senc))
    nws = max(va.workspace_bytes(qtype, N, K, m) for m in (M, M2))
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    for m, residual in ((M, True), (M2, False)):
        note(f"case qtype={qtype} N={N} K={K} M={m} senc={senc} res={residual}")
        x = O.gen_act(m, K, 5200 + m)
        res = O.gen_act(m, N, 5300 + m) if residual else None
        y_ref, _, absterm = O.qlinear(qtype, packed, scales, senc, N, K, x, residual=res)
        outs = []
        for _ in range(2):
            yd = torch.zeros((m, N), dtype=torch.int16, device="cuda")
            rd = None if res is None else dev(torch, res)
            assert va.linear(w, dev(torch, x), yd, residual=rd, workspace=ws).ok()
            torch.cuda.synchronize()
            outs.append(host(yd, np.uint16))
        O.assert_bf16_close(outs[0], y_ref, absterm, rel=REL_TOL)
        np.testing.assert_array_equal(outs[1], outs[0])
    assert missed_sums(ws) == 0


# Seeded random shapes on the K split: K of 24..80 quads (2..8 parts of one
# or two quads per wave), ragged N, rows past the multi-row bound, both scale
# encodings, residual on odd M.
def _k_split_shapes(n=12, seed=0x5EED5):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        qtype = FORMATS[i % len(FORMATS)]
        G = O.group_size(qtype)
        nq = int(rng.choice([24, 28, 30, 32, 35, 36, 40, 42, 45, 48, 56, 64, 72, 80]))
        K = nq * 4 * G
        M = int(rng.integers(max(4, 32768 // K + 1), 17))
        N = int(rng.integers(1, 3000))
        out.append((qtype, N, K, M, int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("qtype,N,K,M,senc", _k_split_shapes())
def test_k_split_random_shapes(torch_dev, qtype, N, K, M, senc):
    # every part writes the int32 dots of its own groups: D bit-exact
    run_case(torch_dev, qtype, N, K, M, seed=5500 + N, scale_enc=senc, residual=(M % 2 == 1))


# Seeded random shapes through the bf16 entry, every dispatch path: 1..16
# rows, K of 1..200 groups (odd group counts on the dot kernel, even ones on
# the pair-swap matrix-core kernel, multiples of 4 on the row-contiguous one,
# long K split or looped; M = 1 on exact, masked or general tilings), ragged
# N, both scale encodings, residual at random.  Group dots bit-exact through
# the partials entry; the production entry's output equal to the partials
# entry's bit for bit (the same arithmetic) and within the bar of the oracle.
def _random_shapes(n=24, seed=0x5EED7):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        qtype = FORMATS[i % len(FORMATS)]
        G = O.group_size(qtype)
        ng = int(rng.choice([1, 2, 3, 4, 7, 8, 12, 16, 20, 33, 40, 48, 64, 80, 96, 100, 120, 160, 168, 200]))
        M = 1 if rng.random() < 0.3 else int(rng.integers(2, 17))
        out.append((qtype, int(rng.integers(1, 3000)), ng * G, M, int(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("qtype,N,K,M,senc,residual", _random_shapes())
def test_random_shapes_every_path(torch_dev, qtype, N, K, M, senc, residual):
    seed = 9100 + N + K + M
    y_part = run_case(torch_dev, qtype, N, K, M, seed=seed, scale_enc=senc, residual=residual)
    y_prod = run_case(torch_dev, qtype, N, K, M, seed=seed, scale_enc=senc, residual=residual, check_partials=False)
    np.testing.assert_array_equal(y_prod, y_part)


# Two different activations at the same row count alternating on one
# workspace: each result must be the oracle's for its own x (a part that
# consumed the previous call's sums would give the other x's output).
def test_k_split_alternating_inputs(torch_dev):
    torch = torch_dev
    qtype, N, K, M = O.Q4_G64, 2560, 10240, 8
    packed, scales = O.gen_weights(qtype, N, K, 5600, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, 64,
                           va.ScaleEnc(O.SCALE_FP16))
    xs = [O.gen_act(M, K, 5601), O.gen_act(M, K, 5602)]
    refs = [O.qlinear(qtype, packed, scales, O.SCALE_FP16, N, K, x) for x in xs]
    ws = torch.zeros(va.workspace_bytes(qtype, N, K, M), dtype=torch.uint8, device="cuda")
    xds = [dev(torch, x) for x in xs]
    for i in range(6):
        note(f"alternating call {i}")
        yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
        assert va.linear(w, xds[i % 2], yd, workspace=ws).ok()
        torch.cuda.synchronize()
        y_ref, _, absterm = refs[i % 2]
        O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)
    assert missed_sums(ws) == 0


def missed_sums(ws):
    """The workspace's count of K-split sums that never arrived (offset 4)."""
    return int(ws[4:8].cpu().numpy().view(np.uint32)[0])


def _split_case(torch, qtype, N, K, M, seed, senc=O.SCALE_FP16, residual=False):
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, seed, senc)
    x = O.gen_act(M, K, seed + 1)
    res = O.gen_act(M, N, seed + 2) if residual else None
    y_ref, _, absterm = O.qlinear(qtype, packed, scales, senc, N, K, x, residual=res)
    xq, _ = O.quantize_act(x, G)
    D_ref = O.group_dots(qtype, packed, N, K, xq)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc(senc))
    return dict(shape=(qtype, N, K, M), w=w, x=dev(torch, x), res=None if res is None else dev(torch, res),
                y_ref=y_ref, absterm=absterm, D_ref=D_ref)


def _run_split_case(torch, c, ws, i):
    qtype, N, K, M = c["shape"]
    note(f"call {i}: qtype={qtype} N={N} K={K} M={M}")
    assert va.workspace_layout(qtype, N, K, M)["sums"] is not None        # this shape runs the K split
    yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    pd = torch.full((M, N, K // O.group_size(qtype)), -7, dtype=torch.int32, device="cuda")
    assert va.linear_partials(c["w"], c["x"], yd, pd, residual=c["res"], workspace=ws).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(pd, np.int32), c["D_ref"])
    O.assert_bf16_close(host(yd, np.uint16), c["y_ref"], c["absterm"], rel=REL_TOL)


# Split shapes of different sizes alternating on one zeroed workspace: each
# row block's record of slots and its counter (whose epoch tags the slots)
# sit at the same offsets for every shape, so a slot can only hold an earlier
# epoch of its own block; the two shapes' blocks cover different rows and
# different slot ranges of the same records.  Every call is checked against
# the oracle (group dots bit-exact); counters are whole epochs after every
# call and no sum may miss.
def test_k_split_shapes_alternate_on_one_workspace(torch_dev):
    torch = torch_dev
    cases = [_split_case(torch, O.Q4_G64, 2048, 10240, 5, 0x5A10),
             _split_case(torch, O.Q4_G64, 640, 10240, 16, 0x5A20, residual=True)]
    nws = max(va.workspace_bytes(*c["shape"]) for c in cases)
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    for i in range(10):
        _run_split_case(torch, cases[i % 2], ws, i)
        counters = ws[256:256 + 4096].cpu().numpy().view(np.uint32)
        assert (counters % 64 == 0).all()
    assert missed_sums(ws) == 0


# Growing sequences on one zeroed workspace (each call's slot region covers
# more of the workspace than the last): M = 5 -> 6 -> 16 at the down shape,
# then N = 1000 -> 2560, then another format and K on the same bytes.
def test_k_split_growing_sequence_one_workspace(torch_dev):
    torch = torch_dev
    shapes = [(O.Q4_G64, 2560, 10240, 5), (O.Q4_G64, 2560, 10240, 6), (O.Q4_G64, 2560, 10240, 16),
              (O.Q4_G64, 1000, 10240, 16), (O.Q4_G64, 2560, 10240, 16), (O.W8_G32, 2048, 6144, 9),
              (O.Q5_G64, 1000, 12288, 12), (O.Q4_G64, 1000, 10240, 5)]
    nws = max(va.workspace_bytes(*s) for s in shapes)
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    for i, (qtype, N, K, M) in enumerate(shapes):
        _run_split_case(torch, _split_case(torch, qtype, N, K, M, 0x5B00 + 17 * i, residual=(i % 3 == 1)), ws, i)
    assert missed_sums(ws) == 0


def test_k_split_two_streams_concurrent(torch_dev):
    # two K-split calls in flight at once on two streams (default priority),
    # each with its own workspace: every result equals its single-stream one
    # bit for bit (no exchange crosses workspaces, no spin runs out)
    torch = torch_dev
    qtype, N, K = O.Q4_G64, 2560, 10240
    cases = []
    for M, seed in ((5, 5700), (16, 5710)):
        packed, scales = O.gen_weights(qtype, N, K, seed, O.SCALE_FP16)
        w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, 64,
                               va.ScaleEnc(O.SCALE_FP16))
        x = dev(torch, O.gen_act(M, K, seed + 1))
        ws = torch.zeros(va.workspace_bytes(qtype, N, K, M), dtype=torch.uint8, device="cuda")
        y0 = torch.zeros((M, N), dtype=torch.int16, device="cuda")
        assert va.linear(w, x, y0, workspace=ws).ok()
        cases.append((w, x, ws, y0))
    outs = [[torch.zeros_like(c[3]) for _ in range(10)] for c in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for i in range(10):
        for (w, x, ws, _), s, o in zip(cases, streams, outs):
            assert va.linear(w, x, o[i], workspace=ws, stream=s).ok()
    torch.cuda.synchronize()
    for (_, _, _, y0), o in zip(cases, outs):
        ref = y0.cpu().numpy()
        for t in o:
            np.testing.assert_array_equal(t.cpu().numpy(), ref)


# BASELINE config 2 as stated: M in {2, 4, 8, 16} at both shapes, full size,
# int32 group dots bit-exact and bf16 within the bar.
@pytest.mark.parametrize("M", [2, 4, 8, 16])
@pytest.mark.parametrize("N,K", [(10240, 2560), (2560, 10240)])
def test_config2_grid_full_size(torch_dev, N, K, M):
    run_case(torch_dev, O.Q4_G64, N, K, M, seed=0x5EED0002 + M, residual=(K == 10240))


# Output rounding (A8) pinned exactly: one non-zero group whose weight scale
# (2^-4) and activation scale (amax 15.875 -> 2^-3) are powers of two, so the
# fp32 sum ws*xs*D is exact and the bf16 output must equal RNE(D * 2^-7) bit
# for bit: ties to even both ways (257 -> 256, 259 -> 260, 383 -> 384), a
# round up past a truncation (515 -> 516) and exact values.  Every other
# group holds zeros (its term is exactly 0).  Runs the M = 1 kernel, the
# multi-row and matrix-core paths and the K split.
A8_CODES = [(2, 0, 1), (2, 2, 1), (4, 7, 0), (3, 0, 0), (-2, -2, -1), (1, 1, 0), (7, 7, 7), (-8, -8, -8),
            (5, 3, 2), (0, 1, 0), (0, 0, 0), (6, -3, 7), (3, 5, -1), (-3, -5, 1), (-4, -7, 0), (7, -8, 5)]


def _rne_bf16_exact(D):
    # D * 2^-7 rounded to 8 significant bits, ties to even, from the integer
    from fractions import Fraction
    out = []
    for d in D:
        v = Fraction(int(d), 128)
        if v == 0:
            out.append(0)
            continue
        sign = 0x8000 if v < 0 else 0
        a = abs(v)
        e = a.numerator.bit_length() - a.denominator.bit_length()
        if Fraction(2) ** e > a:
            e -= 1
        q = a / Fraction(2) ** (e - 7)          # in [128, 256)
        fl = q.numerator // q.denominator
        rem = q - fl
        if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
            fl += 1
        if fl == 256:
            fl, e = 128, e + 1
        out.append(sign | ((e + 127) << 7) | (fl - 128))
    return np.array(out, dtype=np.uint16)


@pytest.mark.parametrize("senc", [O.SCALE_FP16, O.SCALE_BF16])
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("M,K", [(1, 256), (2, 256), (4, 256), (16, 256), (1, 10240), (16, 10240)])
def test_bf16_rounding_exact(torch_dev, qtype, M, K, senc):
    torch = torch_dev
    G = O.group_size(qtype)
    N = len(A8_CODES)
    w = np.zeros((N, K), dtype=np.int8)
    for n, (a, b, c) in enumerate(A8_CODES):
        w[n, :3] = (a, b, c)
    packed = O.pack(qtype, w)
    scales = np.full(N * (K // G), 0x2C00 if senc == O.SCALE_FP16 else 0x3D80, dtype=np.uint16)
    x = np.zeros((M, K), dtype=np.uint16)
    x[:, 0], x[:, 1], x[:, 2] = 0x417E, 0x3E00, 0x3EC0   # 15.875 (q = 127), 0.125 (1), 0.375 (3)
    D = w[:, 0].astype(np.int64) * 127 + w[:, 1] + 3 * w[:, 2]
    expect = np.tile(_rne_bf16_exact(D), (M, 1))
    y_ref, _, _ = O.qlinear(qtype, packed, scales, senc, N, K, x)
    np.testing.assert_array_equal(y_ref, expect)         # the oracle's rounding
    wq = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc(senc))
    nws = va.workspace_bytes(qtype, N, K, M)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda") if nws else None
    note(f"case qtype={qtype} M={M} K={K} senc={senc}")
    yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear(wq, dev(torch, x), yd, workspace=ws).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(yd, np.uint16), expect)


# The K split captured in a HIP graph (its counters are cleared by the
# quantize launch inside the graph, no memset node): every replay, with an
# eager call of another row count on the same workspace between replays,
# equals the eager result bit for bit.
def test_k_split_graph_replays(torch_dev):
    torch = torch_dev
    qtype, N, K, M, M2 = O.Q4_G64, 2560, 10240, 8, 5
    packed, scales = O.gen_weights(qtype, N, K, 5400, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, 64,
                           va.ScaleEnc(O.SCALE_FP16))
    x, x2 = O.gen_act(M, K, 5401), O.gen_act(M2, K, 5402)
    res = O.gen_act(M, N, 5403)
    xd, x2d, rd = dev(torch, x), dev(torch, x2), dev(torch, res)
    ws = torch.zeros(max(va.workspace_bytes(qtype, N, K, m) for m in (M, M2)), dtype=torch.uint8, device="cuda")
    ye = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear(w, xd, ye, residual=rd, workspace=ws).ok()
    torch.cuda.synchronize()
    y_eager = host(ye, np.uint16)
    y_ref, _, absterm = O.qlinear(qtype, packed, scales, O.SCALE_FP16, N, K, x, residual=res)
    O.assert_bf16_close(y_eager, y_ref, absterm, rel=REL_TOL)
    yg = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    y2 = torch.zeros((M2, N), dtype=torch.int16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert va.linear(w, xd, yg, residual=rd, workspace=ws).ok()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = va.linear(w, xd, yg, residual=rd, workspace=ws)
    assert st.ok()
    for i in range(3):
        note(f"replay {i}")
        yg.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(yg, np.uint16), y_eager)
        assert va.linear(w, x2d, y2, workspace=ws).ok()   # eager, same workspace
        torch.cuda.synchronize()


# The reference engine's own shapes (include/viper/model_impl.cuh:107-116:
# hidden 3072, intermediate 10752, 48 x 128 query and 8 x 128 key/value
# heads): q 3072 -> 6144, k / v 3072 -> 1024, o 6144 -> 3072 (+ residual),
# gate / up 3072 -> 10752, down 10752 -> 3072 (+ residual), full size, one
# decode row and a 16-row verify, group dots bit-exact.  At M = 1 they run the
# 6-slot exact tilings (K = 3072: 16 lanes per row, 6144: 32) and the masked
# one (K = 10752: 336 chunks in 64 x 6 slots).
@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("N,K", [(6144, 3072), (1024, 3072), (3072, 6144), (10752, 3072), (3072, 10752)])
def test_engine_shapes_full_size(torch_dev, N, K, M):
    run_case(torch_dev, O.Q4_G64, N, K, M, seed=0xE0000 + K + M, residual=(N == 3072))


# One Q4 / Q5 matrix at K = 3072 takes the 44-row workgroup where its grid
# covers the CUs (N = 10752, 11000, ragged); N = 9000 and Q6 keep the shape
# the picker takes by per-CU rows.
# Q5 from a bf16 row at K = 2560 takes one 40-row workgroup per CU where
# that carries as many rows per CU as two of 20 (N = 10240, 20480); Q4 and
# Q6 keep two of 20, and so does Q5 at N = 5000.  Group dots bit-exact, the
# output against the oracle, the production entry equal to the partials
# entry bit for bit, and the timeline entry's output and grid those of the
# production call.
@pytest.mark.parametrize("qtype,N,K", [(O.Q4_G64, 10752, 3072), (O.Q5_G64, 10752, 3072), (O.Q4_G64, 11000, 3072),
                                       (O.Q4_G64, 9000, 3072), (O.Q6_G64, 10752, 3072), (O.Q5_G64, 10240, 2560),
                                       (O.Q5_G64, 20480, 2560), (O.Q6_G64, 10240, 2560), (O.Q5_G64, 5000, 2560)])
def test_m1_workgroup_choice(torch_dev, qtype, N, K):
    import ctypes as C
    torch = torch_dev
    seed = 0xE3000 + N + qtype
    y_part = run_case(torch, qtype, N, K, 1, seed=seed, residual=False)
    y_prod = run_case(torch, qtype, N, K, 1, seed=seed, residual=False, check_partials=False)
    np.testing.assert_array_equal(y_prod, y_part)
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, seed, O.SCALE_FP16)
    x = O.gen_act(1, K, seed + 1)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc.FP16)
    yt = torch.zeros((1, N), dtype=torch.int16, device="cuda")
    stamps = torch.zeros(1 << 18, dtype=torch.int64, device="cuda")
    grid, waves = C.c_int(0), C.c_int(0)
    assert va.lib().viper_hip_qlinear_timeline(qtype, w.data.data_ptr(), w.scales.data_ptr(), 0, G, N, K,
                                               dev(torch, x).data_ptr(), yt.data_ptr(), stamps.data_ptr(),
                                               stamps.numel() * 8, C.byref(grid), C.byref(waves),
                                               torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(yt, np.uint16), y_prod)
    if K == 3072:
        if qtype != O.Q6_G64 and N != 9000:
            assert (grid.value, waves.value) == ((N + 43) // 44, 11)
        else:
            assert waves.value != 11
    else:
        wide = qtype == O.Q5_G64 and N in (10240, 20480)
        assert (grid.value, waves.value) == (((N + 39) // 40, 10) if wide else ((N + 19) // 20, 5))


# Every format at the engine's K (ragged N, both scale encodings, outliers):
# Q4 / Q5 / Q6 on the 6-slot and masked tilings, W8 on its own (K = 3072:
# 32 lanes x 6, 6144: 64 x 6; 10752 on the general path).
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,senc", [(1000, 3072, O.SCALE_FP16), (777, 6144, O.SCALE_BF16),
                                      (1001, 10752, O.SCALE_FP16), (64, 10752, O.SCALE_BF16)])
def test_engine_k_every_format(torch_dev, qtype, N, K, senc):
    run_case(torch_dev, qtype, N, K, 1, seed=0xE1000 + N + qtype, scale_enc=senc, residual=(N % 2 == 1),
             outlier=0.05)


# Q4 with K a multiple of 256 runs the row-contiguous matrix-core kernel: rows
# per workgroup 8..48 (one workgroup per CU where N allows), one or two
# 4-group quads per wave (K up to 2560, up to 5120), 4-wave workgroups for
# short K, ragged last blocks.
@pytest.mark.parametrize("N,K,M", [
    (4000, 2560, 16),
    (6001, 5120, 9),
    (8000, 4096, 4),
    (10240, 5120, 16),
    (12003, 1024, 2),
    (300, 2816, 13),
])
def test_q4_rowcontig_shapes(torch_dev, N, K, M):
    run_case(torch_dev, O.Q4_G64, N, K, M, seed=5000 + K + M, residual=(M % 2 == 0))


# Staged scales with two loads per thread (W8 with two quads per wave and 40
# or 48 rows per workgroup: the only shapes whose weight-scale block has more
# 8-byte pieces than the workgroup has threads): the unsplit M = 16 launch at
# the north-star shape and the K split with 48-row blocks, with and without
# the partials output (separate kernel variants).
@pytest.mark.parametrize("N,K,M", [(10240, 2560, 16), (6000, 10240, 9)])
@pytest.mark.parametrize("partials", [True, False])
def test_w8_staged_scales_two_loads_per_thread(torch_dev, N, K, M, partials):
    run_case(torch_dev, O.W8_G32, N, K, M, seed=7100 + M, scale_enc=O.SCALE_BF16, residual=True,
             check_partials=partials)


def test_verify_m16_full_size(torch_dev):
    # config 2: M=16 speculative verify at the north-star shape
    run_case(torch_dev, O.Q4_G64, 10240, 2560, 16, seed=0x5EED0002)


def test_verify_m16_down_full_size(torch_dev):
    # M=16 at the down-projection shape: 160 KB of int8 activations, more than
    # one workgroup's LDS, which the matrix-core path never stages
    run_case(torch_dev, O.Q4_G64, 2560, 10240, 16, seed=0x5EED0003, residual=True)


def test_mfma_deterministic(torch_dev):
    a = run_case(torch_dev, O.Q5_G64, 300, 10240, 9, seed=11)
    b = run_case(torch_dev, O.Q5_G64, 300, 10240, 9, seed=11)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("qtype", FORMATS)
def test_residual_and_outliers(torch_dev, qtype):
    run_case(torch_dev, qtype, 130, 2560, 1, seed=31, residual=True, outlier=0.05)


def test_north_star_full_size(torch_dev):
    run_case(torch_dev, O.Q4_G64, 10240, 2560, 1, seed=0x5EED0000)


def test_down_shape_full_size(torch_dev):
    run_case(torch_dev, O.Q4_G64, 2560, 10240, 1, seed=0x5EED0001, residual=True)


@pytest.mark.parametrize("qtype", FORMATS)
def test_format_sweep_full_size(torch_dev, qtype):
    # config 4: K=2560, N=10240 with 5% x20 outlier channels
    run_case(torch_dev, qtype, 10240, 2560, 1, seed=0x5EED0004, outlier=0.05)


@pytest.mark.parametrize("qtype", FORMATS)
def test_format_sweep_m8_full_size(torch_dev, qtype):
    # config 4 at M=8: 40-row workgroups of the row-contiguous matrix-core kernel
    # (W8: two 4-group quads per wave)
    run_case(torch_dev, qtype, 10240, 2560, 8, seed=0x5EED0005, outlier=0.05, residual=True)


def test_row_matches_single_row_call(torch_dev):
    # row m of an M-row call equals an M=1 call on row m, bit for bit
    torch = torch_dev
    N, K, M = 300, 2560, 4
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 5, O.SCALE_FP16)
    x = O.gen_act(M, K, 6)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, scale_enc=va.ScaleEnc.FP16)
    ws = torch.zeros(va.workspace_bytes(4, N, K, M), dtype=torch.uint8, device="cuda")
    pm = torch.zeros((M, N, K // 64), dtype=torch.int32, device="cuda")
    ym = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear_partials(w, dev(torch, x), ym, pm, workspace=ws).ok()
    for m in range(M):
        p1 = torch.zeros((1, N, K // 64), dtype=torch.int32, device="cuda")
        y1 = torch.zeros((1, N), dtype=torch.int16, device="cuda")
        assert va.linear_partials(w, dev(torch, x[m:m + 1]), y1, p1).ok()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(p1.cpu().numpy()[0], pm.cpu().numpy()[m])
        # the multi-row kernel adds each row's group terms in the M = 1 kernel's order (same team
        # size and chunk slots at this shape), so the bf16 outputs agree bit for bit too
        np.testing.assert_array_equal(y1.cpu().numpy()[0], ym.cpu().numpy()[m])


# M = 3..8 from bf16 x: every workgroup quantizes the rows into LDS and runs the
# matrix-core kernel the prequantized entry runs on the workspace layout, with
# the same quantize arithmetic and summation order, so at M = 5..8 (where the
# prequantized entry takes that kernel too) the outputs are bit-identical.
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,M", [(1000, 2560, 5), (2100, 2560, 8), (64, 4096, 6), (10240, 2560, 7)])
def test_bf16_rows_match_prequantized(torch_dev, qtype, N, K, M):
    torch = torch_dev
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, 60 + M, O.SCALE_BF16)
    x = O.gen_act(M, K, 61 + M, outlier_frac=0.05, outlier_mul=20.0)
    res = O.gen_act(M, N, 62 + M)
    xq, xs = O.quantize_act(x, G)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc.BF16)
    ws = torch.zeros(va.workspace_bytes(qtype, N, K, M), dtype=torch.uint8, device="cuda")
    ya = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    yb = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear(w, dev(torch, x), ya, residual=dev(torch, res), workspace=ws).ok()
    assert va.linear_prequantized(w, dev(torch, xq), dev(torch, xs), yb, residual=dev(torch, res)).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ya, np.uint16), host(yb, np.uint16))
    y_ref, _, absterm = O.qlinear(qtype, packed, scales, O.SCALE_BF16, N, K, x, residual=res)
    O.assert_bf16_close(host(ya, np.uint16), y_ref, absterm, rel=REL_TOL)


@pytest.mark.parametrize("N,K,M", [(200, 2560, 3), (70, 10240, 16), (40, 192, 2), (6001, 4096, 16), (45, 10240, 4),
                                   (300, 10240, 3), (130, 7680, 2), (90, 7680, 3), (90, 7680, 4),
                                   (47, 10240, 3)])
def test_prequantized_entry(torch_dev, N, K, M):
    # activations in viper_hip_quantize_act's layout ([M][K] int8, [M][K/G] fp32)
    torch = torch_dev
    for qtype in FORMATS:
        G = O.group_size(qtype)
        packed, scales = O.gen_weights(qtype, N, K, 40 + qtype, O.SCALE_BF16)
        x = O.gen_act(M, K, 41)
        xq, xs = O.quantize_act(x, G)
        res = O.gen_act(M, N, 42)
        y_ref, _, absterm = O.qlinear_prequant(qtype, packed, scales, O.SCALE_BF16, N, K, xq, xs, residual=res)
        w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, va.ScaleEnc.BF16)
        yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
        st = va.linear_prequantized(w, dev(torch, xq), dev(torch, xs), yd, residual=dev(torch, res))
        assert st.ok(), st
        torch.cuda.synchronize()
        O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K", [(2560, 2560), (61, 10240), (10240, 2560), (10010, 2560), (3072, 10752),
                                 (6144, 3072), (3001, 6144), (10752, 3072), (11000, 3072)])
def test_prequantized_m1(torch_dev, qtype, N, K):
    # M = 1 from int8 activations: the M = 1 kernel's prequantized prologue
    # (one octet per thread on 256 threads; Q4's two octets per thread on 320
    # and 640, a ragged last workgroup at N = 10010; the reference engine's K
    # on the 6-slot tilings and the masked K = 10752 one; Q4 / Q5 at K = 3072
    # and N = 10752 / 11000 on the 44-row workgroup, ragged at 11000)
    torch = torch_dev
    G = O.group_size(qtype)
    packed, scales = O.gen_weights(qtype, N, K, 50 + qtype, O.SCALE_FP16)
    xq, xs = O.quantize_act(O.gen_act(1, K, 51, outlier_frac=0.05, outlier_mul=20.0), G)
    res = O.gen_act(1, N, 52)
    y_ref, _, absterm = O.qlinear_prequant(qtype, packed, scales, O.SCALE_FP16, N, K, xq, xs, residual=res)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, scale_enc=va.ScaleEnc.FP16)
    yd = torch.zeros((1, N), dtype=torch.int16, device="cuda")
    assert va.linear_prequantized(w, dev(torch, xq), dev(torch, xs), yd, residual=dev(torch, res)).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


# Two matrices of one shape on one activation in one launch (the reference's
# fused2 for k/v and gate/up): M = 1 (fused quantize), M > 1 (matrix cores),
# K with an odd group count (two v_dot4 launches).
@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,M", [(300, 2560, 1), (5120, 2560, 1), (70, 2560, 16), (90, 2560, 6), (33, 192, 3)])
@pytest.mark.parametrize("prequantized", [False, True])
def test_fused2(torch_dev, qtype, N, K, M, prequantized):
    torch = torch_dev
    G = O.group_size(qtype)
    note(f"fused2 qtype={qtype} N={N} K={K} M={M} pre={prequantized}")
    p0, s0 = O.gen_weights(qtype, N, K, 60 + qtype, O.SCALE_BF16)
    p1, s1 = O.gen_weights(qtype, N, K, 70 + qtype, O.SCALE_BF16)
    x = O.gen_act(M, K, 61)
    xq, xs = O.quantize_act(x, G)
    refs = [O.qlinear_prequant(qtype, p, sc, O.SCALE_BF16, N, K, xq, xs) for p, sc in ((p0, s0), (p1, s1))]
    w0 = va.QuantizedWeight(va.QType(qtype), dev(torch, p0), dev(torch, s0), N, K, G, va.ScaleEnc.BF16)
    w1 = va.QuantizedWeight(va.QType(qtype), dev(torch, p1), dev(torch, s1), N, K, G, va.ScaleEnc.BF16)
    y0 = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    y1 = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    if prequantized:
        st = va.linear_fused2_prequantized(w0, w1, dev(torch, xq), dev(torch, xs), y0, y1)
    else:
        nws = va.workspace_bytes(qtype, N, K, M)
        ws = torch.zeros(max(16, nws), dtype=torch.uint8, device="cuda") if nws else None
        st = va.linear_fused2(w0, w1, dev(torch, x), y0, y1, workspace=ws)
    assert st.ok(), st
    torch.cuda.synchronize()
    for yd, (y_ref, _, absterm) in zip((y0, y1), refs):
        O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


# The same random shapes through the prequantized entry and both fused-pair
# entries (bf16 rows and prequantized), each output against the oracle.
@pytest.mark.parametrize("qtype,N,K,M,senc,residual", _random_shapes(n=16, seed=0x5EED8))
def test_random_shapes_prequantized_and_fused2(torch_dev, qtype, N, K, M, senc, residual):
    torch = torch_dev
    G = O.group_size(qtype)
    note(f"random pre/fused2 qtype={qtype} N={N} K={K} M={M} senc={senc} res={residual}")
    p0, s0 = O.gen_weights(qtype, N, K, 9300 + N, senc)
    p1, s1 = O.gen_weights(qtype, N, K, 9301 + N, senc)
    x = O.gen_act(M, K, 9302 + M, outlier_frac=0.05)
    xq, xs = O.quantize_act(x, G)
    res = O.gen_act(M, N, 9303) if residual else None
    ref_res = O.qlinear_prequant(qtype, p0, s0, senc, N, K, xq, xs, residual=res)
    refs = [O.qlinear_prequant(qtype, p, sc, senc, N, K, xq, xs) for p, sc in ((p0, s0), (p1, s1))]
    w0 = va.QuantizedWeight(va.QType(qtype), dev(torch, p0), dev(torch, s0), N, K, G, va.ScaleEnc(senc))
    w1 = va.QuantizedWeight(va.QType(qtype), dev(torch, p1), dev(torch, s1), N, K, G, va.ScaleEnc(senc))
    xqd, xsd = dev(torch, np.asarray(xq, dtype=np.int8)), dev(torch, np.asarray(xs, dtype=np.float32))
    z = lambda: torch.zeros((M, N), dtype=torch.int16, device="cuda")
    yp, a0, a1, b0, b1 = z(), z(), z(), z(), z()
    assert va.linear_prequantized(w0, xqd, xsd, yp, residual=None if res is None else dev(torch, res)).ok()
    nws = va.workspace_bytes(qtype, N, K, M)
    ws = torch.zeros(max(16, nws), dtype=torch.uint8, device="cuda") if nws else None
    assert va.linear_fused2(w0, w1, dev(torch, x), a0, a1, workspace=ws).ok()
    assert va.linear_fused2_prequantized(w0, w1, xqd, xsd, b0, b1).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(host(yp, np.uint16), ref_res[0], ref_res[2], rel=REL_TOL)
    for pair in ((a0, a1), (b0, b1)):
        for yd, (y_ref, _, absterm) in zip(pair, refs):
            O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


def test_fused2_matches_two_calls(torch_dev):
    # bit-identical to two single-matrix calls
    torch = torch_dev
    N, K, M = 512, 2560, 1
    mats = [O.gen_weights(O.Q4_G64, N, K, s, O.SCALE_FP16) for s in (81, 82)]
    ws = [va.QuantizedWeight(va.QType.Q4_G64, dev(torch, p), dev(torch, sc), N, K, scale_enc=va.ScaleEnc.FP16) for p, sc in mats]
    x = dev(torch, O.gen_act(M, K, 83))
    ya = [torch.zeros((M, N), dtype=torch.int16, device="cuda") for _ in range(2)]
    yb = [torch.zeros((M, N), dtype=torch.int16, device="cuda") for _ in range(2)]
    assert va.linear_fused2(ws[0], ws[1], x, ya[0], ya[1]).ok()
    for w, y in zip(ws, yb):
        assert va.linear(w, x, y).ok()
    torch.cuda.synchronize()
    for a, b in zip(ya, yb):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


@pytest.mark.parametrize("N,K,M", [(10240, 2560, 1), (1000, 2560, 16), (2560, 10240, 5), (640, 2560, 5)])
def test_output_and_residual_two_byte_aligned(torch_dev, N, K, M):
    # y and the residual need only 2-byte alignment: one element off a 16-byte
    # boundary gives the same bits as aligned buffers (M = 1, the matrix-core
    # kernel from fragments, the K split, the one-launch bf16-row path)
    torch = torch_dev
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 91 + M, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, scale_enc=va.ScaleEnc.FP16)
    x = dev(torch, O.gen_act(M, K, 92))
    res = O.gen_act(M, N, 93)
    ws = torch.zeros(max(16, va.workspace_bytes(4, N, K, M)), dtype=torch.uint8, device="cuda") if M > 1 else None
    ya = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    ra = dev(torch, res)
    yb_buf = torch.zeros(M * N + 1, dtype=torch.int16, device="cuda")
    rb_buf = torch.zeros(M * N + 1, dtype=torch.int16, device="cuda")
    rb_buf[1:] = ra.view(-1)
    yb, rb = yb_buf[1:].view(M, N), rb_buf[1:].view(M, N)
    assert yb.data_ptr() % 16 == 2 and rb.data_ptr() % 16 == 2
    assert va.linear(w, x, ya, residual=ra, workspace=ws).ok()
    assert va.linear(w, x, yb, residual=rb, workspace=ws).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ya.cpu().numpy(), yb.cpu().numpy())
    assert int(yb_buf[0].item()) == 0  # nothing written before the output


@pytest.mark.parametrize("M", [1, 3])
def test_residual_in_place(torch_dev, M):
    # y aliasing the residual, as the reference engine calls its residual GEMV
    # (include/viper/model_impl.cuh:720,728: y = residual = x_)
    torch = torch_dev
    N, K = 2560, 2560
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 71, O.SCALE_FP16)
    x = O.gen_act(M, K, 72)
    res = O.gen_act(M, N, 73)
    y_ref, _, absterm = O.qlinear(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, residual=res)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, scale_enc=va.ScaleEnc.FP16)
    yd = dev(torch, res)
    ws = torch.zeros(max(16, va.workspace_bytes(4, N, K, M)), dtype=torch.uint8, device="cuda") if M > 1 else None
    assert va.linear(w, dev(torch, x), yd, residual=yd, workspace=ws).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


def test_wrapper_rejects_non_contiguous(torch_dev):
    # a strided view would be read as a dense array: the wrapper refuses it
    torch = torch_dev
    N, K = 64, 128
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 61, O.SCALE_FP16)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, scale_enc=va.ScaleEnc.FP16)
    xt = torch.zeros((K, 2), dtype=torch.int16, device="cuda").t()
    assert not xt.is_contiguous()
    with pytest.raises(ValueError):
        va.linear(w, xt, torch.zeros((2, N), dtype=torch.int16, device="cuda"),
                  workspace=torch.zeros(va.workspace_bytes(4, N, K, 2), dtype=torch.uint8, device="cuda"))
    # and an fp32 x, which would be read as pairs of bf16
    with pytest.raises(ValueError):
        va.linear(w, torch.zeros((1, K), dtype=torch.float32, device="cuda"),
                  torch.zeros((1, N), dtype=torch.int16, device="cuda"))


def test_zero_weight_kat(torch_dev):
    # all-0x88 Q4 bytes are all-zero weights: y is exactly the residual
    torch = torch_dev
    N, K = 64, 2560
    packed = np.full(N * K // 2, 0x88, np.uint8)
    scales = np.full(N * K // 64, 0x3C00, np.uint16)
    x = O.gen_act(1, K, 3)
    res = O.gen_act(1, N, 4)
    w = va.QuantizedWeight(va.QType.Q4_G64, dev(torch, packed), dev(torch, scales), N, K, scale_enc=va.ScaleEnc.FP16)
    yd = torch.zeros((1, N), dtype=torch.int16, device="cuda")
    assert va.linear(w, dev(torch, x), yd, residual=dev(torch, res)).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(yd, np.uint16), res)


def test_deterministic(torch_dev):
    a = run_case(torch_dev, O.Q6_G64, 513, 4096, 1, seed=9)
    b = run_case(torch_dev, O.Q6_G64, 513, 4096, 1, seed=9)
    np.testing.assert_array_equal(a, b)


def test_device_errors_are_codes(torch_dev):
    torch = torch_dev
    N, K = 64, 128
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 1, O.SCALE_FP16)
    wd, sd = dev(torch, packed), dev(torch, scales)
    x = dev(torch, O.gen_act(2, K, 1))
    y = torch.zeros((2, N), dtype=torch.int16, device="cuda")
    w = va.QuantizedWeight(va.QType.Q4_G64, wd, sd, N, K, scale_enc=va.ScaleEnc.FP16)
    assert va.linear(w, x, y).code == va.StatusCode.INVALID_ARGUMENT        # M=2 without workspace
    small = torch.zeros(16, dtype=torch.uint8, device="cuda")
    assert va.linear(w, x, y, workspace=small).code == va.StatusCode.INVALID_ARGUMENT
    wbad = va.QuantizedWeight(va.QType.BF16, wd, sd, N, K, scale_enc=va.ScaleEnc.FP16)
    assert va.linear(wbad, x, y).code == va.StatusCode.UNIMPLEMENTED
    assert va.linear(w, x[:1], y[:1, :N - 1]).code == va.StatusCode.SHAPE_MISMATCH


def crafted_act(M, K, G, seed):
    """Rows whose groups hit the quantizer's special cases, rotated per row: an all-zero group
    (scale 1e-8, q = 0), a group with amax 127 and exact .5 ties (scale 1: RNE to even), a group of
    values near 1e-6, a x20 outlier group, random groups elsewhere."""
    x = O.bf16_to_f32(O.gen_act(M, K, seed)).copy()
    ties = np.array([127.0, 2.5, 3.5, -2.5, 0.5, -1.5, -0.5, 1.5], dtype=np.float32)
    for m in range(M):
        g0 = (m % 4) * G
        x[m, g0:g0 + G] = 0.0
        g1 = ((m + 1) % 4) * G
        x[m, g1:g1 + G] = np.resize(ties, G)
        g2 = ((m + 2) % 4) * G
        x[m, g2:g2 + G] = np.linspace(-1e-6, 1e-6, G, dtype=np.float32)
        g3 = ((m + 3) % 4) * G
        x[m, g3:g3 + G] *= 20.0
    return O.f32_to_bf16(x)


# The quantize is fused into every GEMV path (the M = 1 prologue, M = 2 rows in
# the M = 1 kernel, M = 3..8 into LDS in the matrix-core kernel, the fragment
# quantize launch beyond): each must give the oracle's int8 values, so the
# group dots are bit-exact on the quantizer's special cases.
@pytest.mark.parametrize("qtype", [O.Q4_G64, O.Q6_G64, O.W8_G32])
@pytest.mark.parametrize("M", [1, 2, 5, 12])
def test_quantizer_edge_cases_every_path(torch_dev, qtype, M):
    torch = torch_dev
    N, K = 77, 2560
    G = O.group_size(qtype)
    note(f"case qtype={qtype} M={M} crafted activations")
    packed, scales = O.gen_weights(qtype, N, K, 90 + M, O.SCALE_FP16)
    x = crafted_act(M, K, G, 91 + M)
    xq, _ = O.quantize_act(x, G)
    assert list(xq[0, G:G + 8]) == [127, 2, 4, -2, 0, -2, 0, 2]   # the ties group of row 0
    D_ref = O.group_dots(qtype, packed, N, K, xq)
    y_ref, _, absterm = O.qlinear(qtype, packed, scales, O.SCALE_FP16, N, K, x)
    w = va.QuantizedWeight(va.QType(qtype), dev(torch, packed), dev(torch, scales), N, K, G, scale_enc=va.ScaleEnc.FP16)
    yd = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    pd = torch.full((M, N, K // G), -7, dtype=torch.int32, device="cuda")
    nws = va.workspace_bytes(qtype, N, K, M)
    wsd = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda") if nws else None
    assert va.linear_partials(w, dev(torch, x), yd, pd, workspace=wsd).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(pd, np.int32), D_ref)
    O.assert_bf16_close(host(yd, np.uint16), y_ref, absterm, rel=REL_TOL)


def test_clock_stamp_probe(torch_dev):
    # two device-clock readings around some work on one stream: ordered, within a second (100 MHz
    # ticks); null and misaligned outputs are rejected before any launch
    torch = torch_dev
    L = va.lib()
    t = torch.zeros(2, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.viper_hip_clock_stamp(t.data_ptr(), st) == 0
    a = torch.randn(1 << 22, device="cuda")
    for _ in range(4):
        a = a * 1.0001
    assert L.viper_hip_clock_stamp(t.data_ptr() + 8, st) == 0
    torch.cuda.synchronize()
    t0, t1 = t.cpu().tolist()
    assert 0 < t1 - t0 < 100_000_000
    assert L.viper_hip_clock_stamp(None, st) == 2
    assert L.viper_hip_clock_stamp(t.data_ptr() + 4, st) == 2


def test_empty_dispatch_probe(torch_dev):
    # the dispatch-cost probe: with y, lane 0 of every 16-lane team stores its row index (as a
    # 16-bit word) and nothing else is written; without y nothing is written; bad launch shapes and a
    # misaligned y are rejected before any launch
    torch = torch_dev
    L = va.lib()
    st = torch.cuda.current_stream().cuda_stream
    wg, nt = 512, 320
    rows = wg * nt // 16
    y = torch.full((rows + 8,), -1, dtype=torch.int16, device="cuda")
    assert L.viper_hip_empty_dispatch(wg, nt, None, st) == 0
    torch.cuda.synchronize()
    assert bool((y == -1).all())
    assert L.viper_hip_empty_dispatch(wg, nt, y.data_ptr(), st) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got[:rows], (np.arange(rows) & 0xFFFF).astype(np.uint16))
    assert (got[rows:] == 0xFFFF).all()
    assert L.viper_hip_empty_dispatch(0, nt, None, st) == 2
    assert L.viper_hip_empty_dispatch(wg, 100, None, st) == 2
    assert L.viper_hip_empty_dispatch(wg, 2048, None, st) == 2
    assert L.viper_hip_empty_dispatch(wg, nt, y.data_ptr() + 1, st) == 2


def test_stream_read_probe(torch_dev):
    # the measurement probe reads every byte: a lane whose chunks fold to the
    # magic word writes it to the sink, zeros leave the sink alone; with y,
    # lane 0 of every 16-lane team stores its fold to y[row] (rows of
    # 16 * loads 16-byte chunks, any workgroup order)
    torch = torch_dev
    L = va.lib()
    threads, loads = 320, 5
    rowb = 16 * loads * 16
    rows = 20 * 40
    buf = torch.zeros(rows * rowb, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.viper_hip_stream_read(buf.data_ptr(), buf.numel(), threads, loads, None, 0, None, sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert int(sink[0]) == 0
    words = buf.view(torch.int32)
    words[buf.numel() // 4 - 4] = np.int32(np.uint32(0x9E3779B9).view(np.int32))   # the last 16 bytes
    assert L.viper_hip_stream_read(buf.data_ptr(), buf.numel(), threads, loads, None, 0, None, sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert np.uint32(int(sink[0]) & 0xFFFFFFFF) == np.uint32(0x9E3779B9)
    # the side blocks (one per workgroup, as the GEMV's scale blocks) are read
    # too: the magic word in the last workgroup's block reaches the sink
    buf.zero_()
    sink.zero_()
    nwg, sb = rows // 20, 1600
    side = torch.zeros(nwg * sb, dtype=torch.uint8, device="cuda")
    assert L.viper_hip_stream_read(buf.data_ptr(), buf.numel(), threads, loads, side.data_ptr(), sb, None,
                                   sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert int(sink[0]) == 0
    side.view(torch.int32)[(nwg * sb - 16) // 4] = np.int32(np.uint32(0x9E3779B9).view(np.int32))
    assert L.viper_hip_stream_read(buf.data_ptr(), buf.numel(), threads, loads, side.data_ptr(), sb, None,
                                   sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert np.uint32(int(sink[0]) & 0xFFFFFFFF) == np.uint32(0x9E3779B9)
    buf.zero_()
    words[torch.arange(rows, device="cuda") * (rowb // 4)] = torch.arange(rows, dtype=torch.int32, device="cuda")
    y = torch.full((buf.numel() // (16 * 4 * 16),), -1, dtype=torch.int16, device="cuda")   # rows of the smallest row size
    for th, ld in ((320, 5), (640, 5), (64, 16), (1024, 4)):
        rb = 16 * ld * 16
        n = buf.numel() // (th * ld * 16) * (th * ld * 16)
        assert n // rb <= y.numel()
        words.zero_()
        words[torch.arange(n // rb, device="cuda") * (rb // 4)] = torch.arange(n // rb, dtype=torch.int32, device="cuda")
        y.fill_(-1)
        assert L.viper_hip_stream_read(buf.data_ptr(), n, th, ld, None, 0, y.data_ptr(), sink.data_ptr(), st) == 0
        torch.cuda.synchronize()
        got = y.cpu().numpy()[: n // rb].astype(np.int64)
        np.testing.assert_array_equal(got, np.arange(n // rb))


@pytest.mark.parametrize("qt", [O.Q4_G64, O.Q5_G64, O.Q6_G64, O.W8_G32])
def test_timeline_entry_matches_gemv(torch_dev, qt):
    # the measurement entry point runs the production GEMV with stamps: y equal
    # to viper_hip_qlinear's bit for bit, 8 non-decreasing readings per wave,
    # and shapes without an exact tiling rejected
    import ctypes as C
    torch = torch_dev
    L = va.lib()
    N, K = 4000, 2560
    G = 32 if qt == O.W8_G32 else 64
    packed, scales = O.gen_weights(qt, N, K, 0x71, O.SCALE_FP16)
    x = O.gen_act(1, K, 0x72)
    wd, sd, xd = dev(torch, packed), dev(torch, scales), dev(torch, x)
    y0 = torch.zeros((1, N), dtype=torch.int16, device="cuda")
    y1 = torch.full((1, N), 7, dtype=torch.int16, device="cuda")
    stamps = torch.zeros(1 << 18, dtype=torch.int64, device="cuda")
    grid, waves = C.c_int(0), C.c_int(0)
    st = torch.cuda.current_stream().cuda_stream
    assert L.viper_hip_qlinear(qt, wd.data_ptr(), sd.data_ptr(), 0, G, N, K, xd.data_ptr(), 1, y0.data_ptr(),
                               None, None, 0, st) == 0
    assert L.viper_hip_qlinear_timeline(qt, wd.data_ptr(), sd.data_ptr(), 0, G, N, K, xd.data_ptr(), y1.data_ptr(),
                                        stamps.data_ptr(), stamps.numel() * 8, C.byref(grid), C.byref(waves), st) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y1, np.uint16), host(y0, np.uint16))
    nw = grid.value * waves.value
    assert nw > 0
    t = stamps[: nw * 8].view(nw, 8).cpu().numpy()
    assert (np.diff(t, axis=1) >= 0).all() and (t[:, 0] > 0).all()
    assert L.viper_hip_qlinear_timeline(qt, wd.data_ptr(), sd.data_ptr(), 0, G, N, K, xd.data_ptr(), y1.data_ptr(),
                                        stamps.data_ptr(), 64, None, None, st) == 2          # stamps too small
    assert L.viper_hip_qlinear_timeline(qt, wd.data_ptr(), sd.data_ptr(), 0, G, N, 2496, xd.data_ptr(),
                                        y1.data_ptr(), stamps.data_ptr(), stamps.numel() * 8, None, None, st) == 2
