"""Pins of the CPU oracle (oracle/viper_oracle.c) before it is trusted as the
checker of the HIP kernels.  CPU only.

Each test is chosen so that a plausible restatement mistake fails it:
  * the Q4 weight format against the reference's own converter
    (tools/convert/convert.cpp:91-127, built from /root/reference into oracle/_ref);
  * pack/unpack of every format against an independent numpy statement of the
    documented bit layout, over every code value in every position;
  * fp16/bf16 conversions against numpy's IEEE routines, exhaustively;
  * the activation quantizer (rmsnorm_quantize.cu:93,101; linear_multim.cu:51,57)
    against known answers (zero group -> scale 1e-8, ties to even, amax -> 127)
    and numpy's IEEE float32 divide + rint;
  * the division-free identity used on the GPU, exhaustively over bf16;
  * group dots against an int64 numpy brute force, linearity, the all-0x88
    zero-weight known answer (tests/dp4a_clean.cu:248 fills weights with 0x88);
  * the fp32 combine against a float64 sum and the bf16 rounding closed form.
"""
import numpy as np
import pytest

import oracle as O

FORMATS = [O.Q4_G64, O.Q5_G64, O.Q6_G64, O.W8_G32]


# ---------------------------------------------------------------- layouts

def np_pack(qtype, w):
    """Independent numpy statement of the documented layouts (oracle/viper_oracle.h)."""
    w = w.astype(np.int64)
    N, K = w.shape
    if qtype == O.W8_G32:
        return w.astype(np.int8).view(np.uint8).reshape(-1)
    off = {O.Q4_G64: 8, O.Q5_G64: 16, O.Q6_G64: 32}[qtype]
    u = w + off
    lo = ((u[:, 0::2] & 15) | ((u[:, 1::2] & 15) << 4)).astype(np.uint8).reshape(-1)
    if qtype == O.Q4_G64:
        return lo
    u5 = u.reshape(N, K // 32, 4, 4, 2)  # [n, c, i, b, p]
    i = np.arange(4).reshape(4, 1, 1)
    b = np.arange(4).reshape(1, 4, 1)
    p = np.arange(2).reshape(1, 1, 2)
    if qtype == O.Q5_G64:
        sh = (8 * b + 2 * i + p).astype(np.uint64)
        bits = ((u5 >> 4) & 1).astype(np.uint64) << sh
        W = bits.reshape(N, K // 32, -1).sum(axis=2).astype(np.uint32)  # disjoint bits
        hi = W.reshape(-1).view(np.uint8)
    else:
        sh = (8 * b + 4 * (i % 2) + 2 * p).astype(np.uint64)
        f = ((u5 >> 4) & 3).astype(np.uint64) << sh
        W = np.stack([f[:, :, 0:2].reshape(N, K // 32, -1).sum(axis=2),
                      f[:, :, 2:4].reshape(N, K // 32, -1).sum(axis=2)], axis=2).astype(np.uint32)
        hi = W.reshape(-1).view(np.uint8)
    return np.concatenate([lo, hi])


@pytest.mark.parametrize("qtype", FORMATS)
def test_pack_every_code_every_position(qtype):
    lo, hi = O.wrange(qtype)
    codes = np.arange(lo, hi + 1)
    K = 64 * ((len(codes) + 63) // 64) if qtype != O.W8_G32 else 256
    # row r holds the codes rotated by r, so every code visits every column phase
    N = len(codes)
    base = np.resize(codes, K)
    w = np.stack([np.roll(base, r) for r in range(N)]).astype(np.int8)
    packed = O.pack(qtype, w)
    assert packed.size == O.packed_bytes(qtype, N, K)
    np.testing.assert_array_equal(packed, np_pack(qtype, w))
    np.testing.assert_array_equal(O.unpack(qtype, packed, N, K), w)


def test_q4_known_bytes():
    # all-0x88 bytes decode to all-zero weights; 0x0F -> (k even: 7, k odd: -8)
    np.testing.assert_array_equal(O.unpack(O.Q4_G64, np.full(32, 0x88, np.uint8), 1, 64), 0)
    w = O.unpack(O.Q4_G64, np.full(32, 0x0F, np.uint8), 1, 64)
    np.testing.assert_array_equal(w[0, 0::2], 7)
    np.testing.assert_array_equal(w[0, 1::2], -8)


# ---------------------------------------------------- reference converter

def _ref_or_skip():
    if O.ref_lib() is None:
        pytest.skip("oracle/_ref not built (needs /root/reference)")


def _bf16(a):
    return O.f32_to_bf16(np.asarray(a, np.float32))


@pytest.mark.parametrize("shape,seed", [((8, 64), 1), ((33, 192), 2), ((128, 2560), 3)])
def test_q4_weight_quantizer_matches_reference_convert(shape, seed):
    _ref_or_skip()
    rng = np.random.default_rng(seed)
    w = rng.standard_normal(shape).astype(np.float32) * rng.uniform(0.01, 3.0, (shape[0], 1)).astype(np.float32)
    w[0, :64] = 0.0                                   # all-zero group: scale floor 1e-8
    if shape[0] > 1:                                  # exact ties v/scale = k + 0.5
        w[1, :64] = 0.25 * np.resize(np.arange(-7.5, 8.0, 1.0), 64)
        w[1, 0] = 7 * 0.25
    if shape[0] > 2:
        w[2, :64] = rng.standard_normal(64) * 1e-30       # tiny values
    wb = _bf16(w)
    p_ref, s_ref = O.ref_quantize_q4_g64(wb)
    p, s = O.quantize_weights(O.Q4_G64, wb, O.SCALE_BF16)
    np.testing.assert_array_equal(p, p_ref)
    np.testing.assert_array_equal(s, s_ref)


@pytest.mark.parametrize("scale_enc", [O.SCALE_BF16, O.SCALE_FP16])
@pytest.mark.parametrize("qtype", O.QTYPES)
def test_weight_quantizer_roundtrip_every_format(qtype, scale_enc):
    """vo_quantize_weights on representable weights w = c * 2^e: each group's
    largest |c| is the format's top code wmax, so scale = wmax*2^e / wmax =
    2^e exactly (both 16-bit encodings hold it) and every code comes back.
    Half-way values (c + 1/2) * 2^e round half away from zero, as
    convert.cpp:115-117's std::round; the low end -wmax-1 (Q5/Q6: -16/-32)
    is reached by a tie only.  No reference pins the Q5/Q6/W8 branches, so
    the closed form does."""
    rng = np.random.default_rng(100 + qtype)
    G = O.group_size(qtype)
    wmin, wmax = O.wrange(qtype)
    N, K = 6, 4 * G
    codes = rng.integers(-wmax, wmax + 1, size=(N, K))
    e = rng.integers(-12, 3, size=(N, K // G))
    for n in range(N):
        for g in range(K // G):
            codes[n, g * G + int(rng.integers(0, G))] = wmax if rng.random() < 0.5 else -wmax
    expo = np.repeat(e, G, axis=1).astype(np.float64)
    w = codes * 2.0 ** expo
    p, s = O.quantize_weights(qtype, _bf16(w), scale_enc)
    np.testing.assert_array_equal(O.unpack(qtype, p, N, K), codes)
    if scale_enc == O.SCALE_BF16:
        got = O.bf16_to_f32(s).reshape(N, K // G)
    else:
        got = s.view(np.float16).astype(np.float32).reshape(N, K // G)
    np.testing.assert_array_equal(got, (2.0 ** e).astype(np.float32))
    # ties: (c + 1/2) * 2^e -> c + 1 for c >= 0, c - 1 ... away from zero, in range
    wt = np.zeros((1, G))
    wt[0, 0] = wmax                                   # scale 1
    half = np.arange(-(wmax - 1), wmax - 1) + 0.5     # every tie whose result is a valid code
    wt[0, 1:1 + min(len(half), G - 1)] = half[:G - 1]
    p, s = O.quantize_weights(qtype, _bf16(wt), scale_enc)
    got = O.unpack(qtype, p, 1, G)[0, 1:1 + min(len(half), G - 1)]
    h = half[:G - 1]
    np.testing.assert_array_equal(got, np.where(h > 0, np.floor(h) + 1, np.ceil(h) - 1))


def test_reference_ties_round_half_away():
    _ref_or_skip()
    # max 1.75 -> scale 0.25 exactly; 0.625/0.25 = 2.5 -> 3 (away from zero)
    w = np.zeros((1, 64), np.float32)
    w[0, 0] = 1.75
    w[0, 1] = 0.625
    w[0, 2] = -0.625
    p, s = O.ref_quantize_q4_g64(_bf16(w))
    wq = O.unpack(O.Q4_G64, p, 1, 64)
    assert wq[0, 0] == 7 and wq[0, 1] == 3 and wq[0, 2] == -3
    assert O.bf16_to_f32(s[0]) == np.float32(0.25)


# ------------------------------------------------------------ conversions

def test_f16_roundtrip_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    L = O.lib()
    f = np.array([L.vo_f16_to_f32(int(v)) for v in h], np.float32)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(f[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(f[np.isnan(ref)]).all()


def test_f32_to_f16_and_bf16_rne():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(1e-3),
        rng.uniform(-70000, 70000, 2000).astype(np.float32),
        np.float32([1e-8, 6.1e-5, 5.96e-8, 65504.0, 65520.0, -0.0, 2.0 ** -25]),
        # exact half-way cases for bf16 (low 16 bits = 0x8000)
        ((rng.integers(0x3f000000, 0x40ffffff, 500, dtype=np.uint32) & 0xFFFF0000) | 0x8000).view(np.float32),
    ])
    L = O.lib()
    f16 = np.array([L.vo_f32_to_f16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(f16, vals.astype(np.float16).view(np.uint16))
    bf = np.array([L.vo_f32_to_bf16(float(v)) for v in vals], np.uint16)
    # bf16 RNE via float64: nearest multiple of the bf16 spacing, ties to even mantissa
    u = vals.view(np.uint32).astype(np.uint64)
    trunc = (u >> 16)
    rem = u & 0xFFFF
    up = (rem > 0x8000) | ((rem == 0x8000) & ((trunc & 1) == 1))
    np.testing.assert_array_equal(bf, (trunc + up).astype(np.uint16))


# ---------------------------------------------------- activation quantize

def np_quantize_act(x_bf16, group):
    """numpy IEEE float32: s = max(amax/127, 1e-8); q = rint(x/s) clipped."""
    x = O.bf16_to_f32(x_bf16).astype(np.float32)
    M, K = x.shape
    xg = x.reshape(M, K // group, group)
    amax = np.abs(xg).max(axis=2)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(xg / s[:, :, None]), -127, 127).astype(np.int8)
    return q.reshape(M, K), s


@pytest.mark.parametrize("group", [64, 32])
def test_quantize_act_known_answers(group):
    x = np.zeros((1, 4 * group), np.float32)
    # group 0: all zero -> scale 1e-8, q = 0
    # group 1: amax 127 -> scale exactly 1; ties 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0
    g1 = x[0, group:2 * group]
    g1[0], g1[1], g1[2], g1[3], g1[4], g1[5] = 127.0, 2.5, 3.5, -2.5, 0.5, -1.5
    # group 2: negative amax element -> -127
    x[0, 2 * group:3 * group] = np.linspace(-3.0, 1.0, group)
    # group 3: tiny values below the floor: scale 1e-8, q = RNE(x / 1e-8)
    x[0, 3 * group:4 * group] = np.linspace(-1e-6, 1e-6, group)
    xb = _bf16(x)
    q, s = O.quantize_act(xb, group)
    assert s[0, 0] == np.float32(1e-8) and (q[0, :group] == 0).all()
    assert s[0, 1] == np.float32(1.0)
    assert list(q[0, group:group + 6]) == [127, 2, 4, -2, 0, -2]
    assert q[0, 2 * group] == -127
    assert s[0, 3] == np.float32(1e-8)
    nq, ns = np_quantize_act(xb, group)
    np.testing.assert_array_equal(q, nq)
    np.testing.assert_array_equal(s, ns)


@pytest.mark.parametrize("group", [64, 32])
def test_quantize_act_matches_numpy_and_invariants(group):
    x = O.gen_act(5, 2560, 99, outlier_frac=0.05, outlier_mul=20.0)
    q, s = O.quantize_act(x, group)
    nq, ns = np_quantize_act(x, group)
    np.testing.assert_array_equal(q, nq)
    np.testing.assert_array_equal(s, ns)
    xf = O.bf16_to_f32(x)
    assert np.abs(q.astype(int)).max() <= 127
    assert ((np.sign(q) == np.sign(xf)) | (q == 0)).all()
    # every group holds its amax element at +-127
    assert (np.abs(q.reshape(5, -1, group)).max(axis=2) == 127).all()


def test_division_free_identity_exhaustive():
    bad, n = O.check_markstein(0, 254)
    assert n == 532701120
    assert bad == 0


# ------------------------------------------------------------------ dots

def _dots_np(qtype, packed, N, K, xq):
    w = O.unpack(qtype, packed, N, K).astype(np.int64)
    G = O.group_size(qtype)
    M = xq.shape[0]
    wg = w.reshape(N, K // G, G)
    qg = xq.astype(np.int64).reshape(M, K // G, G)
    return np.einsum("ngj,mgj->mng", wg, qg)


@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("N,K,M", [(3, 64, 1), (8, 128, 5), (5, 256, 16)])
def test_group_dots_bruteforce_and_linearity(qtype, N, K, M):
    packed, _ = O.gen_weights(qtype, N, K, 1234 + N, O.SCALE_FP16)
    rng = np.random.default_rng(K + M)
    q1 = rng.integers(-63, 64, (M, K)).astype(np.int8)
    q2 = rng.integers(-63, 64, (M, K)).astype(np.int8)
    D1 = O.group_dots(qtype, packed, N, K, q1)
    np.testing.assert_array_equal(D1, _dots_np(qtype, packed, N, K, q1))
    D2 = O.group_dots(qtype, packed, N, K, q2)
    D12 = O.group_dots(qtype, packed, N, K, (q1.astype(np.int16) + q2).astype(np.int8))
    np.testing.assert_array_equal(D12, D1 + D2)


def test_extreme_dot_magnitude():
    # |D| <= G * max|w| * 127; Q6 at -32 x -127 is the largest per-weight term
    for qtype in FORMATS:
        lo, hi = O.wrange(qtype)
        G = O.group_size(qtype)
        w = np.full((1, 64), lo, np.int8)
        packed = O.pack(qtype, w)
        D = O.group_dots(qtype, packed, 1, 64, np.full((1, 64), -127, np.int8))
        assert (D == lo * -127 * G).all()


# --------------------------------------------------------------- combine

def test_zero_weight_kat():
    N, K = 16, 128
    packed = np.full(N * K // 2, 0x88, np.uint8)
    scales = np.full(N * K // 64, 0x3C00, np.uint16)  # fp16 1.0
    x = O.gen_act(2, K, 5)
    res = O.gen_act(2, N, 6)
    y, yf, _ = O.qlinear(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x)
    assert (y == 0).all() and (yf == 0).all()
    y, _, _ = O.qlinear(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, residual=res)
    np.testing.assert_array_equal(y, res)


@pytest.mark.parametrize("qtype", FORMATS)
@pytest.mark.parametrize("scale_enc", [O.SCALE_FP16, O.SCALE_BF16])
def test_combine_against_float64(qtype, scale_enc):
    N, K, M = 24, 512, 3
    packed, scales = O.gen_weights(qtype, N, K, 77, scale_enc)
    x = O.gen_act(M, K, 78)
    res = O.gen_act(M, N, 79)
    y, yf, ya = O.qlinear(qtype, packed, scales, scale_enc, N, K, x, residual=res)
    G = O.group_size(qtype)
    xq, xs = O.quantize_act(x, G)
    D = O.group_dots(qtype, packed, N, K, xq).astype(np.float64)
    if scale_enc == O.SCALE_FP16:
        ws = scales.view(np.float16).astype(np.float64)
    else:
        ws = O.bf16_to_f32(scales).astype(np.float64)
    ws = ws.reshape(N, K // G)
    exact = np.einsum("ng,mg,mng->mn", ws, xs.astype(np.float64), D) + O.bf16_to_f32(res)
    # fp32 sequential sum vs exact: bounded by ng * eps * sum|terms|
    assert (np.abs(yf - exact) <= (K // G + 2) * 2.0 ** -24 * ya).all()
    np.testing.assert_array_equal(y, O.f32_to_bf16(yf))
    # prequantized entry gives the identical result
    y2, yf2, _ = O.qlinear_prequant(qtype, packed, scales, scale_enc, N, K, xq, xs, residual=res)
    np.testing.assert_array_equal(yf2, yf)


def test_omp_matches_serial():
    N, K = 100, 640
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 3, O.SCALE_FP16)
    x = O.gen_act(2, K, 4)
    y, _, _ = O.qlinear(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x)
    np.testing.assert_array_equal(O.qlinear_omp(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, 4), y)


# ------------------------------------------------------------- generator

def test_generator_deterministic_and_in_range():
    for qtype in FORMATS:
        p1, s1 = O.gen_weights(qtype, 16, 256, 0x5EED0000, O.SCALE_FP16)
        p2, s2 = O.gen_weights(qtype, 16, 256, 0x5EED0000, O.SCALE_FP16)
        np.testing.assert_array_equal(p1, p2)
        np.testing.assert_array_equal(s1, s2)
        w = O.unpack(qtype, p1, 16, 256)
        lo, hi = O.wrange(qtype)
        assert w.min() == lo and w.max() == hi
        sf = s1.view(np.float16).astype(np.float32)
        assert sf.min() >= np.float32(np.float16(1e-3)) and sf.max() <= np.float32(np.float16(1e-2))
    x = O.bf16_to_f32(O.gen_act(64, 1024, 1))
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02
    xo = O.bf16_to_f32(O.gen_act(64, 1024, 1, outlier_frac=0.05, outlier_mul=20.0))
    frac = float((np.abs(xo - x) > 0).any(axis=0).mean())
    assert 0.03 < frac < 0.07


# ---- producers of the activation (rmsnorm, swiglu) before the quantize

def _bf16(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


def test_rmsnorm_closed_form_constant_row():
    # x = c everywhere, gamma = 1: every output is bf16(c / sqrt(c^2 + eps))
    H, eps = 2560, 1e-6
    for c in (0.5, -3.0, 1e-3, 7.25):
        x = np.tile(_bf16([c]), (1, H))
        out = O.rmsnorm_bf16(x, np.tile(_bf16([1.0]), H), eps)
        cf = float(O.bf16_to_f32(_bf16([c]))[0])
        want = _bf16([cf / np.sqrt(cf * cf + eps)])[0]
        assert (out == want).all(), (c, out[0, 0], want)


def test_rmsnorm_invariants_and_float64():
    rng = np.random.default_rng(3)
    M, H, eps = 3, 2560, 1e-5
    x = _bf16(rng.standard_normal((M, H)))
    gamma = _bf16(1.0 + 0.1 * rng.standard_normal(H))
    out = O.rmsnorm_bf16(x, gamma, eps)
    # scale invariance: x -> 4x with eps -> 16 eps scales ss/H + eps by 16 and
    # inv by 1/4, all exactly (powers of two), so every output is unchanged
    x4 = _bf16(O.bf16_to_f32(x) * 4.0)
    assert (O.rmsnorm_bf16(x4, gamma, eps * 16.0) == out).all()
    # gamma linearity: 2*gamma doubles every output exactly
    g2 = _bf16(O.bf16_to_f32(gamma) * 2.0)
    np.testing.assert_array_equal(O.bf16_to_f32(O.rmsnorm_bf16(x, g2, eps)), 2.0 * O.bf16_to_f32(out))
    # float64 restatement, within one bf16 ulp
    xf = O.bf16_to_f32(x).astype(np.float64)
    ref = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + eps) * O.bf16_to_f32(gamma)
    assert (np.abs(O.bf16_to_f32(out) - ref) <= O.bf16_ulp(out)).all()


def test_swiglu_known_values_and_float64():
    g = _bf16([0.0, 20.0, -20.0, 1.0, -1.0, 3.5])
    u = _bf16([5.0, 1.0, 1.0, 2.0, 2.0, -1.0])
    out = O.bf16_to_f32(O.swiglu_bf16(g[None, :], u[None, :]))[0]
    assert out[0] == 0.0                      # silu(0) = 0
    assert out[1] == 20.0                     # silu(20) = 20 to within bf16
    assert -1e-6 < out[2] < 0.0               # silu(-20) = -20 e^-20
    # silu(g) - silu(-g) = g
    assert abs((out[3] - out[4]) / 2.0 - 1.0) <= 2 * 2.0 ** -8
    rng = np.random.default_rng(4)
    G = _bf16(3.0 * rng.standard_normal((2, 4096)))
    U = _bf16(rng.standard_normal((2, 4096)))
    got = O.swiglu_bf16(G, U)
    gf, uf = O.bf16_to_f32(G).astype(np.float64), O.bf16_to_f32(U).astype(np.float64)
    ref = gf / (1.0 + np.exp(-gf)) * uf
    assert (np.abs(O.bf16_to_f32(got) - ref) <= O.bf16_ulp(got)).all()


# ---- bf16 GEMV (LM head) and greedy argmax

def test_linear_bf16_known_answers_and_float64():
    rng = np.random.default_rng(5)
    K = 2560
    x = _bf16(rng.standard_normal((2, K)))
    # unit rows pick one input each: y = x[k] exactly
    w = np.zeros((4, K), dtype=np.uint16)
    for n, k in enumerate((0, 7, 1000, K - 1)):
        w[n, k] = _bf16([1.0])[0]
    y, _, _ = O.linear_bf16(w, x)
    np.testing.assert_array_equal(y, x[:, [0, 7, 1000, K - 1]])
    # random: within the bf16 rounding of the float64 product
    W = _bf16(0.05 * rng.standard_normal((300, K)))
    y, yf, ya = O.linear_bf16(W, x)
    ref = O.bf16_to_f32(x).astype(np.float64) @ O.bf16_to_f32(W).astype(np.float64).T
    assert (np.abs(yf - ref) <= 1e-6 * ya + 1e-30).all()
    np.testing.assert_array_equal(y, O.f32_to_bf16(yf))


def test_argmax_ties_nan_inf():
    f = lambda v: _bf16(v)
    rows = np.stack([
        f([1.0, 3.0, 3.0, 2.0, -1.0]),              # tie: first index
        f([np.nan, 0.5, np.nan, 0.25, 0.5]),        # NaN never wins
        f([-np.inf] * 5),                           # nothing above -inf: 0
        f([-np.inf, -5.0, np.inf, np.inf, 0.0]),    # +inf, first occurrence
        f([-2.0, -1.0, -3.0, -1.0, -7.0]),
    ])
    np.testing.assert_array_equal(O.argmax_bf16(rows), [1, 1, 0, 2, 1])
    rng = np.random.default_rng(6)
    big = _bf16(rng.standard_normal((3, 166144)))
    np.testing.assert_array_equal(O.argmax_bf16(big), np.argmax(O.bf16_to_f32(big), axis=1))
