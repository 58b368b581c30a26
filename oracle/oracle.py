"""ctypes wrapper over the C oracle (liboracle.so).  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this module, and only as the checker.  The product path
(``viper_amd``) never imports it.

Reference semantics restated by each wrapped C function are listed in
``oracle/viper_oracle.h``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_convert.so")

Q4_G64, Q5_G64, Q6_G64, W8_G32 = 4, 5, 6, 8
QTYPES = (Q4_G64, Q5_G64, Q6_G64, W8_G32)
SCALE_FP16, SCALE_BF16 = 0, 1

_lib = None
_ref = None


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, u64, sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_size_t
        L.vo_bf16_to_f32.argtypes, L.vo_bf16_to_f32.restype = [C.c_uint16], C.c_float
        L.vo_f32_to_bf16.argtypes, L.vo_f32_to_bf16.restype = [C.c_float], C.c_uint16
        L.vo_f16_to_f32.argtypes, L.vo_f16_to_f32.restype = [C.c_uint16], C.c_float
        L.vo_f32_to_f16.argtypes, L.vo_f32_to_f16.restype = [C.c_float], C.c_uint16
        L.vo_group_size.argtypes, L.vo_group_size.restype = [i32], i32
        L.vo_wmin.argtypes, L.vo_wmin.restype = [i32], i32
        L.vo_wmax.argtypes, L.vo_wmax.restype = [i32], i32
        L.vo_packed_bytes.argtypes, L.vo_packed_bytes.restype = [i32, i64, i64], sz
        L.vo_pack.argtypes, L.vo_pack.restype = [i32, vp, i32, i32, vp], i32
        L.vo_unpack.argtypes, L.vo_unpack.restype = [i32, vp, i32, i32, vp], i32
        L.vo_gen_weights.argtypes = [i32, i32, i32, u64, i32, vp, vp]
        L.vo_gen_weights.restype = i32
        L.vo_gen_act.argtypes, L.vo_gen_act.restype = [i32, i32, u64, C.c_double, C.c_float, vp], None
        L.vo_quantize_weights.argtypes = [i32, vp, i32, i32, i32, vp, vp]
        L.vo_quantize_weights.restype = i32
        L.vo_quantize_act.argtypes, L.vo_quantize_act.restype = [vp, i32, i32, i32, vp, vp], i32
        L.vo_rmsnorm_bf16.argtypes, L.vo_rmsnorm_bf16.restype = [vp, vp, C.c_float, i32, i32, vp], i32
        L.vo_swiglu_bf16.argtypes, L.vo_swiglu_bf16.restype = [vp, vp, i32, i32, vp], i32
        L.vo_linear_bf16.argtypes, L.vo_linear_bf16.restype = [vp, vp, i32, i32, i32, vp, vp, vp], i32
        L.vo_argmax_bf16.argtypes, L.vo_argmax_bf16.restype = [vp, i32, i32, vp], i32
        L.vo_group_dots.argtypes, L.vo_group_dots.restype = [i32, vp, i32, i32, vp, i32, vp], i32
        L.vo_qlinear_prequant.argtypes = [i32, vp, vp, i32, i32, i32, vp, vp, i32, vp, vp, vp, vp]
        L.vo_qlinear_prequant.restype = i32
        L.vo_qlinear.argtypes = [i32, vp, vp, i32, i32, i32, vp, i32, vp, vp, vp, vp]
        L.vo_qlinear.restype = i32
        L.vo_qlinear_omp.argtypes = [i32, vp, vp, i32, i32, i32, vp, i32, vp, vp, vp, vp, i32]
        L.vo_qlinear_omp.restype = i32
        L.vo_omp_max_threads.argtypes, L.vo_omp_max_threads.restype = [], i32
        L.vo_check_markstein.argtypes = [i32, i32, C.POINTER(C.c_int64)]
        L.vo_check_markstein.restype = C.c_int64
        _lib = L
    return _lib


def ref_lib():
    """The reference converter's own quantizer, or None when it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        R = C.CDLL(REF_LIB_PATH)
        R.ref_quantize_q4_g64.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        R.ref_quantize_q4_g64.restype = C.c_int
        _ref = R
    return _ref


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with {rc}")


def group_size(qtype):
    return lib().vo_group_size(qtype)


def wrange(qtype):
    return lib().vo_wmin(qtype), lib().vo_wmax(qtype)


def packed_bytes(qtype, N, K):
    return lib().vo_packed_bytes(qtype, N, K)


def pack(qtype, w):
    w = np.ascontiguousarray(w, dtype=np.int8)
    N, K = w.shape
    out = np.zeros(packed_bytes(qtype, N, K), dtype=np.uint8)
    _check(lib().vo_pack(qtype, _p(w), N, K, _p(out)), "pack")
    return out


def unpack(qtype, packed, N, K):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    w = np.zeros((N, K), dtype=np.int8)
    _check(lib().vo_unpack(qtype, _p(packed), N, K, _p(w)), "unpack")
    return w


def gen_weights(qtype, N, K, seed, scale_enc=SCALE_FP16):
    G = group_size(qtype)
    packed = np.zeros(packed_bytes(qtype, N, K), dtype=np.uint8)
    scales = np.zeros(N * (K // G), dtype=np.uint16)
    _check(lib().vo_gen_weights(qtype, N, K, seed, scale_enc, _p(packed), _p(scales)), "gen_weights")
    return packed, scales


def gen_act(M, K, seed, outlier_frac=0.0, outlier_mul=20.0):
    x = np.zeros((M, K), dtype=np.uint16)
    lib().vo_gen_act(M, K, seed, outlier_frac, outlier_mul, _p(x))
    return x


def quantize_weights(qtype, w_bf16, scale_enc=SCALE_BF16):
    w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    N, K = w_bf16.shape
    G = group_size(qtype)
    packed = np.zeros(packed_bytes(qtype, N, K), dtype=np.uint8)
    scales = np.zeros(N * (K // G), dtype=np.uint16)
    _check(lib().vo_quantize_weights(qtype, _p(w_bf16), N, K, scale_enc, _p(packed), _p(scales)),
           "quantize_weights")
    return packed, scales


def ref_quantize_q4_g64(w_bf16):
    R = ref_lib()
    if R is None:
        return None
    w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    N, K = w_bf16.shape
    packed = np.zeros(N * K // 2, dtype=np.uint8)
    scales = np.zeros(N * (K // 64), dtype=np.uint16)
    _check(R.ref_quantize_q4_g64(_p(w_bf16), N, K, _p(packed), _p(scales)), "ref_quantize_q4_g64")
    return packed, scales


def quantize_act(x_bf16, group):
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M, K = x_bf16.shape
    xq = np.zeros((M, K), dtype=np.int8)
    xs = np.zeros((M, K // group), dtype=np.float32)
    _check(lib().vo_quantize_act(_p(x_bf16), M, K, group, _p(xq), _p(xs)), "quantize_act")
    return xq, xs


def rmsnorm_bf16(x_bf16, gamma_bf16, eps):
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M, H = x_bf16.shape
    gamma = np.ascontiguousarray(gamma_bf16, dtype=np.uint16)
    out = np.zeros((M, H), dtype=np.uint16)
    _check(lib().vo_rmsnorm_bf16(_p(x_bf16), _p(gamma), C.c_float(eps), M, H, _p(out)), "rmsnorm_bf16")
    return out


def swiglu_bf16(gate_bf16, up_bf16):
    gate = np.ascontiguousarray(gate_bf16, dtype=np.uint16)
    up = np.ascontiguousarray(up_bf16, dtype=np.uint16)
    M, I = gate.shape
    out = np.zeros((M, I), dtype=np.uint16)
    _check(lib().vo_swiglu_bf16(_p(gate), _p(up), M, I, _p(out)), "swiglu_bf16")
    return out


def linear_bf16(w_bf16, x_bf16):
    """(y_bf16 [M,N], y_f32, absterm) of x [M,K] times w [N,K]^T, all bf16 in."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    N, K = w.shape
    M = x.shape[0]
    y = np.zeros((M, N), dtype=np.uint16)
    yf = np.zeros((M, N), dtype=np.float32)
    ya = np.zeros((M, N), dtype=np.float64)
    _check(lib().vo_linear_bf16(_p(w), _p(x), M, N, K, _p(y), _p(yf), _p(ya)), "linear_bf16")
    return y, yf, ya


def argmax_bf16(logits_bf16):
    lg = np.ascontiguousarray(logits_bf16, dtype=np.uint16)
    B, V = lg.shape
    out = np.zeros(B, dtype=np.int32)
    _check(lib().vo_argmax_bf16(_p(lg), B, V, _p(out)), "argmax_bf16")
    return out


def group_dots(qtype, packed, N, K, xq):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    M = xq.shape[0]
    G = group_size(qtype)
    D = np.zeros((M, N, K // G), dtype=np.int32)
    _check(lib().vo_group_dots(qtype, _p(np.ascontiguousarray(packed)), N, K, _p(xq), M, _p(D)),
           "group_dots")
    return D


def qlinear(qtype, packed, scales, scale_enc, N, K, x_bf16, residual=None):
    """Returns (y_bf16 [M,N] uint16, y_f32 [M,N], absterm [M,N] float64)."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M = x_bf16.shape[0]
    y = np.zeros((M, N), dtype=np.uint16)
    yf = np.zeros((M, N), dtype=np.float32)
    ya = np.zeros((M, N), dtype=np.float64)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.uint16)
    _check(lib().vo_qlinear(qtype, _p(np.ascontiguousarray(packed)), _p(np.ascontiguousarray(scales)),
                            scale_enc, N, K, _p(x_bf16), M, _p(res), _p(y), _p(yf), _p(ya)), "qlinear")
    return y, yf, ya


def qlinear_prequant(qtype, packed, scales, scale_enc, N, K, xq, xs, residual=None):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    M = xq.shape[0]
    y = np.zeros((M, N), dtype=np.uint16)
    yf = np.zeros((M, N), dtype=np.float32)
    ya = np.zeros((M, N), dtype=np.float64)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.uint16)
    _check(lib().vo_qlinear_prequant(qtype, _p(np.ascontiguousarray(packed)),
                                     _p(np.ascontiguousarray(scales)), scale_enc, N, K, _p(xq), _p(xs),
                                     M, _p(res), _p(y), _p(yf), _p(ya)), "qlinear_prequant")
    return y, yf, ya


def qlinear_omp(qtype, packed, scales, scale_enc, N, K, x_bf16, nthreads=0, residual=None, full=False):
    """qlinear over OpenMP threads: y_bf16, or (y_bf16, y_f32, absterm) with full=True."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M = x_bf16.shape[0]
    y = np.zeros((M, N), dtype=np.uint16)
    yf = np.zeros((M, N), dtype=np.float32) if full else None
    ya = np.zeros((M, N), dtype=np.float64) if full else None
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.uint16)
    _check(lib().vo_qlinear_omp(qtype, _p(np.ascontiguousarray(packed)), _p(np.ascontiguousarray(scales)),
                                scale_enc, N, K, _p(x_bf16), M, _p(res), _p(y), _p(yf), _p(ya), nthreads),
           "qlinear_omp")
    return (y, yf, ya) if full else y


def omp_max_threads():
    return lib().vo_omp_max_threads()


def check_markstein(exp_lo=0, exp_hi=254):
    n = C.c_int64(0)
    bad = lib().vo_check_markstein(exp_lo, exp_hi, C.byref(n))
    return bad, n.value


# ---- numpy helpers shared by the tests -------------------------------------

def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_ulp(h):
    """Spacing of bf16 numbers at |value of h| (finite inputs)."""
    f = np.abs(bf16_to_f32(h)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(f, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_bf16_close(y_gpu, y_ref, absterm, rel=1e-5, what="y"):
    """Pass when each output is within 1 bf16 ulp of the oracle's bf16 output,
    or within rel * sum|terms| of it (condition-aware bound)."""
    yg = bf16_to_f32(y_gpu).astype(np.float64)
    yr = bf16_to_f32(y_ref).astype(np.float64)
    diff = np.abs(yg - yr)
    ulp = np.maximum(bf16_ulp(y_ref), bf16_ulp(y_gpu))
    ok = (diff <= ulp) | (diff <= rel * np.asarray(absterm, dtype=np.float64))
    if not ok.all():
        idx = np.argwhere(~ok)[:5]
        raise AssertionError(
            f"{what}: {int((~ok).sum())} of {ok.size} outputs outside tolerance; first at "
            f"{idx.tolist()}: gpu={yg[tuple(idx[0])]} ref={yr[tuple(idx[0])]} "
            f"absterm={np.asarray(absterm)[tuple(idx[0])]}")
