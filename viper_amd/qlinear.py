"""ctypes binding of the gfx950 quantized-linear C ABI (include/viper_qlinear.h).

Torch is plumbing here: tensors provide device memory and the stream; every
compute call goes through ``libviper_qlinear.so``.  There is no fallback path:
a missing library raises at load time.

The Python surface mirrors the reference's host API (itzrnvr/viper):
``QuantizedWeight`` is ``viper::quant::QuantizedWeight`` (include/viper/quant.h:34-41)
plus the explicit scale encoding, ``QType``/``qtype_name``/``is_lossless`` are the
closed registry (quant.h:19-29, src/viper/quant.cpp:6-20), and ``linear`` returns a
``Status`` instead of raising, as ``viper::ops::linear_forward`` does
(include/viper/ops.h:30-33, src/viper/linear.cpp:16-36).
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libviper_qlinear.so")
HOST_LIB_PATH = os.path.join(HERE, "lib", "libviper.so")


class StatusCode(enum.IntEnum):
    """Numbering of viper::StatusCode (include/viper/status.h:12-21)."""
    OK = 0
    UNIMPLEMENTED = 1
    INVALID_ARGUMENT = 2
    CUDA_ERROR = 3  # device error
    SHAPE_MISMATCH = 4
    OUT_OF_MEMORY = 5
    IO_ERROR = 6
    INTERNAL = 99


@dataclass(frozen=True)
class Status:
    code: StatusCode = StatusCode.OK
    message: str = ""

    def ok(self) -> bool:
        return self.code == StatusCode.OK

    def __bool__(self) -> bool:
        return self.ok()


class QType(enum.IntEnum):
    """Closed weight-format registry (include/viper/quant.h:19-26)."""
    BF16 = 0
    FP32 = 1
    Q4_G64 = 4
    Q5_G64 = 5
    Q6_G64 = 6
    W8_G32 = 8


class ScaleEnc(enum.IntEnum):
    FP16 = 0
    BF16 = 1


def qtype_name(q) -> str:
    """src/viper/quant.cpp:6-16."""
    try:
        return QType(int(q)).name
    except ValueError:
        return "UNKNOWN"


def is_lossless(q) -> bool:
    """src/viper/quant.cpp:18-20."""
    return int(q) in (QType.BF16, QType.FP32)


GROUP = {QType.Q4_G64: 64, QType.Q5_G64: 64, QType.Q6_G64: 64, QType.W8_G32: 32}
MAX_M = 16


def packed_bytes(qtype, rows, cols) -> int:
    q = QType(int(qtype))
    if q == QType.Q4_G64:
        return rows * cols // 2
    if q == QType.Q5_G64:
        return rows * cols // 2 + rows * cols // 8
    if q == QType.Q6_G64:
        return rows * cols // 2 + rows * cols // 4
    if q == QType.W8_G32:
        return rows * cols
    raise ValueError(f"not a quantized qtype: {qtype_name(q)}")


@dataclass
class QuantizedWeight:
    """Device view of one quantized matrix (reference quant.h:34-41).

    ``data`` and ``scales`` are torch tensors on the device (uint8 / int16 or
    uint16-sized storage); ``rows`` = N output channels, ``cols`` = K inputs.
    """
    qtype: QType
    data: object
    scales: object
    rows: int
    cols: int
    group_size: int = 64
    scale_enc: ScaleEnc = ScaleEnc.BF16


_lib = None

_SYMBOLS = (
    "viper_hip_abi_version",
    "viper_hip_group_size",
    "viper_hip_qlinear_workspace_bytes",
    "viper_hip_qlinear_workspace_layout",
    "viper_hip_qlinear",
    "viper_hip_quantize_act",
    "viper_hip_qlinear_prequantized",
    "viper_hip_qlinear_partials",
    "viper_hip_check_quantizer",
    "viper_hip_stream_read",
    "viper_hip_qlinear_fused2",
    "viper_hip_qlinear_fused2_prequantized",
    "viper_hip_rmsnorm_quantize",
    "viper_hip_swiglu_quantize",
    "viper_hip_linear_bf16",
    "viper_hip_sampling_greedy",
    "viper_hip_sampling_greedy_workspace_bytes",
    "viper_hip_sampling_greedy_split",
    "viper_hip_qlinear_m1",
    "viper_hip_qlinear_m1_swiglu",
    "viper_hip_qlinear_static",
    "viper_hip_qlinear_timeline",
    "viper_hip_check_bf16_rounding",
    "viper_hip_clock_stamp",
    "viper_hip_empty_dispatch",
    "viper_hip_prefetch",
    "viper_hip_rmsnorm_quantize_frag",
    "viper_hip_swiglu_quantize_frag",
    "viper_hip_qlinear_prequantized_frag",
    "viper_hip_qlinear_frag_workspace_bytes",
    "viper_hip_qlinear_fused2_prequantized_frag",
    "viper_hip_qlinear_frag_timeline",
)


def lib():
    """Load libviper_qlinear.so; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"viper_amd HIP library missing: {LIB_PATH}. Build it with __graft_entry__.build(); "
            "there is no CPU fallback.")
    L = C.CDLL(LIB_PATH)
    vp, i32, sz = C.c_void_p, C.c_int, C.c_size_t
    L.viper_hip_abi_version.argtypes, L.viper_hip_abi_version.restype = [], i32
    L.viper_hip_group_size.argtypes, L.viper_hip_group_size.restype = [i32], i32
    L.viper_hip_qlinear_workspace_bytes.argtypes = [i32, i32, i32, i32]
    L.viper_hip_qlinear_workspace_bytes.restype = sz
    L.viper_hip_qlinear_workspace_layout.argtypes = [i32, i32, i32, i32, vp]
    L.viper_hip_qlinear_workspace_layout.restype = sz
    L.viper_hip_qlinear.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, i32, vp, vp, vp, sz, vp]
    L.viper_hip_qlinear.restype = i32
    L.viper_hip_quantize_act.argtypes = [i32, vp, i32, i32, vp, vp, vp]
    L.viper_hip_quantize_act.restype = i32
    L.viper_hip_qlinear_prequantized.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, vp, i32, vp, vp, vp]
    L.viper_hip_qlinear_prequantized.restype = i32
    L.viper_hip_qlinear_partials.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, i32, vp, vp, vp, sz, vp, vp]
    L.viper_hip_qlinear_partials.restype = i32
    L.viper_hip_qlinear_static.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, i32, vp, vp, vp]
    L.viper_hip_qlinear_static.restype = i32
    L.viper_hip_qlinear_timeline.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, vp, vp, sz, vp, vp, vp]
    L.viper_hip_qlinear_timeline.restype = i32
    L.viper_hip_check_bf16_rounding.argtypes = [vp, vp]
    L.viper_hip_check_bf16_rounding.restype = i32
    L.viper_hip_check_quantizer.argtypes = [i32, i32, vp, vp]
    L.viper_hip_check_quantizer.restype = i32
    L.viper_hip_stream_read.argtypes = [vp, sz, i32, i32, vp, i32, vp, vp, vp]
    L.viper_hip_stream_read.restype = i32
    L.viper_hip_clock_stamp.argtypes = [vp, vp]
    L.viper_hip_clock_stamp.restype = i32
    L.viper_hip_empty_dispatch.argtypes = [i32, i32, vp, vp]
    L.viper_hip_empty_dispatch.restype = i32
    L.viper_hip_prefetch.argtypes = [vp, sz, i32, vp, vp]
    L.viper_hip_prefetch.restype = i32
    L.viper_hip_rmsnorm_quantize_frag.argtypes = [vp, vp, C.c_float, i32, i32, i32, vp, vp, vp, vp]
    L.viper_hip_rmsnorm_quantize_frag.restype = i32
    L.viper_hip_swiglu_quantize_frag.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp]
    L.viper_hip_swiglu_quantize_frag.restype = i32
    L.viper_hip_qlinear_prequantized_frag.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, vp, i32, vp, vp, vp, sz,
                                                      vp]
    L.viper_hip_qlinear_prequantized_frag.restype = i32
    L.viper_hip_qlinear_frag_workspace_bytes.argtypes = [i32, i32, i32, i32]
    L.viper_hip_qlinear_frag_workspace_bytes.restype = sz
    L.viper_hip_qlinear_fused2_prequantized_frag.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, i32,
                                                             vp, vp, vp]
    L.viper_hip_qlinear_fused2_prequantized_frag.restype = i32
    L.viper_hip_qlinear_frag_timeline.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, vp, i32, vp, vp, sz, vp, vp,
                                                  vp, sz, vp]
    L.viper_hip_qlinear_frag_timeline.restype = i32
    L.viper_hip_qlinear_fused2.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, vp, vp, vp, sz, vp]
    L.viper_hip_qlinear_fused2.restype = i32
    L.viper_hip_qlinear_fused2_prequantized.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, i32,
                                                        vp, vp, vp]
    L.viper_hip_qlinear_fused2_prequantized.restype = i32
    L.viper_hip_rmsnorm_quantize.argtypes = [vp, vp, C.c_float, i32, i32, i32, vp, vp, vp, vp]
    L.viper_hip_rmsnorm_quantize.restype = i32
    L.viper_hip_swiglu_quantize.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp]
    L.viper_hip_swiglu_quantize.restype = i32
    L.viper_hip_linear_bf16.argtypes = [vp, vp, vp, i32, i32, i32, vp]
    L.viper_hip_linear_bf16.restype = i32
    L.viper_hip_sampling_greedy.argtypes = [vp, vp, i32, i32, vp]
    L.viper_hip_sampling_greedy.restype = i32
    L.viper_hip_sampling_greedy_workspace_bytes.argtypes = [i32]
    L.viper_hip_sampling_greedy_workspace_bytes.restype = sz
    L.viper_hip_sampling_greedy_split.argtypes = [vp, vp, i32, i32, vp, sz, vp]
    L.viper_hip_sampling_greedy_split.restype = i32
    L.viper_hip_qlinear_m1.argtypes = [i32, i32, i32, i32, i32, vp, vp, C.c_float, vp, i32, vp, vp, vp, vp, vp, vp]
    L.viper_hip_qlinear_m1.restype = i32
    L.viper_hip_qlinear_m1_swiglu.argtypes = [i32, i32, i32, i32, i32, vp, vp, C.c_float, vp, vp, vp, vp, vp, i32,
                                              vp, vp, vp, vp]
    L.viper_hip_qlinear_m1_swiglu.restype = i32
    _lib = L
    return L


def ptr(t, itemsize: Optional[int] = None) -> Optional[int]:
    """Device address of a torch tensor (None stays None).  The kernels read and write every tensor as a
    dense array of fixed-size elements in device memory, so a CPU tensor (a host address on the GPU), a
    non-contiguous view (read as if dense) or elements of another size than the argument's (itemsize:
    1 for packed weights and int8 activations, 2 for bf16 data and 16-bit scales, 4 for fp32 scales and
    int32 outputs) raise ValueError instead of reaching the C ABI."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("viper_amd: tensor arguments must be GPU tensors")
    if not t.is_contiguous():
        raise ValueError("viper_amd: tensor arguments must be contiguous")
    if itemsize is not None and t.element_size() != itemsize:
        raise ValueError(f"viper_amd: expected {itemsize}-byte elements, got {t.dtype}")
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _status(rc: int, what: str) -> Status:
    if rc == 0:
        return Status()
    try:
        code = StatusCode(rc)
    except ValueError:
        code = StatusCode.INTERNAL
    return Status(code, f"{what}: {code.name}")


def workspace_bytes(qtype, N, K, M) -> int:
    """Bytes of the M > 1 workspace (zero-filled before its first use); 0 at M = 1."""
    return int(lib().viper_hip_qlinear_workspace_bytes(int(qtype), N, K, M))


WS_PARTS = ("missed", "counters", "sums", "xq", "xs", "split_blocks")


def workspace_layout(qtype, N, K, M) -> dict:
    """Byte offsets of the workspace's parts for this shape (None where the shape has none) and its
    total size: the K split's missed-sum count (offset 4) and block counters (from 256) for every M > 1
    shape, the K split's records of part sums (from 4352), xq and xs; split_blocks is the K split's
    count of row blocks (0 without it)."""
    off = (C.c_size_t * 6)()
    total = int(lib().viper_hip_qlinear_workspace_layout(int(qtype), N, K, M, C.cast(off, C.c_void_p)))
    none = (1 << (8 * C.sizeof(C.c_size_t))) - 1
    out = {k: (None if int(v) == none else int(v)) for k, v in zip(WS_PARTS, off)}
    out["total"] = total
    return out


def frag_workspace_bytes(qtype, N, K, M) -> int:
    """Bytes of workspace the fragment-input entry splits long K with (0: the shape needs none)."""
    return int(lib().viper_hip_qlinear_frag_workspace_bytes(int(qtype), N, K, M))


def qlinear_raw(qtype, w, s, scale_enc, group, N, K, x, M, y, residual=None, workspace=None,
                workspace_nbytes=0, stream=None) -> int:
    """Direct call of viper_hip_qlinear with device addresses (ints)."""
    return lib().viper_hip_qlinear(int(qtype), w, s, int(scale_enc), group, N, K, x, M, y, residual,
                                   workspace, workspace_nbytes, _stream(stream))


def _shape_mk(x, K):
    if x.dim() == 1:
        return 1
    return int(x.numel() // K)


def linear(w: QuantizedWeight, x, y, residual=None, workspace=None, stream=None) -> Status:
    """y[M, N] = x[M, K] (bf16) through the quantized weight w; returns Status."""
    if is_lossless(w.qtype):
        return Status(StatusCode.UNIMPLEMENTED, f"linear {qtype_name(w.qtype)}: not on this path")
    if int(w.qtype) not in GROUP:
        return Status(StatusCode.INVALID_ARGUMENT, "linear: bad weight qtype")
    K, N = w.cols, w.rows
    if x.numel() % K or y.numel() % N:
        return Status(StatusCode.SHAPE_MISMATCH, "linear: x/y do not match the weight shape")
    M = _shape_mk(x, K)
    if y.numel() != M * N:
        return Status(StatusCode.SHAPE_MISMATCH, "linear: y rows != x rows")
    if residual is not None and residual.numel() != M * N:
        return Status(StatusCode.SHAPE_MISMATCH, "linear: residual shape")
    ws_ptr, ws_n = (None, 0) if workspace is None else (ptr(workspace), workspace.numel() * workspace.element_size())
    rc = lib().viper_hip_qlinear(int(w.qtype), ptr(w.data, 1), ptr(w.scales, 2), int(w.scale_enc), w.group_size,
                                 N, K, ptr(x, 2), M, ptr(y, 2), ptr(residual, 2), ws_ptr, ws_n, _stream(stream))
    return _status(rc, "viper_hip_qlinear")


def linear_partials(w: QuantizedWeight, x, y, partials, residual=None, workspace=None, stream=None) -> Status:
    K, N = w.cols, w.rows
    M = _shape_mk(x, K)
    ws_ptr, ws_n = (None, 0) if workspace is None else (ptr(workspace), workspace.numel() * workspace.element_size())
    rc = lib().viper_hip_qlinear_partials(int(w.qtype), ptr(w.data, 1), ptr(w.scales, 2), int(w.scale_enc),
                                          w.group_size, N, K, ptr(x, 2), M, ptr(y, 2), ptr(residual, 2), ws_ptr, ws_n,
                                          ptr(partials, 4), _stream(stream))
    return _status(rc, "viper_hip_qlinear_partials")


def quantize_act(x, group, xq, xs, stream=None) -> Status:
    K = xq.shape[-1]
    M = int(xq.numel() // K)
    rc = lib().viper_hip_quantize_act(group, ptr(x, 2), M, K, ptr(xq, 1), ptr(xs, 4), _stream(stream))
    return _status(rc, "viper_hip_quantize_act")


def linear_prequantized(w: QuantizedWeight, xq, xs, y, residual=None, stream=None) -> Status:
    K, N = w.cols, w.rows
    M = int(xq.numel() // K)
    rc = lib().viper_hip_qlinear_prequantized(int(w.qtype), ptr(w.data, 1), ptr(w.scales, 2), int(w.scale_enc),
                                              w.group_size, N, K, ptr(xq, 1), ptr(xs, 4), M, ptr(y, 2), ptr(residual, 2),
                                              _stream(stream))
    return _status(rc, "viper_hip_qlinear_prequantized")


def _same_kind(w0: QuantizedWeight, w1: QuantizedWeight) -> bool:
    return (w0.qtype, w0.rows, w0.cols, w0.group_size, w0.scale_enc) == \
        (w1.qtype, w1.rows, w1.cols, w1.group_size, w1.scale_enc)


def linear_fused2(w0: QuantizedWeight, w1: QuantizedWeight, x, y0, y1, workspace=None, stream=None) -> Status:
    """y0 = x w0 and y1 = x w1 in one launch (two matrices of one shape)."""
    if not _same_kind(w0, w1):
        return Status(StatusCode.SHAPE_MISMATCH, "linear_fused2: the two weights differ in kind or shape")
    K, N = w0.cols, w0.rows
    M = _shape_mk(x, K)
    ws_ptr, ws_n = (None, 0) if workspace is None else (ptr(workspace), workspace.numel() * workspace.element_size())
    rc = lib().viper_hip_qlinear_fused2(int(w0.qtype), ptr(w0.data, 1), ptr(w0.scales, 2), ptr(w1.data, 1), ptr(w1.scales, 2),
                                        int(w0.scale_enc), w0.group_size, N, K, ptr(x, 2), M, ptr(y0, 2), ptr(y1, 2),
                                        ws_ptr, ws_n, _stream(stream))
    return _status(rc, "viper_hip_qlinear_fused2")


def linear_fused2_prequantized(w0: QuantizedWeight, w1: QuantizedWeight, xq, xs, y0, y1, stream=None) -> Status:
    if not _same_kind(w0, w1):
        return Status(StatusCode.SHAPE_MISMATCH, "linear_fused2: the two weights differ in kind or shape")
    K, N = w0.cols, w0.rows
    M = int(xq.numel() // K)
    rc = lib().viper_hip_qlinear_fused2_prequantized(int(w0.qtype), ptr(w0.data, 1), ptr(w0.scales, 2), ptr(w1.data, 1),
                                                     ptr(w1.scales, 2), int(w0.scale_enc), w0.group_size, N, K,
                                                     ptr(xq, 1), ptr(xs, 4), M, ptr(y0, 2), ptr(y1, 2), _stream(stream))
    return _status(rc, "viper_hip_qlinear_fused2_prequantized")


def rmsnorm_quantize(x, gamma, eps, group, xq, xs, out=None, stream=None) -> Status:
    """xq/xs (and out, bf16) from rmsnorm(x) * gamma, per row of x [M, H]."""
    H = gamma.numel()
    M = int(x.numel() // H)
    rc = lib().viper_hip_rmsnorm_quantize(ptr(x, 2), ptr(gamma, 2), float(eps), M, H, group, ptr(out, 2), ptr(xq, 1),
                                          ptr(xs, 4), _stream(stream))
    return _status(rc, "viper_hip_rmsnorm_quantize")


def swiglu_quantize(gate, up, group, xq, xs, out=None, stream=None) -> Status:
    """xq/xs (and out, bf16; may be gate itself) from silu(gate) * up, rows of [M, I]."""
    I = gate.shape[-1]
    M = int(gate.numel() // I)
    rc = lib().viper_hip_swiglu_quantize(ptr(gate, 2), ptr(up, 2), M, I, group, ptr(out, 2), ptr(xq, 1), ptr(xs, 4),
                                         _stream(stream))
    return _status(rc, "viper_hip_swiglu_quantize")


def frag_bytes(K: int, group: int):
    """Bytes of the fragment-order activation buffers for up to 16 rows: (xfrag, xsfrag)."""
    return K * 16, (K // group) * 16 * 4


def rmsnorm_quantize_frag(x, gamma, eps, group, xfrag, xsfrag, out=None, stream=None) -> Status:
    """rmsnorm_quantize for M <= 16 rows of x [M, H], the int8 rows and scales in fragment order."""
    H = gamma.numel()
    M = int(x.numel() // H)
    rc = lib().viper_hip_rmsnorm_quantize_frag(ptr(x, 2), ptr(gamma, 2), float(eps), M, H, group, ptr(out, 2),
                                               ptr(xfrag, 1), ptr(xsfrag, 4), _stream(stream))
    return _status(rc, "viper_hip_rmsnorm_quantize_frag")


def swiglu_quantize_frag(gate, up, group, xfrag, xsfrag, out=None, stream=None) -> Status:
    """swiglu_quantize for M <= 16 rows of [M, I], the int8 rows and scales in fragment order."""
    I = gate.shape[-1]
    M = int(gate.numel() // I)
    rc = lib().viper_hip_swiglu_quantize_frag(ptr(gate, 2), ptr(up, 2), M, I, group, ptr(out, 2), ptr(xfrag, 1),
                                              ptr(xsfrag, 4), _stream(stream))
    return _status(rc, "viper_hip_swiglu_quantize_frag")


def linear_prequantized_frag(w: QuantizedWeight, xfrag, xsfrag, y, residual=None, workspace=None,
                             stream=None) -> Status:
    """y [M, N] (M = 2..16) from int8 rows in fragment order (rmsnorm/swiglu_quantize_frag); with a
    workspace of frag_workspace_bytes (zero-filled before its first use) long K splits over workgroups."""
    K, N = w.cols, w.rows
    M = int(y.numel() // N)
    nws = 0 if workspace is None else int(workspace.numel() * workspace.element_size())
    rc = lib().viper_hip_qlinear_prequantized_frag(int(w.qtype), ptr(w.data, 1), ptr(w.scales, 2), int(w.scale_enc),
                                                   w.group_size, N, K, ptr(xfrag, 1), ptr(xsfrag, 4), M, ptr(y, 2),
                                                   ptr(residual, 2), ptr(workspace, 1), nws, _stream(stream))
    return _status(rc, "viper_hip_qlinear_prequantized_frag")


def linear_fused2_prequantized_frag(w0: QuantizedWeight, w1: QuantizedWeight, xfrag, xsfrag, y0, y1,
                                    stream=None) -> Status:
    if not _same_kind(w0, w1):
        return Status(StatusCode.SHAPE_MISMATCH, "linear_fused2: the two weights differ in kind or shape")
    K, N = w0.cols, w0.rows
    M = int(y0.numel() // N)
    rc = lib().viper_hip_qlinear_fused2_prequantized_frag(int(w0.qtype), ptr(w0.data, 1), ptr(w0.scales, 2),
                                                          ptr(w1.data, 1), ptr(w1.scales, 2), int(w0.scale_enc),
                                                          w0.group_size, N, K, ptr(xfrag, 1), ptr(xsfrag, 4), M,
                                                          ptr(y0, 2), ptr(y1, 2), _stream(stream))
    return _status(rc, "viper_hip_qlinear_fused2_prequantized_frag")


class Prologue(enum.IntEnum):
    BF16 = 0
    INT8 = 1
    RMSNORM = 2
    SWIGLU = 3


def linear_m1(ws, prologue, a, b, ys, eps=0.0, norm_out=None, residual=None, stream=None) -> Status:
    """One launch at M = 1: ys[i] = linear(ws[i], v) for 1..3 weights of one kind and K,
    v produced by the prologue from a (and b): bf16 x; int8 xq + fp32 xs;
    rmsnorm(x) * gamma; silu(gate) * up.  residual is added to ys[0]."""
    n = len(ws)
    if n < 1 or n > 3 or len(ys) != n:
        return Status(StatusCode.INVALID_ARGUMENT, "linear_m1: 1 to 3 weights, one output each")
    w0 = ws[0]
    if any((w.qtype, w.cols, w.group_size, w.scale_enc) != (w0.qtype, w0.cols, w0.group_size, w0.scale_enc)
           for w in ws):
        return Status(StatusCode.SHAPE_MISMATCH, "linear_m1: weights differ in kind or K")
    arr = lambda vals: (C.c_void_p * n)(*vals)
    rc = lib().viper_hip_qlinear_m1(int(w0.qtype), int(w0.scale_enc), w0.group_size, w0.cols, int(prologue),
                                    ptr(a, 1 if int(prologue) == int(Prologue.INT8) else 2), ptr(b, 4 if int(prologue) == int(Prologue.INT8) else 2), float(eps), ptr(norm_out, 2), n,
                                    arr([ptr(w.data, 1) for w in ws]), arr([ptr(w.scales, 2) for w in ws]),
                                    (C.c_int * n)(*[w.rows for w in ws]), arr([ptr(y, 2) for y in ys]),
                                    ptr(residual, 2), _stream(stream))
    return _status(rc, "viper_hip_qlinear_m1")


def linear_m1_swiglu(w_gate, w_up, prologue, a, b, h, eps=0.0, norm_out=None, gate_out=None, up_out=None,
                     stream=None) -> Status:
    """One launch at M = 1: g = linear(w_gate, v), u = linear(w_up, v) and h = bf16(silu(g) * u) from the
    bf16-rounded g and u; v from the BF16 or RMSNORM prologue as in linear_m1.  gate_out / up_out
    (optional) receive g and u."""
    if (w_gate.qtype, w_gate.rows, w_gate.cols, w_gate.group_size, w_gate.scale_enc) != \
            (w_up.qtype, w_up.rows, w_up.cols, w_up.group_size, w_up.scale_enc):
        return Status(StatusCode.SHAPE_MISMATCH, "linear_m1_swiglu: gate and up differ in kind or shape")
    rc = lib().viper_hip_qlinear_m1_swiglu(int(w_gate.qtype), int(w_gate.scale_enc), w_gate.group_size, w_gate.cols,
                                           int(prologue), ptr(a, 1 if int(prologue) == int(Prologue.INT8) else 2), ptr(b, 4 if int(prologue) == int(Prologue.INT8) else 2), float(eps), ptr(norm_out, 2),
                                           ptr(w_gate.data, 1), ptr(w_gate.scales, 2), ptr(w_up.data, 1), ptr(w_up.scales, 2),
                                           w_gate.rows, ptr(h, 2), ptr(gate_out, 2), ptr(up_out, 2), _stream(stream))
    return _status(rc, "viper_hip_qlinear_m1_swiglu")


def linear_bf16(w, x, y, stream=None) -> Status:
    """y[M, N] = x[M, K] w[N, K]^T, all bf16 (the LM head)."""
    N, K = w.shape
    M = int(x.numel() // K)
    rc = lib().viper_hip_linear_bf16(ptr(w, 2), ptr(x, 2), ptr(y, 2), M, N, K, _stream(stream))
    return _status(rc, "viper_hip_linear_bf16")


def sampling_greedy(logits, out_token, stream=None, workspace=None) -> Status:
    """out_token[b] = argmax of logits[b, :] (bf16), smallest index on ties.  With a workspace
    (greedy_workspace_bytes(B) bytes, zero before its first use) each row is split over many
    workgroups (viper_hip_sampling_greedy_split)."""
    V = logits.shape[-1]
    B = int(logits.numel() // V)
    if workspace is not None:
        nbytes = workspace.numel() * workspace.element_size()
        rc = lib().viper_hip_sampling_greedy_split(ptr(logits, 2), ptr(out_token, 4), B, V, ptr(workspace), nbytes,
                                                   _stream(stream))
        return _status(rc, "viper_hip_sampling_greedy_split")
    rc = lib().viper_hip_sampling_greedy(ptr(logits, 2), ptr(out_token, 4), B, V, _stream(stream))
    return _status(rc, "viper_hip_sampling_greedy")


def greedy_workspace_bytes(B: int) -> int:
    return int(lib().viper_hip_sampling_greedy_workspace_bytes(B))


def check_quantizer(exp_lo, exp_hi, counts, stream=None) -> Status:
    rc = lib().viper_hip_check_quantizer(exp_lo, exp_hi, ptr(counts), _stream(stream))
    return _status(rc, "viper_hip_check_quantizer")
