"""C-ABI library checks that need no GPU: it loads, exports every entry point
include/viper_qlinear.h declares, and rejects bad arguments with the
reference's status codes (include/viper/status.h:12-21) before touching the
device.  Argument rules follow the reference launchers
(kernels/ops/linear_multim.cu:152, dp4a_smem_kernel.cu:82, linear.cpp:33-35)."""
import ctypes as C
import os
import re

import pytest

import viper_amd as va
from viper_amd import qlinear as ql

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "viper_qlinear.h")


def declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(viper_hip_\w+)\s*\(", txt, re.M)))


def test_header_symbols_exported():
    L = va.lib()
    names = declared()
    assert len(names) >= 9
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(ql._SYMBOLS)
    assert L.viper_hip_abi_version() == 7


def test_group_sizes_and_workspace():
    L = va.lib()
    assert [L.viper_hip_group_size(q) for q in (4, 5, 6, 8, 0, 1, 7)] == [64, 64, 64, 32, 0, 0, 0]
    assert va.workspace_bytes(4, 10240, 2560, 1) == 0
    # the K split's control words and 1024 block counters (4352 bytes, for
    # every M > 1 shape), int8 activations with room for 16 rows, then fp32
    # scales for 16 rows per group
    CTL = 256 + 4 * 1024
    assert va.workspace_bytes(4, 10240, 2560, 4) == CTL + 16 * 2560 + 40 * 16 * 4
    assert va.workspace_bytes(8, 10, 2560, 3) == CTL + 16 * 2560 + 80 * 16 * 4
    assert va.workspace_bytes(6, 10, 2496, 3) == CTL + 16 * 2496 + 39 * 16 * 4
    # long K (the K split): one record of 8 parts x 16 rows x 48 64-bit slots
    # per row block (down shape: 107 blocks of 24 rows), before xq and xs
    REC = 8 * 16 * 48 * 8
    assert va.workspace_bytes(4, 2560, 10240, 16) == CTL + 107 * REC + 16 * 10240 + 160 * 16 * 4
    nb8 = va.workspace_layout(8, 2560, 10240, 3)["split_blocks"]     # W8: 80 quads, 8 parts of 10
    assert 0 < nb8 <= 107
    assert va.workspace_bytes(8, 2560, 10240, 3) == CTL + nb8 * REC + 16 * 10240 + 320 * 16 * 4
    assert va.workspace_bytes(4, 2560, 5120, 16) == CTL + 16 * 5120 + 80 * 16 * 4   # one segment: no split
    # the fragment-input entry: control words and records only, 0 without a split
    assert va.frag_workspace_bytes(4, 2560, 10240, 16) == CTL + 107 * REC
    assert va.frag_workspace_bytes(4, 10240, 2560, 16) == 0
    assert va.frag_workspace_bytes(4, 2560, 10240, 1) == 0
    # K = 6144 (24 quads: 3 parts of 8, 128 blocks of 24 rows)
    assert va.workspace_layout(4, 3072, 6144, 16)["split_blocks"] == 128


def _split_shapes():
    for qtype in (4, 5, 6, 8):
        for K in (6144, 10240, 10752, 12288, 20480):
            for M in (5, 6, 9, 12, 16):
                for N in (64, 640, 1000, 2048, 2560, 3072, 10240):
                    yield qtype, N, K, M


def test_split_layout_fixed_for_every_shape():
    # The K split's counters and records of part sums sit at the same offsets
    # for every shape (a record is written only by its own row block, whose
    # counter carries the epoch the record's tags are made from), the missed-sum
    # count at 4; xq and xs follow the records and nothing overlaps.
    CTL, REC = 256 + 4 * 1024, 8 * 16 * 48 * 8
    seen = 0
    for qtype, N, K, M in _split_shapes():
        lay = va.workspace_layout(qtype, N, K, M)
        assert lay["missed"] == 4 and lay["counters"] == 256, (qtype, N, K, M)
        nb = lay["split_blocks"]
        if lay["sums"] is None:
            assert nb == 0 and lay["xq"] == CTL
            continue
        seen += 1
        assert 0 < nb <= 1024 and lay["sums"] == CTL
        assert nb * 48 >= N and (nb - 1) * 8 < N                 # blocks of 8..48 rows cover N
        assert lay["xq"] == CTL + nb * REC
        assert lay["xq"] % 16 == 0 and lay["xs"] % 16 == 0
        assert lay["xq"] + 16 * K <= lay["xs"]
        G = 32 if qtype == 8 else 64
        assert lay["xs"] + (K // G) * 16 * 4 == lay["total"] == va.workspace_bytes(qtype, N, K, M)
        assert va.frag_workspace_bytes(qtype, N, K, M) == CTL + nb * REC
    assert seen > 300
    lay = va.workspace_layout(4, 10240, 2560, 8)
    assert lay["sums"] is None and lay["split_blocks"] == 0 and lay["counters"] == 256
    assert va.workspace_layout(4, 10240, 2560, 1)["total"] == 0


def test_split_tag_cannot_match_library_words():
    # A slot is accepted when its high word equals the call's tag, whose top
    # byte is 0x80.  The other words the library stores where slots can lie
    # are int8 activations and fp32 activation scales (the counters have a
    # region of their own): the
    # quantizer's bytes never include 0x80 (|q| <= 127, also for groups
    # holding the largest finite bf16 values, and the device quantizer equals
    # the oracle's on every finite bf16 pair, test_device_quantizer_exhaustive)
    # and its scales are positive (bit 31 clear, unlike every tag).
    import numpy as np
    import oracle as O
    rng = np.random.default_rng(0x7A6)
    x = (rng.standard_normal((4, 4096)) * np.exp(rng.uniform(-30, 30, (4, 1)))).astype(np.float32)
    x[0, :64] = np.float32(3.3895e38)                      # the largest bf16 magnitudes
    x[1, 64:128] = -np.float32(3.3895e38)
    x[2, 128:192] = 0.0
    x[3, 192:256] = np.float32(1e-38)
    xb = O.f32_to_bf16(x)
    for G in (64, 32):
        q, s = O.quantize_act(xb, G)
        assert 0x80 not in set(np.asarray(q, dtype=np.int8).view(np.uint8).ravel().tolist())
        sb = np.asarray(s, dtype=np.float32).view(np.uint32)
        assert np.all((sb & np.uint32(0x80000000)) == 0)
    assert all((0x80000000 | (g & 0xFFFFFF)) >> 24 == 0x80 for g in (0, 1, 0xFFFFFF, 0x1000000, 0xFFFFFFFF))


FAKE = 0x10000  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("args,code", [
    (dict(qtype=0), 1),             # BF16: not on this path (UNIMPLEMENTED, as linear.cpp:19-24)
    (dict(qtype=1), 1),
    (dict(qtype=7), 2),             # bad dtype -> INVALID_ARGUMENT (linear.cpp:33-35)
    (dict(w=None), 2),
    (dict(s=None), 2),
    (dict(x=None), 2),
    (dict(y=None), 2),
    (dict(M=17), 2),                # M > 16 (linear_multim.cu:152)
    (dict(M=0), 2),
    (dict(N=0), 2),
    (dict(K=96), 2),                # K % 64 != 0 (dp4a_smem_kernel.cu:82)
    (dict(K=(1 << 24) + 64), 2),    # K past VIPER_QLINEAR_MAX_K (32-bit block addressing)
    (dict(group=32), 2),            # group does not match the format
    (dict(senc=2), 2),
    (dict(w=FAKE + 8), 2),          # weights not 16-byte aligned
    (dict(s=FAKE + 2), 2),          # scales not 16-byte aligned (read in 16-byte blocks)
    (dict(s=FAKE + 8), 2),
    (dict(x=FAKE + 4), 2),
    (dict(M=2), 2),                 # M > 1 needs a workspace
])
def test_argument_validation(args, code):
    a = dict(qtype=4, w=FAKE, s=FAKE, senc=0, group=64, N=64, K=128, x=FAKE, M=1, y=FAKE)
    a.update(args)
    rc = va.lib().viper_hip_qlinear(a["qtype"], a["w"], a["s"], a["senc"], a["group"], a["N"], a["K"],
                                    a["x"], a["M"], a["y"], None, None, 0, None)
    assert rc == code


def test_other_entry_validation():
    L = va.lib()
    assert L.viper_hip_quantize_act(48, FAKE, 1, 96, FAKE, FAKE, None) == 2
    assert L.viper_hip_quantize_act(64, FAKE, 1, 96, FAKE, FAKE, None) == 2
    assert L.viper_hip_qlinear_prequantized(4, FAKE, FAKE, 0, 64, 8, 64, None, FAKE, 1, FAKE, None, None) == 2
    assert L.viper_hip_qlinear_partials(4, FAKE, FAKE, 0, 64, 8, 64, FAKE, 1, FAKE, None, None, 0, None, None) == 2
    assert L.viper_hip_check_quantizer(10, 5, FAKE, None) == 2
    assert L.viper_hip_check_quantizer(0, 255, FAKE, None) == 2
    assert L.viper_hip_sampling_greedy_workspace_bytes(3) == 48
    assert L.viper_hip_sampling_greedy_workspace_bytes(0) == 0
    assert L.viper_hip_sampling_greedy_split(FAKE, FAKE, 2, 4096, None, 32, None) == 2        # no workspace
    assert L.viper_hip_sampling_greedy_split(FAKE, FAKE, 2, 4096, FAKE, 31, None) == 2        # too small
    assert L.viper_hip_sampling_greedy_split(FAKE, FAKE, 2, 4096, FAKE + 4, 32, None) == 2    # not 8-byte aligned
    assert L.viper_hip_sampling_greedy_split(FAKE, FAKE, 0, 4096, FAKE, 32, None) == 2
    assert L.viper_hip_sampling_greedy_split(FAKE + 1, FAKE, 2, 4096, FAKE, 32, None) == 2    # logits not bf16-aligned
    assert L.viper_hip_empty_dispatch(0, 64, None, None) == 2
    assert L.viper_hip_empty_dispatch(1, 65, None, None) == 2                                 # not whole waves
    assert L.viper_hip_empty_dispatch(1, 1088, None, None) == 2
    assert L.viper_hip_empty_dispatch(1, 64, FAKE + 1, None) == 2                             # y not 2-byte aligned
    W = 320 * 5 * 16                                                      # one workgroup's bytes
    assert L.viper_hip_stream_read(None, W, 320, 5, None, 0, None, FAKE, None) == 2
    assert L.viper_hip_stream_read(FAKE, 0, 320, 5, None, 0, None, FAKE, None) == 2
    assert L.viper_hip_stream_read(FAKE, W + 16, 320, 5, None, 0, None, FAKE, None) == 2  # not whole workgroups
    assert L.viper_hip_stream_read(FAKE + 8, W, 320, 5, None, 0, None, FAKE, None) == 2   # buffer not 16-byte aligned
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, None, 0, None, None, None) == 2
    assert L.viper_hip_stream_read(FAKE, W, 300, 5, None, 0, None, FAKE, None) == 2       # no such shape
    assert L.viper_hip_stream_read(FAKE, W, 320, 6, None, 0, None, FAKE, None) == 2
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, None, 0, FAKE + 1, FAKE, None) == 2   # y not 2-byte aligned
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, FAKE, 1608, None, FAKE, None) == 2    # side not whole words
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, FAKE, 16 * 321, None, FAKE, None) == 2  # side past one per thread
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, None, 1600, None, FAKE, None) == 2    # side bytes without side
    assert L.viper_hip_stream_read(FAKE, W, 320, 5, FAKE, 0, None, FAKE, None) == 2       # side without bytes
    assert L.viper_hip_stream_read(FAKE + 8, W, 320, 5, FAKE + 8, 16, None, FAKE, None) == 2


def test_registry_mirror():
    assert [va.qtype_name(q) for q in (0, 1, 4, 5, 6, 8, 3)] == [
        "BF16", "FP32", "Q4_G64", "Q5_G64", "Q6_G64", "W8_G32", "UNKNOWN"]
    assert va.is_lossless(0) and va.is_lossless(1) and not va.is_lossless(4)
    assert va.packed_bytes(va.QType.Q5_G64, 2, 64) == 2 * 32 + 2 * 8


def test_wrapper_rejects_host_tensors():
    # a CPU tensor's address would reach the kernels as a device address
    torch = pytest.importorskip("torch")
    with pytest.raises(ValueError):
        ql.ptr(torch.zeros(4))
    assert ql.ptr(None) is None

