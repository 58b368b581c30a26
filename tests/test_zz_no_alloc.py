"""The allocation-free entry point viper_hip_qlinear_static, through the C ABI.

Its output must equal viper_hip_qlinear's (same kernels, caller workspace) bit
for bit and the oracle's to the parity bar, on calls in a row on one GPU: the
static array keeps the previous call's contents (K-split control words and
sums, activation fragments), so sequences shrink, grow and alternate between
K-split shapes.  Shapes past the static array are rejected before any device
work.
"""
import ctypes as C

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


def _dev(torch, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda")


def _call_pair(torch, L, qtype, N, K, M, seed, residual):
    G = O.group_size(qtype)
    print(f"case qtype={qtype} N={N} K={K} M={M} seed={seed} res={residual}", flush=True)
    packed, scales = O.gen_weights(qtype, N, K, seed, O.SCALE_FP16)
    x = O.gen_act(M, K, seed + 1)
    wd, sd, xd = _dev(torch, packed), _dev(torch, scales), _dev(torch, x)
    rd = _dev(torch, O.gen_act(M, N, seed + 2)) if residual else None
    nws = L.viper_hip_qlinear_workspace_bytes(qtype, N, K, M)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")
    y_ref = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    y_st = torch.full((M, N), 7, dtype=torch.int16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    r = rd.data_ptr() if rd is not None else None
    rc = L.viper_hip_qlinear(qtype, wd.data_ptr(), sd.data_ptr(), O.SCALE_FP16, G, N, K, xd.data_ptr(), M,
                             y_ref.data_ptr(), r, ws.data_ptr() if nws else None, nws, st)
    assert rc == 0
    rc = L.viper_hip_qlinear_static(qtype, wd.data_ptr(), sd.data_ptr(), O.SCALE_FP16, G, N, K, xd.data_ptr(), M,
                                    y_st.data_ptr(), r, st)
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y_st.cpu().numpy(), y_ref.cpu().numpy())
    res = None if rd is None else O.gen_act(M, N, seed + 2)
    y_o, _, absterm = O.qlinear(qtype, packed, scales, O.SCALE_FP16, N, K, x, residual=res)
    O.assert_bf16_close(y_st.cpu().numpy().view(np.uint16), y_o, absterm, rel=1e-5)
    return y_st


# (qtype, N, K, M) sequences: shrinking (the K split (long K) with its
# counters and records of sums, the fragment quantize + matrix-core path, the
# multi-row path, and M = 1 with no workspace at all), growing (each call's
# K-split sums cover more of the array than the last), two K-split shapes
# alternating, and K splits in 4 and 3 parts (K = 10240, 10752) alternating.
SEQUENCES = [
    [(O.Q4_G64, 2560, 10240, 16), (O.Q4_G64, 1000, 10240, 5)],
    [(O.W8_G32, 2048, 10240, 12), (O.W8_G32, 777, 6144, 4)],
    [(O.Q5_G64, 10240, 2560, 16), (O.Q5_G64, 4000, 2560, 8)],
    [(O.Q4_G64, 10240, 2560, 8), (O.Q4_G64, 2560, 2560, 2), (O.Q4_G64, 2560, 2560, 1)],
    [(O.Q4_G64, 2560, 10240, 5), (O.Q4_G64, 2560, 10240, 6), (O.Q4_G64, 2560, 10240, 16),
     (O.Q4_G64, 1000, 10240, 16), (O.Q4_G64, 2560, 10240, 16)],
    [(O.Q4_G64, 2048, 10240, 5), (O.Q4_G64, 640, 10240, 16)] * 5,
    [(O.Q4_G64, 3072, 10752, 16), (O.Q4_G64, 2560, 10240, 9)] * 3,
]


@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_static_equals_workspace_entry(torch_dev, seq):
    L = va.lib()
    for i, (qtype, N, K, M) in enumerate(SEQUENCES[seq]):
        _call_pair(torch_dev, L, qtype, N, K, M, seed=0x5A7100 + 31 * seq + i, residual=(i % 2 == 1))


def test_static_rejects_past_the_array():
    L = va.lib()
    cap = 8 << 20
    for N, K, M in ((64, 1 << 20, 16),        # int8 activations alone: 16 * 2^20 bytes
                    (4096, 1 << 19, 9)):      # 8 MiB of int8 activations plus their scales
        assert L.viper_hip_qlinear_workspace_bytes(O.Q4_G64, N, K, M) > cap
        fake = C.c_void_p(0x10000)          # never dereferenced: the size check comes first
        rc = L.viper_hip_qlinear_static(O.Q4_G64, fake, fake, 0, 64, N, K, fake, M, fake, None, None)
        assert rc == 2
