"""GPU parity of the LM head (bf16 GEMV) and greedy sampling against the CPU
oracle, through the C ABI.

Bar: logits within 1 bf16 ulp of the oracle's, or within 1e-5 * sum|w x|
(the reference's fp32 summation order is its own); the greedy token exactly
the oracle's argmax of the device's logits, and of the oracle's logits.
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


def bf16(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


@pytest.mark.parametrize("M,N,K", [(1, 4097, 2560), (3, 100, 1000), (1, 50, 64), (16, 33, 2048), (3, 70, 10240)])
def test_linear_bf16(torch_dev, M, N, K):
    torch = torch_dev
    print(f"linear_bf16 M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K + M)
    w = bf16(0.05 * rng.standard_normal((N, K)))
    x = O.gen_act(M, K, 900 + K)
    y_ref, _, absterm = O.linear_bf16(w, x)
    y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    assert va.linear_bf16(dev(torch, w), dev(torch, x), y).ok()
    torch.cuda.synchronize()
    O.assert_bf16_close(host_u16(y), y_ref, absterm, rel=1e-5)


def test_linear_bf16_limits_are_codes(torch_dev):
    torch = torch_dev
    w = torch.zeros((8, 10240), dtype=torch.int16, device="cuda")
    x = torch.zeros((5, 10240), dtype=torch.int16, device="cuda")   # 100 KiB of activations: over the LDS limit
    y = torch.zeros((5, 8), dtype=torch.int16, device="cuda")
    assert va.linear_bf16(w, x, y).code == va.StatusCode.INVALID_ARGUMENT
    x = torch.zeros((1, 10236), dtype=torch.int16, device="cuda")   # K % 8 != 0
    assert va.linear_bf16(torch.zeros((8, 10236), dtype=torch.int16, device="cuda"), x, y[:1]).code == \
        va.StatusCode.INVALID_ARGUMENT


def test_lm_head_full_size_greedy(torch_dev):
    # config 3's head: K=2560, N=166144 (850 MB of bf16 weights), M=1
    torch = torch_dev
    N, K = 166144, 2560
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0003)
    wd = (0.02 * torch.randn((N, K), device="cuda", generator=g)).to(torch.bfloat16)
    x = O.gen_act(1, K, 0x5EED0013)
    y = torch.zeros((1, N), dtype=torch.int16, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    assert va.linear_bf16(wd, dev(torch, x), y).ok()
    assert va.sampling_greedy(y, tok).ok()
    torch.cuda.synchronize()
    w = wd.view(torch.int16).cpu().numpy().view(np.uint16)
    y_ref, _, absterm = O.linear_bf16(w, x)
    yg = host_u16(y)
    O.assert_bf16_close(yg, y_ref, absterm, rel=1e-5)
    assert int(tok.item()) == int(O.argmax_bf16(yg)[0])
    assert int(tok.item()) == int(O.argmax_bf16(y_ref)[0])


def ws(torch, B, split):
    """The split entry point's workspace (zeroed once), or None for the one-workgroup kernel."""
    return torch.zeros(va.greedy_workspace_bytes(B), dtype=torch.uint8, device="cuda") if split else None


@pytest.mark.parametrize("split", [False, True])
def test_sampling_greedy_known_answers(torch_dev, split):
    torch = torch_dev
    rows = np.stack([
        bf16([1.0, 3.0, 3.0, 2.0, -1.0, 0.0, 0.0, 0.0]),
        bf16([np.nan, 0.5, np.nan, 0.25, 0.5, 0.0, -0.0, 0.1]),
        bf16([-np.inf] * 8),
        bf16([-np.inf, -5.0, np.inf, np.inf, 0.0, 0.0, 0.0, 0.0]),
        bf16([-2.0, -1.0, -3.0, -1.0, -7.0, -9.0, -9.0, -9.0]),
    ])
    out = torch.zeros(5, dtype=torch.int32, device="cuda")
    assert va.sampling_greedy(dev(torch, rows), out, workspace=ws(torch, 5, split)).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), [1, 1, 0, 2, 1])


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("B,V", [(3, 166144), (2, 1001), (4, 7), (2, 8200)])
def test_sampling_greedy_random(torch_dev, B, V, split):
    torch = torch_dev
    rng = np.random.default_rng(V)
    lg = bf16(rng.standard_normal((B, V)))
    lg[0, V // 3] = lg[0, V // 2] = bf16([9.0])[0]   # a tie across lanes: the smaller index
    out = torch.zeros(B, dtype=torch.int32, device="cuda")
    assert va.sampling_greedy(dev(torch, lg), out, workspace=ws(torch, B, split)).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), O.argmax_bf16(lg))
    assert out.cpu().numpy()[0] == V // 3


@pytest.mark.parametrize("split", [False, True])
def test_sampling_greedy_ties_within_a_lane(torch_dev, split):
    # Lane l scans octets l, l + 1024, ... in order: equal maxima in two octets
    # of one lane and twice within one octet (16-byte aligned rows), and in
    # the elements past the last octet (one row, V % 8 != 0), must all resolve
    # to the smallest index.
    torch = torch_dev
    top = bf16([7.5])[0]
    V = 166144
    lg = np.full((2, V), bf16([-1.0])[0], dtype=np.uint16)
    lg[0, 8 * 1030 + 6] = lg[0, 8 * 6 + 3] = top               # octets 6 and 1030: same lane
    lg[1, 8 * 2000 + 4] = lg[1, 8 * 2000 + 2] = top             # one octet, two equal values
    lg[1, 8 * 2000 + 1] = bf16([np.nan])[0]
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    assert va.sampling_greedy(dev(torch, lg), out, workspace=ws(torch, 2, split)).ok()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), [8 * 6 + 3, 8 * 2000 + 2])
    np.testing.assert_array_equal(out.cpu().numpy(), O.argmax_bf16(lg))
    Vt = 166144 + 5
    lt = np.full((1, Vt), bf16([-1.0])[0], dtype=np.uint16)
    lt[0, Vt - 2] = lt[0, Vt - 1] = top                         # the tail past the last octet
    lt[0, 8 * 17 + 1] = bf16([7.25])[0]
    ot = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert va.sampling_greedy(dev(torch, lt), ot, workspace=ws(torch, 1, split)).ok()
    torch.cuda.synchronize()
    assert ot.cpu().numpy()[0] == Vt - 2 == O.argmax_bf16(lt)[0]


def test_sampling_greedy_split_across_workgroups(torch_dev):
    # The split kernel's workgroups cover 4096 logits each and meet through
    # one 64-bit key per row: equal maxima in different workgroups resolve to
    # the smaller index, -0 and +0 are equal (the first wins), a row with
    # nothing above -inf (NaN included) gives 0, and the workspace is zero
    # again after every call, so calls in a row reuse it with other shapes.
    torch = torch_dev
    V = 166144
    neg = bf16([-1.0])[0]
    lg = np.full((4, V), neg, dtype=np.uint16)
    lg[0, 4096 * 30 + 5] = lg[0, 4096 * 7 + 4095] = lg[0, V - 1] = bf16([3.0])[0]   # workgroups 7, 30, 40
    lg[1, :] = bf16([-2.0])[0]
    lg[1, 4096 * 9 + 1] = bf16([-0.0])[0]
    lg[1, 4096 * 2 + 3] = bf16([0.0])[0]                                             # +0 first: it wins
    lg[1, 4096 * 20] = bf16([-0.0])[0]
    lg[2, :] = bf16([-np.inf])[0]
    lg[2, 4096 * 12 + 8] = bf16([np.nan])[0]
    lg[3, :] = bf16([np.nan])[0]
    lg[3, 4096 * 39 + 77] = bf16([-np.inf])[0]
    lg[3, 4096 * 40 + 1] = bf16([-65504.0])[0]                                       # the only finite value
    expect = O.argmax_bf16(lg)
    np.testing.assert_array_equal(expect, [4096 * 7 + 4095, 4096 * 2 + 3, 0, 4096 * 40 + 1])
    w = ws(torch, 8, True)
    out = torch.full((4,), -1, dtype=torch.int32, device="cuda")
    for rows, V2 in ((4, V), (1, V), (3, 8200), (4, V)):
        src = lg[:rows, :V2]
        e = O.argmax_bf16(np.ascontiguousarray(src))
        out.fill_(-1)
        assert va.sampling_greedy(dev(torch, src), out[:rows], workspace=w).ok()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out[:rows].cpu().numpy(), e)
        assert int(w.count_nonzero()) == 0


def test_sampling_greedy_split_two_streams_concurrent(torch_dev):
    # two split greedy picks in flight at once on two streams (default
    # priority), each with its own workspace, called repeatedly: every token
    # equals the oracle's argmax and each workspace is zero afterwards
    torch = torch_dev
    V, B = 166144, 3
    rng = np.random.default_rng(7)
    lgs = [bf16(rng.standard_normal((B, V)).astype(np.float32)) for _ in range(2)]
    expect = [O.argmax_bf16(lg) for lg in lgs]
    lds = [dev(torch, lg) for lg in lgs]
    wss = [ws(torch, B, True) for _ in range(2)]
    outs = [[torch.full((B,), -1, dtype=torch.int32, device="cuda") for _ in range(8)] for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for i in range(8):
        for k in range(2):
            assert va.sampling_greedy(lds[k], outs[k][i], stream=streams[k], workspace=wss[k]).ok()
    torch.cuda.synchronize()
    for k in range(2):
        for o in outs[k]:
            np.testing.assert_array_equal(o.cpu().numpy(), expect[k])
        assert int(wss[k].sum().item()) == 0
