"""nmq_moe_down_static, the allocation-free form of nmq_moe_down (its two-launch form keeps the slot
results in the library's own device array): through the C ABI, two calls in a row -- the second with a
smaller input -- each equal bit for bit to nmq_moe_down on a workspace of its own; also the one-launch
shape, a shape too large for the array (refused), and a call captured in a HIP graph and replayed."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import random_blocks

pytestmark = pytest.mark.gpu

TYPE = {"Q6_K": 14, "Q4_K": 12, "Q8_0": 8}
BV = {"Q6_K": 256, "Q4_K": 256, "Q8_0": 32}


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def nmq():
    from ggufengine_amd import _native
    if not _native.available("cuda"):
        pytest.fail("libnmq.so not loaded or device is not gfx950 -- the HIP path must run here")
    return _native


def _case(fmt, L, k, E, FF, n_exp, seed):
    raw = random_blocks(fmt, n_exp * E * FF // BV[fmt], seed=seed)
    rng = np.random.default_rng(seed + 1)
    w = torch.from_numpy(raw).cuda()
    gu = torch.from_numpy(rng.standard_normal((2 * L * k, FF)).astype(np.float32)).cuda()
    ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
    wts = torch.from_numpy(rng.random((L, k)).astype(np.float32)).cuda()
    return w, raw.size // n_exp, gu, ids, wts


def _with_workspace(nmq, fmt, w, per, gu, ids, wts, L, k, E, FF):
    need = ctypes.c_int64(0)
    nmq.check(nmq.lib().nmq_moe_down_work_bytes(TYPE[fmt], L, k, E, FF, ctypes.byref(need)))
    work = torch.empty(max(need.value, 256), dtype=torch.uint8, device="cuda")
    out = torch.empty(L, E, device="cuda")
    n = L * k
    nmq.check(nmq.lib().nmq_moe_down(TYPE[fmt], w.data_ptr(), ids.data_ptr(), L, k, per, gu.data_ptr(),
                                     nmq.X_SILU_MUL_BF16, gu[n:].data_ptr(), wts.data_ptr(), out.data_ptr(), E, FF,
                                     work.data_ptr(), work.numel(), nmq.stream_ptr()))
    torch.cuda.synchronize()
    return out


def _static(nmq, fmt, w, per, gu, ids, wts, L, k, E, FF, out=None):
    out = torch.empty(L, E, device="cuda") if out is None else out
    n = L * k
    rc = nmq.lib().nmq_moe_down_static(TYPE[fmt], w.data_ptr(), ids.data_ptr(), L, k, per, gu.data_ptr(),
                                       nmq.X_SILU_MUL_BF16, gu[n:].data_ptr(), wts.data_ptr(), out.data_ptr(), E, FF,
                                       nmq.stream_ptr())
    nmq.check(rc)
    return out


@pytest.mark.parametrize("fmt,E,FF", [("Q6_K", 1024, 5120), ("Q8_0", 768, 4160), ("Q6_K", 2048, 768)])
def test_static_equals_workspace_two_calls(nmq, fmt, E, FF):
    """FF 5120 / 4160: rows longer than the one-launch kernel takes, so the slot results go through the
    library's array; FF 768: the one-launch kernel (the array is not used).  First call L=4, k=8, then a
    smaller one (L=1, k=4) on new inputs: both equal nmq_moe_down on a workspace."""
    for call, (L, k) in enumerate(((4, 8), (1, 4))):
        w, per, gu, ids, wts = _case(fmt, L, k, E, FF, 12, 300 + call + FF)
        say("moe_down_static", fmt, E, FF, L, k)
        got = _static(nmq, fmt, w, per, gu, ids, wts, L, k, E, FF)
        torch.cuda.synchronize()
        want = _with_workspace(nmq, fmt, w, per, gu, ids, wts, L, k, E, FF)
        assert torch.equal(got, want), (fmt, E, FF, L, k)


def test_static_refuses_results_larger_than_its_array(nmq):
    """L*k x n_out fp32 beyond NMQ_MOE_SCRATCH_BYTES (8 MiB): refused before anything is launched."""
    L, k, E, FF = 64, 16, 2048, 5120            # 64*16*2048*4 = 8 MiB + 0 -> 2^23 bytes: the limit itself
    w, per, gu, ids, wts = _case("Q6_K", 1, 1, E, FF, 2, 311)
    big_ids = torch.zeros(L * k + 64, dtype=torch.int64, device="cuda")
    big_w = torch.ones(L + 4, k, device="cuda")
    out = torch.empty(L + 4, E, device="cuda")
    gu_big = torch.zeros(2 * (L + 4) * k, FF, device="cuda")
    n = (L + 4) * k
    rc = nmq.lib().nmq_moe_down_static(14, w.data_ptr(), big_ids.data_ptr(), L + 4, k, per, gu_big.data_ptr(),
                                       nmq.X_SILU_MUL_BF16, gu_big[n:].data_ptr(), big_w.data_ptr(), out.data_ptr(),
                                       E, FF, nmq.stream_ptr())
    assert rc == nmq.NMQ_ERR_SHAPE


def test_static_in_a_graph(nmq):
    """One call captured and replayed with new ids written between the replays (eager work in between):
    every replay equals nmq_moe_down on a workspace."""
    L, k, E, FF = 2, 8, 1024, 5120
    w, per, gu, ids, wts = _case("Q6_K", L, k, E, FF, 12, 321)
    out = torch.empty(L, E, device="cuda")
    say("moe_down_static graph")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _static(nmq, "Q6_K", w, per, gu, ids, wts, L, k, E, FF, out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _static(nmq, "Q6_K", w, per, gu, ids, wts, L, k, E, FF, out)
    rng = np.random.default_rng(322)
    for rep in range(3):
        ids.copy_(torch.from_numpy(rng.integers(0, 12, L * k)))
        g.replay()
        torch.cuda.synchronize()
        want = _with_workspace(nmq, "Q6_K", w, per, gu, ids, wts, L, k, E, FF)
        assert torch.equal(out, want), rep
