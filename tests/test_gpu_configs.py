"""GPU parity at the workloads' own shapes and data, through the C ABI and the default launch plan:

  - Q8_0 4096x4096, one token, W ~N(0,0.02) (seed 11), x ~N(0,1) (seed 12);
  - Q4_K 14336x4096 / 4096x4096 (seeds 31, 32) at 1, 2, 3, 4 and 8 tokens (x seed 33) -- the speculative
    verify shapes, 2..4 tokens also bit for bit equal to one-token launches;
  - Q4_0 14336x4096 at one token;
  - TQ2_0 (codes with P(0) = 0.4, P(+-1) = 0.3, fp16 d = |N(0,0.02)|, seed 51) and IQ2_XXS (encoded from
    N(0,0.02), seed 52) at 4096x4096 and 12288x4096, one token (x seed 53), from the two-stage input and
    from fp32 values -- the 12288-row launches run the persistent kernel with hand-issued reads;
  - every format on small matrices with the persistent one-token kernel forced (its hand-issued and
    compiler-scheduled reads), from the two-stage input and from fp32 values;
  - the MoE expert layer with all 128 experts (gate/up 768x2048 Q4_K, down 2048x768 Q6_K, seed 41; router
    logits seed 42, top-8 softmax renormalised; x seed 43) at 1 and 4 tokens, each stage and the layer end
    to end against the oracle.

Bars: fp32 outputs per output row-vector max|y - ref| / max|ref| <= 1e-3 against dequantise + matmul on
the same x, and <= 2e-5 against the oracle of the same integer decomposition (two-stage int8 input).
"""
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TYPE = {"Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ2_XXS": 16, "TQ2_0": 35}
BV = {"Q4_0": 32, "Q8_0": 32, "Q4_K": 256, "Q6_K": 256, "TQ2_0": 256, "IQ2_XXS": 256}
TOL_DEQ = 1e-3
TOL_INT = 2e-5
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def nmq():
    from ggufengine_amd import _native
    if not _native.available("cuda"):
        pytest.fail("libnmq.so not loaded or device is not gfx950 -- the HIP path must run here")
    return _native


def gauss(seed, shape, scale=1.0):
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    return x * np.float32(scale) if scale != 1.0 else x


def weights(fmt, rows, n_in, seed):
    from ggufengine_amd import encode
    return encode.encode(fmt, gauss(seed, (rows * n_in,), 0.02), threads=THREADS)


def ternary(rows, n_in, seed):
    from ggufengine_amd import encode
    g = np.random.Generator(np.random.PCG64(seed))
    nb = rows * n_in // 256
    codes = g.choice(np.array([0, 1, 2], dtype=np.uint8), size=(nb, 256), p=[0.3, 0.4, 0.3])
    d16 = np.abs(g.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    return encode.pack_ternary(codes, d16)


def mv_abi(nmq, fmt, w_dev, x_np, rows, n_in, values=False):
    """y (n, rows) of nmq_mv on x's two-stage input, or of nmq_mv_x on x's fp32 values (one token)."""
    from ggufengine_amd import mmvq
    L = nmq.lib()
    n = x_np.shape[0]
    x = torch.from_numpy(np.ascontiguousarray(x_np)).cuda()
    y = torch.empty(n, rows, dtype=torch.float32, device="cuda")
    if values:
        assert n == 1
        import ctypes
        ws = (ctypes.c_void_p * 1)(w_dev.data_ptr())
        ns = (ctypes.c_int * 1)(rows)
        ys = (ctypes.c_void_p * 1)(y.data_ptr())
        nmq.check(L.nmq_mv_x(TYPE[fmt], 1, ws, ns, ys, x.data_ptr(), nmq.X_F32, None, n_in, nmq.stream_ptr()))
    else:
        e = mmvq.Eingang(x)
        nmq.check(L.nmq_mv(TYPE[fmt], w_dev.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                           e.xs.data_ptr(), y.data_ptr(), rows, n_in, n, nmq.stream_ptr()))
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check(oracle, fmt, raw, rows, n_in, x_np, y):
    ref = oracle.mv_deq(fmt, raw, rows, n_in, x_np)
    err = float(oracle.rel_err_rows(y, ref).max())
    assert err <= TOL_DEQ, (fmt, rows, n_in, err)
    xq, xq2, xd, xs = oracle.quant_q8(x_np)
    ref_i = oracle.mv_int(fmt, raw, rows, n_in, xq, xq2, xd, xs, ncols=x_np.shape[0])
    err_i = float(oracle.rel_err_rows(y, ref_i).max())
    assert err_i <= TOL_INT, (fmt, rows, n_in, err_i)


def test_q8_0_4096_batch1(nmq, oracle):
    raw = weights("Q8_0", 4096, 4096, 11)
    x = gauss(12, (1, 4096))
    say("Q8_0 4096x4096 batch 1")
    w = torch.from_numpy(raw).cuda()
    check(oracle, "Q8_0", raw, 4096, 4096, x, mv_abi(nmq, "Q8_0", w, x, 4096, 4096))
    check(oracle, "Q8_0", raw, 4096, 4096, x, mv_abi(nmq, "Q8_0", w, x, 4096, 4096, values=True))


@pytest.fixture(scope="module")
def q4k_spec():
    return {rows: weights("Q4_K", rows, 4096, seed) for rows, seed in ((14336, 31), (4096, 32))}


@pytest.mark.parametrize("rows", [14336, 4096])
def test_q4k_speculative_verify(nmq, oracle, q4k_spec, rows):
    raw = q4k_spec[rows]
    X = gauss(33, (8, 4096))
    w = torch.from_numpy(raw).cuda()
    ones = [mv_abi(nmq, "Q4_K", w, X[c:c + 1], rows, 4096)[0] for c in range(8)]
    for n in (1, 2, 3, 4, 8):
        say("Q4_K speculative", rows, "x 4096, tokens", n)
        y = mv_abi(nmq, "Q4_K", w, X[:n], rows, 4096)
        check(oracle, "Q4_K", raw, rows, 4096, X[:n], y)
        if n <= 4:   # the few-token kernel promises the one-token results bit for bit
            for c in range(n):
                assert np.array_equal(y[c].view(np.uint32), ones[c].view(np.uint32)), (rows, n, c)


def test_q4_0_14336_batch1(nmq, oracle):
    raw = weights("Q4_0", 14336, 4096, 31)
    x = gauss(53, (1, 4096))
    say("Q4_0 14336x4096 batch 1")
    w = torch.from_numpy(raw).cuda()
    check(oracle, "Q4_0", raw, 14336, 4096, x, mv_abi(nmq, "Q4_0", w, x, 14336, 4096))


@pytest.fixture(scope="module")
def lowbit():
    iq = weights("IQ2_XXS", 12288, 4096, 52)
    tq = ternary(12288, 4096, 51)
    out = {}
    for rows in (4096, 12288):
        nbytes = rows * 16 * 66
        out[("TQ2_0", rows)] = tq[:nbytes] if rows == 12288 else ternary(rows, 4096, 51)
        out[("IQ2_XXS", rows)] = iq[:nbytes]      # the first rows of the larger matrix
    return out


@pytest.mark.parametrize("fmt", ["TQ2_0", "IQ2_XXS"])
@pytest.mark.parametrize("rows", [4096, 12288])
@pytest.mark.parametrize("values", [False, True])
@pytest.mark.parametrize("hand", [True, False])
def test_lowbit_batch1(nmq, oracle, tune, lowbit, fmt, rows, values, hand):
    """12288 rows: the persistent kernel (more than 24 rows per CU) with its hand-issued reads, and with
    the compiler-scheduled loop (MV1_HR = 0); 4096 rows: the chunk kernel (hand makes no difference)."""
    if rows == 4096 and not hand:
        pytest.skip("the chunk kernel has one read schedule")
    if not hand:
        tune(MV1_HR=0)
    raw = lowbit[(fmt, rows)]
    x = gauss(53, (1, 4096))
    say("lowbit", fmt, rows, "values" if values else "two-stage", "hand" if hand else "compiler")
    w = torch.from_numpy(raw).cuda()
    check(oracle, fmt, raw, rows, 4096, x, mv_abi(nmq, fmt, w, x, rows, 4096, values=values))


@pytest.mark.parametrize("fmt", ["Q4_0", "Q8_0", "Q4_K", "Q6_K", "TQ2_0", "IQ2_XXS"])
@pytest.mark.parametrize("values", [False, True])
@pytest.mark.parametrize("hand", [True, False])
def test_persistent_kernel_forced(nmq, oracle, tune, fmt, values, hand):
    """The persistent one-token kernel at any row count (MV1_MODE = 2): rows that end inside a team,
    fewer rows than waves, one and two units per lane."""
    from conftest import random_blocks
    tune(MV1_MODE=2)
    if not hand:
        tune(MV1_HR=0)
    for rows, n_in in ((1000, 4096), (37, 2048), (613, 8192), (4100, 1024)):
        raw = random_blocks(fmt, rows * n_in // BV[fmt], seed=rows + n_in)
        x = gauss(rows, (1, n_in))
        say("persistent forced", fmt, rows, n_in, values, hand)
        w = torch.from_numpy(raw).cuda()
        check(oracle, fmt, raw, rows, n_in, x, mv_abi(nmq, fmt, w, x, rows, n_in, values=values))


def _expert(raw, n_exp, e):
    per = raw.size // n_exp
    return raw[e * per:(e + 1) * per]


@pytest.fixture(scope="module")
def moe_weights():
    n_exp, E, FF = 128, 2048, 768
    g = np.random.Generator(np.random.PCG64(41))

    def enc(fmt, rows, n_in):
        from ggufengine_amd import encode
        w = g.standard_normal(n_exp * rows * n_in, dtype=np.float32) * np.float32(0.02)
        return encode.encode(fmt, w, threads=THREADS)
    return {"gate": enc("Q4_K", FF, E), "up": enc("Q4_K", FF, E), "down": enc("Q6_K", E, FF)}


@pytest.mark.parametrize("L", [1, 4])
def test_moe_128_experts(nmq, oracle, moe_weights, L):
    from ggufengine_amd import experts
    n_exp, k, E, FF = 128, 8, 2048, 768
    raw = moe_weights
    gate = experts.PackedExperts(torch.from_numpy(raw["gate"]).cuda(), 12, n_exp, FF, E)
    up = experts.PackedExperts(torch.from_numpy(raw["up"]).cuda(), 12, n_exp, FF, E)
    down = experts.PackedExperts(torch.from_numpy(raw["down"]).cuda(), 14, n_exp, E, FF)
    layer = experts.Experten(gate, up, down)
    logits = gauss(42, (L, n_exp))
    x = gauss(43, (L, E))
    idx, w = experts.auswahl(torch.from_numpy(logits).cuda(), k)
    say("moe 128 experts, tokens", L)
    out = layer(torch.from_numpy(x).cuda(), idx, w).cpu().numpy()
    torch.cuda.synchronize()
    ids = idx.cpu().numpy()
    wts = w.cpu().numpy().astype(np.float64)
    # the router against softmax / top-k / renormalise in fp64
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :k]
    assert np.array_equal(np.sort(ids, 1), np.sort(top, 1))
    ref_w = np.take_along_axis(p, ids, 1)
    ref_w /= ref_w.sum(1, keepdims=True)
    assert np.abs(wts - ref_w).max() <= 1e-6
    # the chain in the oracle: gate and up on each token's bf16 input, silu(g) * u rounded to bf16,
    # down on each slot, the weighted sum
    xb = oracle.round_bf16(x)
    pairs = [(t, int(ids[t, j])) for t in range(L) for j in range(k)]
    g_o = np.stack([oracle.mv_deq("Q4_K", _expert(raw["gate"], n_exp, e), FF, E, xb[t:t + 1])[0] for t, e in pairs])
    u_o = np.stack([oracle.mv_deq("Q4_K", _expert(raw["up"], n_exp, e), FF, E, xb[t:t + 1])[0] for t, e in pairs])
    act = oracle.round_bf16((g_o / (1.0 + np.exp(-g_o)) * u_o).astype(np.float32))
    y_o = np.stack([oracle.mv_deq("Q6_K", _expert(raw["down"], n_exp, e), E, FF, act[i:i + 1])[0]
                    for i, (_, e) in enumerate(pairs)])
    full = (y_o.reshape(L, k, E) * wts[:, :, None]).sum(1)
    err = float(oracle.rel_err_rows(out, full).max())
    assert err <= TOL_DEQ, err
    # stage by stage: gate and up launches
    fl = idx.reshape(-1)
    g = gate.matvec_tokens(idx, torch.from_numpy(x).cuda()).cpu().numpy()
    u = up.matvec_tokens(idx, torch.from_numpy(x).cuda()).cpu().numpy()
    assert oracle.rel_err_rows(g, g_o).max() <= TOL_DEQ
    assert oracle.rel_err_rows(u, u_o).max() <= TOL_DEQ
    y = down.matvec_je(fl, torch.from_numpy(act).cuda()).cpu().numpy()
    assert oracle.rel_err_rows(y, y_o).max() <= TOL_DEQ
