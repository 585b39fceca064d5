"""GPU parity of the layer mirrors: the block-format linear layer's dispatch by token count
(reference models/common.py:400-431) and the MoE expert layer of the Qwen3-30B-A3B-style
configuration (128 experts cut to 16 for time; gate/up 768x2048 Q4_K, down 2048x768 Q6_K, top-8
softmax routing renormalised), each stage against the oracle."""
import sys

import numpy as np
import pytest
import torch

from conftest import random_blocks

pytestmark = pytest.mark.gpu

BV = {"Q4_0": 32, "Q8_0": 32, "Q4_K": 256, "Q6_K": 256, "TQ2_0": 256, "IQ2_XXS": 256}


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def nmq():
    from ggufengine_amd import _native
    if not _native.available("cuda"):
        pytest.fail("libnmq.so not loaded or device is not gfx950 -- the HIP path must run here")
    return _native


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# (format, tokens M, branch of PackedLinear._rechnen expected)
DISPATCH = [("Q4_K", 1, "mmvq.mv"), ("Q4_K", 8, "mmvq.mv"), ("Q4_K", 9, "mmvq.mm"), ("Q4_K", 40, "mmvq.mm"),
            ("Q4_K", 120, "unpack"), ("Q6_K", 4, "mmvq.mv"), ("Q6_K", 8, "mmvq.mv"), ("Q6_K", 9, "mmvq.mm"),
            ("Q6_K", 17, "mmvq.mm"),
            ("TQ2_0", 1, "cudakern.mv"), ("TQ2_0", 5, "cudakern.mm"), ("TQ2_0", 17, "unpack"),
            ("IQ2_XXS", 1, "cudakern.mv"), ("IQ2_XXS", 16, "cudakern.mm"), ("Q8_0", 1, "cudakern.mv"),
            ("Q8_0", 8, "cudakern.mm"), ("Q8_0", 24, "unpack"), ("Q4_0", 1, "cudakern.mv"),
            ("Q4_0", 3, "cudakern.mm"), ("Q4_0", 20, "unpack")]


# long rows: (format, row length, tokens M, branch)
DISPATCH_LONG = [("Q6_K", 14336, 6, "mmvq.mv"), ("Q6_K", 14336, 9, "mmvq.mm"), ("Q4_K", 14336, 8, "mmvq.mv"),
                 ("Q4_K", 11008, 2, "mmvq.mm"), ("Q6_K", 11008, 4, "mmvq.mv"), ("Q6_K", 11008, 5, "mmvq.mm")]


@pytest.mark.parametrize("fmt,n_in,M,branch", DISPATCH_LONG)
def test_packed_linear_dispatch_long_rows(nmq, oracle, monkeypatch, fmt, n_in, M, branch):
    """PackedLinear on rows beyond 4096 values: the mat-vec kernels up to mmvq.mv_bis tokens (8 where the
    dense kernel splits the row into K ranges, otherwise 1 for Q4_K and 4 for Q6_K), the fp16 matrix
    cores above; results against the oracle."""
    from ggufengine_amd import mmvq, packed
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out = 96
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=93 + M)
    x = np.random.default_rng(94 + M).standard_normal((M, n_in)).astype(np.float32)
    taken = []
    for name in ("mv", "mm"):
        orig = getattr(mmvq, name)
        monkeypatch.setattr(mmvq, name, lambda *a, _o=orig, _n=f"mmvq.{name}", **k: (taken.append(_n), _o(*a, **k))[1])
    say("packed linear long rows", fmt, n_in, M, branch)
    lin = packed.PackedLinear(dev(raw), TYPE_ID[fmt], n_out, n_in, dtype=torch.float32)
    y = lin(dev(x)).cpu().numpy()
    assert taken and set(taken) == {branch}, taken
    err = oracle.rel_err_rows(y, oracle.mv_deq(fmt, raw, n_out, n_in, x))
    assert err.max() <= 1e-3, (fmt, n_in, M, branch, float(err.max()))


@pytest.mark.parametrize("fmt,M,branch", DISPATCH)
def test_packed_linear_dispatch(nmq, oracle, monkeypatch, fmt, M, branch):
    from ggufengine_amd import cudakern, mmvq, packed
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = 96, 1024
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=91 + M)
    rng = np.random.default_rng(92 + M)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    b = rng.standard_normal(n_out).astype(np.float32)
    taken = []
    for mod, name in ((mmvq, "mv"), (mmvq, "mm"), (cudakern, "mv"), (cudakern, "mm")):
        orig = getattr(mod, name)
        monkeypatch.setattr(mod, name, lambda *a, _o=orig, _n=f"{mod.__name__.split('.')[-1]}.{name}", **k:
                            (taken.append(_n), _o(*a, **k))[1])
    orig_unpack = packed.unpack
    monkeypatch.setattr(packed, "unpack", lambda *a, **k: (taken.append("unpack"), orig_unpack(*a, **k))[1])
    say("packed linear", fmt, M, branch)
    lin = packed.PackedLinear(dev(raw), TYPE_ID[fmt], n_out, n_in, bias=dev(b), dtype=torch.float32)
    y = lin(dev(x)).cpu().numpy()
    assert y.shape == (M, n_out)
    assert taken and set(taken) == {branch}, taken
    if branch == "unpack":
        w = oracle.round_bf16(oracle.dequant(fmt, raw)).reshape(n_out, n_in).astype(np.float64)
        ref = x.astype(np.float64) @ w.T
        tol = 1e-5
    else:
        xin = x if branch.startswith("mmvq") else oracle.round_bf16(x)
        ref = oracle.mv_deq(fmt, raw, n_out, n_in, xin)
        tol = 1e-3
    err = oracle.rel_err_rows(y - b, ref)
    assert err.max() <= tol, (fmt, M, branch, float(err.max()))


def _expert_rows(raw, fmt, n_exp, n_out, n_in, e):
    per = raw.size // n_exp
    return raw[e * per:(e + 1) * per]


@pytest.mark.parametrize("L", [1, 4])
def test_moe_layer_stages(nmq, oracle, L):
    from ggufengine_amd import experts
    n_exp, k, E, FF = 16, 8, 2048, 768
    g_raw = random_blocks("Q4_K", n_exp * FF * E // 256, seed=81)
    u_raw = random_blocks("Q4_K", n_exp * FF * E // 256, seed=82)
    d_raw = random_blocks("Q6_K", n_exp * E * FF // 256, seed=83)
    gate = experts.PackedExperts(dev(g_raw), 12, n_exp, FF, E)
    up = experts.PackedExperts(dev(u_raw), 12, n_exp, FF, E)
    down = experts.PackedExperts(dev(d_raw), 14, n_exp, E, FF)
    layer = experts.Experten(gate, up, down)
    rng = np.random.Generator(np.random.PCG64(42 + L))
    logits = rng.standard_normal((L, n_exp)).astype(np.float32)
    x = rng.standard_normal((L, E)).astype(np.float32)
    idx, w = experts.auswahl(dev(logits), k)
    say("moe layer", L)
    out = layer(dev(x), idx, w).cpu().numpy()
    assert out.shape == (L, E)

    ids = idx.cpu().numpy()
    wts = w.cpu().numpy().astype(np.float64)
    xb = oracle.round_bf16(x)
    # stage 1: gate and up on each token's input, every (token, slot)
    if L == 1:
        g = gate.matvec(idx[0], dev(x[0])).cpu().numpy()
        u = up.matvec(idx[0], dev(x[0])).cpu().numpy()
    else:
        g = gate.matvec_tokens(idx, dev(x)).cpu().numpy()
        u = up.matvec_tokens(idx, dev(x)).cpu().numpy()
    pairs = [(t, j, int(ids[t, j])) for t in range(L) for j in range(k)]
    g_ref = np.stack([oracle.mv_deq("Q4_K", _expert_rows(g_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
                      for t, _, e in pairs])
    u_ref = np.stack([oracle.mv_deq("Q4_K", _expert_rows(u_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
                      for t, _, e in pairs])
    assert oracle.rel_err_rows(g, g_ref).max() <= 1e-3
    assert oracle.rel_err_rows(u, u_ref).max() <= 1e-3
    # stage 2: down on each slot's own activation silu(g) * u (ours, rounded to bf16 as the kernel's input)
    act = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    y = down.matvec_je(idx.reshape(-1), dev(act)).cpu().numpy()
    ab = oracle.round_bf16(act)
    y_ref = np.stack([oracle.mv_deq("Q6_K", _expert_rows(d_raw, "Q6_K", n_exp, E, FF, e), E, FF, ab[i:i + 1])[0]
                      for i, (_, _, e) in enumerate(pairs)])
    assert oracle.rel_err_rows(y, y_ref).max() <= 1e-3
    # stage 3: the layer (its own fused silu * up: exp may differ from torch's by an ulp, which can move
    # a bf16-rounded activation by one step) against the combine of the stage outputs above
    comb = (y.astype(np.float64).reshape(L, k, E) * wts[:, :, None]).sum(1)
    assert oracle.rel_err_rows(out, comb).max() <= 1e-3
    # end to end against the oracle chain (dequantised weights all the way)
    g_o, u_o = g_ref, u_ref
    act_o = g_o / (1.0 + np.exp(-g_o)) * u_o
    y_o = np.stack([oracle.mv_deq("Q6_K", _expert_rows(d_raw, "Q6_K", n_exp, E, FF, e), E, FF,
                                  oracle.round_bf16(act_o[i:i + 1].astype(np.float32)))[0]
                    for i, (_, _, e) in enumerate(pairs)])
    full = (y_o.reshape(L, k, E) * wts[:, :, None]).sum(1)
    assert oracle.rel_err_rows(out, full).max() <= 2e-3


# ---- fused entry points of the expert layer --------------------------------------------------------------

def _eingang_dev(n):
    from ggufengine_amd import mmvq
    return mmvq.Eingang(n=n, device=torch.device("cuda"))


def test_quant_rounds_to_bf16_first(nmq, oracle):
    rng = np.random.default_rng(101)
    x = (rng.standard_normal(32 * 500) * 3).astype(np.float32)
    x[:32] = 0.0
    xt = dev(x)
    a, b = _eingang_dev(x.size), _eingang_dev(x.size)
    say("quant mode 2")
    nmq.check(nmq.lib().nmq_quant_q8(xt.data_ptr(), 2, a.xq.data_ptr(), a.xq2.data_ptr(), a.xd.data_ptr(),
                                     a.xs.data_ptr(), x.size, nmq.stream_ptr()))
    xb = xt.to(torch.bfloat16)
    nmq.check(nmq.lib().nmq_quant_q8(xb.data_ptr(), 0, b.xq.data_ptr(), b.xq2.data_ptr(), b.xd.data_ptr(),
                                     b.xs.data_ptr(), x.size, nmq.stream_ptr()))
    torch.cuda.synchronize()
    ref = oracle.quant_q8(oracle.round_bf16(x))
    for name, ta, tb, r in zip(("xq", "xq2", "xd", "xs"), (a.xq, a.xq2, a.xd, a.xs), (b.xq, b.xq2, b.xd, b.xs), ref):
        assert torch.equal(ta, tb), name
        assert np.array_equal(ta.cpu().numpy().view(np.uint8), np.ascontiguousarray(r).view(np.uint8)), name


def test_silu_mul_quant(nmq, oracle):
    rng = np.random.default_rng(102)
    n = 32 * 800
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 2).astype(np.float32)
    g[:32] = 0.0                       # a zero group (silu(0) = 0)
    e = _eingang_dev(n)
    say("silu_mul_quant")
    g_d = dev(g)  # kept alive until the launch has run
    u_d = dev(u)  # kept alive until the launch has run
    nmq.check(nmq.lib().nmq_silu_mul_quant(g_d.data_ptr(), u_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                           e.xd.data_ptr(), e.xs.data_ptr(), n, nmq.stream_ptr()))
    torch.cuda.synchronize()
    act = oracle.round_bf16((g / (np.float32(1) + np.exp(-g, dtype=np.float32)) * u).astype(np.float32))
    xq, xq2, xd, xs = (t.cpu().numpy() for t in (e.xq, e.xq2, e.xd, e.xs))
    rxq, rxq2, rxd, rxs = oracle.quant_q8(act)
    # the activation the kernel quantised, reconstructed, against the restated one: within the two-stage
    # resolution plus one bf16 step (expf here and numpy's exp may differ in the last bit)
    d = np.repeat(xd, 32).astype(np.float64)
    rec = xq * d + xq2 * d / 254.0
    step = np.abs(act.astype(np.float64)) * 2.0 ** -8
    assert np.all(np.abs(rec - act) <= d / 508.0 + step + 1e-30)
    # and bit for bit in every group whose bf16 activations the device's expf cannot move: the fp32 value
    # silu(g) * u here and on the device differ by a few ulp at most (expf against numpy's exp, then the
    # correctly rounded division and product), so a group whose values all round to the same bf16 value
    # anywhere within 4 ulp of numpy's must match exactly
    pre = (g / (np.float32(1) + np.exp(-g, dtype=np.float32)) * u).astype(np.float32)
    lo, hi = pre.copy(), pre.copy()
    for _ in range(4):
        lo = np.nextafter(lo, np.float32(-np.inf))
        hi = np.nextafter(hi, np.float32(np.inf))
    fixed = ~(oracle.round_bf16(lo) != oracle.round_bf16(hi)).reshape(-1, 32).any(1)
    same = (np.all((xq == rxq).reshape(-1, 32), 1) & np.all((xq2 == rxq2).reshape(-1, 32), 1) & (xd == rxd) & (xs == rxs))
    assert fixed.mean() >= 0.99, fixed.mean()
    assert np.all(same[fixed]), np.flatnonzero(fixed & ~same)
    assert np.all(xq[:32] == 0) and xd[0] == 0.0


def _quant_matches(oracle, e, v):
    """The Eingang e is, bit for bit, the two-stage input of the fp32 values v."""
    got = [t.cpu().numpy() for t in (e.xq, e.xq2, e.xd, e.xs)]
    for a, b in zip(got, oracle.quant_q8(v)):
        assert np.array_equal(a, b)


# (n, with rest, rs): n % 4096 == 0 takes the four-values-per-lane first pass
NORM = [(4096, False, 1.0), (4096, True, 1.0), (14336, True, 0.5), (2112, False, 1.0), (2112, True, 0.25),
        (65536, True, 1.0), (32, False, 1.0)]


@pytest.mark.parametrize("n,with_rest,rs", NORM)
def test_norm_q8(nmq, oracle, n, with_rest, rs):
    """mmvq.norm_q8 (reference mmvq.py:102-120, 951-961): the new h bit for bit, xn within 2e-6 of the
    fp64 RMS norm (per row, max |err| / max |xn|), its Eingang bit for bit the quantisation of xn."""
    from ggufengine_amd import mmvq
    rng = np.random.default_rng(120 + n)
    h = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32) if with_rest else None
    eps = 1e-5
    say("norm_q8", n, with_rest, rs)
    h_d, w_d = dev(h), dev(w)
    r_d = dev(r) if with_rest else None
    xn, e, hn = mmvq.norm_q8(h_d, w_d, eps, rest=r_d, rs=rs)
    torch.cuda.synchronize()
    v, ref = oracle.norm_row(h, w, eps, r=r, rs=rs)
    if with_rest:
        assert hn.data_ptr() != h_d.data_ptr()
        assert np.array_equal(hn.cpu().numpy(), v)
    else:
        assert hn is h_d
    xn_np = xn.cpu().numpy()
    assert oracle.rel_err_rows(xn_np, ref).max() <= 2e-6
    _quant_matches(oracle, e, xn_np)


def test_norm_q8_feeds_mv(nmq, oracle):
    """The Eingang of norm_q8 read by a mat-vec: equal to quantising the returned xn separately."""
    from ggufengine_amd import mmvq
    n_out, n = 256, 4096
    rng = np.random.default_rng(130)
    raw_d = dev(random_blocks("Q4_K", n_out * n // 256, seed=131))
    h_d = dev(rng.standard_normal(n).astype(np.float32))
    w_d = dev(np.ones(n, np.float32))
    say("norm_q8 -> mv")
    xn, e, _ = mmvq.norm_q8(h_d, w_d, 1e-6)
    y1 = mmvq.mv("Q4_K", raw_d, e, n_out, n)
    y2 = mmvq.mv("Q4_K", raw_d, xn, n_out, n)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


# (n, gelu, with u)
AKT = [(14336, False, True), (14336, True, True), (2048, False, False), (2048, True, False), (96, True, True)]


@pytest.mark.parametrize("n,gelu,with_u", AKT)
def test_akt_q8(nmq, oracle, n, gelu, with_u):
    """mmvq.akt_q8 (reference mmvq.py:122-133, 964-971): a within 1e-6 of the fp64 activation (per row,
    max |err| / max |a|), its Eingang bit for bit the quantisation of a; zero groups stay zero."""
    from ggufengine_amd import mmvq
    rng = np.random.default_rng(140 + n + gelu)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:32] = 0.0
    u = (rng.standard_normal(n) * 2).astype(np.float32) if with_u else None
    say("akt_q8", n, gelu, with_u)
    g_d = dev(g)
    u_d = dev(u) if with_u else None
    a, e = mmvq.akt_q8(g_d, u_d, gelu)
    torch.cuda.synchronize()
    a_np = a.cpu().numpy()
    assert oracle.rel_err_rows(a_np, oracle.akt(g, u, gelu)).max() <= 1e-6
    assert np.all(a_np[:32] == 0.0)
    _quant_matches(oracle, e, a_np)


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "IQ2_XXS"])
def test_mv_experts2_matches_two_launches(nmq, fmt):
    from ggufengine_amd.gguf_types import TYPE_ID
    n_exp, n_out, n_in, L, k = 12, 160, 2048, 3, 4
    a = dev(random_blocks(fmt, n_exp * n_out * n_in // 256, seed=111))
    b = dev(random_blocks(fmt, n_exp * n_out * n_in // 256, seed=112))
    per = a.numel() // n_exp
    ids = torch.tensor(np.random.default_rng(113).integers(0, n_exp, L * k), dtype=torch.int64, device="cuda")
    x = dev(np.random.default_rng(114).standard_normal((L, n_in)).astype(np.float32))
    from ggufengine_amd import mmvq
    e = mmvq.Eingang(x)
    args = (e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k)
    y2 = torch.full((2 * L * k, n_out), float("nan"), device="cuda")
    ya = torch.empty(L * k, n_out, device="cuda")
    yb = torch.empty(L * k, n_out, device="cuda")
    say("mv_experts2", fmt)
    Lb = nmq.lib()
    nmq.check(Lb.nmq_mv_experts2(TYPE_ID[fmt], a.data_ptr(), b.data_ptr(), ids.data_ptr(), L * k, per, *args,
                                 y2.data_ptr(), n_out, n_in, nmq.stream_ptr()))
    nmq.check(Lb.nmq_mv_experts(TYPE_ID[fmt], a.data_ptr(), ids.data_ptr(), L * k, per, *args, ya.data_ptr(), n_out,
                                n_in, nmq.stream_ptr()))
    nmq.check(Lb.nmq_mv_experts(TYPE_ID[fmt], b.data_ptr(), ids.data_ptr(), L * k, per, *args, yb.data_ptr(), n_out,
                                n_in, nmq.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(y2[:L * k], ya) and torch.equal(y2[L * k:], yb)


def test_moe_combine(nmq):
    rng = np.random.default_rng(121)
    L, k, E = 4, 8, 2048
    y = rng.standard_normal((L * k, E)).astype(np.float32)
    w = rng.random((L, k)).astype(np.float32)
    out = torch.full((L, E), float("nan"), device="cuda")
    say("moe_combine")
    y_d = dev(y)  # kept alive until the launch has run
    w_d = dev(w)  # kept alive until the launch has run
    nmq.check(nmq.lib().nmq_moe_combine(y_d.data_ptr(), w_d.data_ptr(), L, k, E, out.data_ptr(),
                                        nmq.stream_ptr()))
    torch.cuda.synchronize()
    ref = (y.astype(np.float64).reshape(L, k, E) * w.astype(np.float64)[:, :, None]).sum(1)
    assert np.max(np.abs(out.cpu().numpy() - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("L", [1, 4])
def test_expert_layer_three_launches_equal_five(nmq, L):
    """Experten: the three-launch layer (inputs quantised inside the gathered launches) equals, bit for
    bit, the layer with its two input quantisations as launches of their own."""
    from ggufengine_amd import experts
    n_exp, k, E, FF = 16, 8, 2048, 768
    gate = experts.PackedExperts(dev(random_blocks("Q4_K", n_exp * FF * E // 256, seed=131)), 12, n_exp, FF, E)
    up = experts.PackedExperts(dev(random_blocks("Q4_K", n_exp * FF * E // 256, seed=132)), 12, n_exp, FF, E)
    down = experts.PackedExperts(dev(random_blocks("Q6_K", n_exp * E * FF // 256, seed=133)), 14, n_exp, E, FF)
    layer = experts.Experten(gate, up, down)
    rng = np.random.default_rng(134 + L)
    x = dev(rng.standard_normal((L, E)).astype(np.float32))
    idx, w = experts.auswahl(dev(rng.standard_normal((L, n_exp)).astype(np.float32)), k)
    say("expert layer 3 vs 5 launches", L)
    a = layer(x, idx, w)
    b = layer._aufgeteilt(x, idx, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _expert_parts(n_exp, E, FF, seed):
    from ggufengine_amd import experts
    g_raw = random_blocks("Q4_K", n_exp * FF * E // 256, seed=seed)
    u_raw = random_blocks("Q4_K", n_exp * FF * E // 256, seed=seed + 1)
    d_raw = random_blocks("Q6_K", n_exp * E * FF // 256, seed=seed + 2)
    gu_raw = np.concatenate([g_raw.reshape(n_exp, -1), u_raw.reshape(n_exp, -1)], axis=1).reshape(-1)
    P = experts.PackedExperts
    return (g_raw, u_raw, d_raw, P(dev(g_raw), 12, n_exp, FF, E), P(dev(u_raw), 12, n_exp, FF, E),
            P(dev(d_raw), 14, n_exp, E, FF), P(dev(gu_raw), 12, n_exp, 2 * FF, E))


@pytest.mark.parametrize("L", [1, 4])
def test_expert_layer_fused_gate_up_tensor(nmq, L):
    """Experten on one [gate | up] tensor (2*FF rows per expert, as GGUF's ffn_gate_up_exps) equals the layer
    on separate gate and up tensors bit for bit, in the two-launch and the five-launch forms."""
    from ggufengine_amd import experts
    n_exp, k, E, FF = 12, 8, 2048, 768
    _, _, _, G, U, D, GU = _expert_parts(n_exp, E, FF, 601)
    sep = experts.Experten(G, U, D)
    fus = experts.Experten(None, None, D, gate_up=GU)
    rng = np.random.default_rng(602 + L)
    x = dev(rng.standard_normal((L, E)).astype(np.float32))
    idx, w = experts.auswahl(dev(rng.standard_normal((L, n_exp)).astype(np.float32)), k)
    say("expert layer fused gate_up", L)
    a, b = sep(x, idx, w), fus(x, idx, w)
    c, d = sep._aufgeteilt(x, idx, w), fus._aufgeteilt(x, idx, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)


@pytest.mark.parametrize("form", ["bias_gelu", "no_gate", "fused_bias_glu"])
def test_expert_layer_general_forms(nmq, oracle, form):
    """The layer's other forms (reference moe.py:205-277): per-expert biases with the tanh-gelu activation;
    up alone (act(up)); the fused [gate | up] tensor with its bias and a custom glu.  Against the oracle:
    gate/up products on the tokens' bf16 inputs, biases, the activation in fp64 rounded to bf16 (the down
    launch's input), down products plus bias, the weighted sum; max relative error per row <= 2e-3."""
    from ggufengine_amd import experts
    n_exp, k, E, FF, L = 10, 4, 1024, 512, 3
    g_raw, u_raw, d_raw, G, U, D, GU = _expert_parts(n_exp, E, FF, 611)
    rng = np.random.default_rng(612)
    bias = {n: (rng.standard_normal((n_exp, wd)) * 0.05).astype(np.float32)
            for n, wd in (("gate", FF), ("up", FF), ("gate_up", 2 * FF), ("down", E))}
    glu_t = lambda g, u: g * torch.sigmoid(1.702 * g) * (u + 1.0)
    glu_n = lambda g, u: g / (1.0 + np.exp(-1.702 * g)) * (u + 1.0)
    if form == "bias_gelu":
        layer = experts.Experten(G, U, D, bias={n: dev(bias[n]) for n in ("gate", "up", "down")}, akt="gelu")
    elif form == "no_gate":
        layer = experts.Experten(None, U, D)
    else:
        layer = experts.Experten(None, None, D, gate_up=GU, bias={n: dev(bias[n]) for n in ("gate_up", "down")},
                                 glu=glu_t)
    x = rng.standard_normal((L, E)).astype(np.float32)
    idx, w = experts.auswahl(dev(rng.standard_normal((L, n_exp)).astype(np.float32)), k)
    say("expert layer form", form)
    out = layer(dev(x), idx, w).cpu().numpy()
    ids, wts = idx.cpu().numpy(), w.cpu().numpy().astype(np.float64)
    xb = oracle.round_bf16(x)
    ref = np.zeros((L, E))
    for t in range(L):
        for j in range(k):
            e = int(ids[t, j])
            g = oracle.mv_deq("Q4_K", _expert_rows(g_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
            u = oracle.mv_deq("Q4_K", _expert_rows(u_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
            if form == "bias_gelu":
                a = oracle.akt(g + bias["gate"][e], u + bias["up"][e], gelu=True)
            elif form == "no_gate":
                a = oracle.akt(u)
            else:
                a = glu_n(g + bias["gate_up"][e, :FF], u + bias["gate_up"][e, FF:])
            ab = oracle.round_bf16(a.astype(np.float32))
            y = oracle.mv_deq("Q6_K", _expert_rows(d_raw, "Q6_K", n_exp, E, FF, e), E, FF, ab[None])[0]
            if form != "no_gate":
                y = y + bias["down"][e]
            ref[t] += wts[t, j] * y
    assert oracle.rel_err_rows(out, ref).max() <= 2e-3


@pytest.mark.parametrize("form", ["silu", "fused_bias_gelu"])
def test_expert_layer_many_tokens_sorted(nmq, oracle, form):
    """Many tokens (at least SORTIERT_AB pairs per expert): the (token, slot) pairs sorted by expert, each
    used expert's rows as one matrix call (1 to 20 rows here: mat-vec, matrix-core and unpack routes), put
    back and summed in (token, slot) order; against the oracle chain, max relative error per row <= 2e-3."""
    from ggufengine_amd import experts
    n_exp, k, E, FF, L = 6, 2, 1024, 512, 40
    g_raw, u_raw, d_raw, G, U, D, GU = _expert_parts(n_exp, E, FF, 621)
    rng = np.random.default_rng(622)
    bias = {n: (rng.standard_normal((n_exp, wd)) * 0.05).astype(np.float32) for n, wd in (("gate_up", 2 * FF), ("down", E))}
    if form == "silu":
        layer = experts.Experten(G, U, D)
    else:
        layer = experts.Experten(None, None, D, gate_up=GU, bias={n: dev(b) for n, b in bias.items()}, akt="gelu")
    x = rng.standard_normal((L, E)).astype(np.float32)
    logits = rng.standard_normal((L, n_exp)).astype(np.float32)
    logits[:, 0] += 3.0                       # expert 0 takes most tokens, others few
    idx, w = experts.auswahl(dev(logits), k)
    assert idx.numel() >= experts.SORTIERT_AB * n_exp
    say("expert layer sorted", form)
    out = layer(dev(x), idx, w).cpu().numpy()
    ids, wts = idx.cpu().numpy(), w.cpu().numpy().astype(np.float64)
    xb = oracle.round_bf16(x)
    ref = np.zeros((L, E))
    for t in range(L):
        for j in range(k):
            e = int(ids[t, j])
            g = oracle.mv_deq("Q4_K", _expert_rows(g_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
            u = oracle.mv_deq("Q4_K", _expert_rows(u_raw, "Q4_K", n_exp, FF, E, e), FF, E, xb[t:t + 1])[0]
            if form == "silu":
                a = oracle.akt(g, u)
            else:
                a = oracle.akt(g + bias["gate_up"][e, :FF], u + bias["gate_up"][e, FF:], gelu=True)
            ab = oracle.round_bf16(a.astype(np.float32))
            y = oracle.mv_deq("Q6_K", _expert_rows(d_raw, "Q6_K", n_exp, E, FF, e), E, FF, ab[None])[0]
            if form != "silu":
                y = y + bias["down"][e]
            ref[t] += wts[t, j] * y
    assert oracle.rel_err_rows(out, ref).max() <= 2e-3


def test_llama3_8b_layer_full_size(nmq, oracle):
    """The mat-vecs of a full Llama-3-8B decoder layer at batch 1 (q, k, v, o, gate, up Q4_K; down Q6_K
    4096x14336), weights ~N(0, 0.02) quantised by the library's encoders, run as the layer runs them
    (q/k/v and gate/up each in one launch on the fp32 input, o on its own, down through an Eingang):
    every output within the parity bar of the oracle (dequantise + fp64 matmul) and within 2e-5 of the
    oracle's integer decomposition."""
    import os
    from ggufengine_amd import encode, mmvq
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    spec = {"q": ("Q4_K", 4096, 4096, 21), "k": ("Q4_K", 1024, 4096, 22), "v": ("Q4_K", 1024, 4096, 23),
            "o": ("Q4_K", 4096, 4096, 24), "gate": ("Q4_K", 14336, 4096, 25), "up": ("Q4_K", 14336, 4096, 26),
            "down": ("Q6_K", 4096, 14336, 27)}
    raw = {}
    for n, (f, r, c, sd) in spec.items():
        w = np.random.Generator(np.random.PCG64(sd)).standard_normal(r * c, dtype=np.float32) * np.float32(0.02)
        raw[n] = encode.encode(f, w, threads=threads)
    xs = {n: np.random.Generator(np.random.PCG64(sd)).standard_normal(c, dtype=np.float32)
          for n, (c, sd) in {"x_attn": (4096, 28), "attn_out": (4096, 30), "x_ffn": (4096, 31), "act": (14336, 29)}.items()}
    wd = {n: dev(r) for n, r in raw.items()}
    xd = {n: dev(x) for n, x in xs.items()}
    say("llama3-8b layer")
    y = dict(zip(("q", "k", "v"), mmvq.mv_mehrere("Q4_K", [wd["q"], wd["k"], wd["v"]], xd["x_attn"],
                                                  [4096, 1024, 1024], 4096)))
    y["o"] = mmvq.mv("Q4_K", wd["o"], xd["attn_out"], 4096, 4096)
    y.update(zip(("gate", "up"), mmvq.mv_mehrere("Q4_K", [wd["gate"], wd["up"]], xd["x_ffn"], [14336, 14336], 4096)))
    y["down"] = mmvq.mv("Q6_K", wd["down"], xd["act"], 4096, 14336)
    torch.cuda.synchronize()
    inp = {"q": "x_attn", "k": "x_attn", "v": "x_attn", "o": "attn_out", "gate": "x_ffn", "up": "x_ffn", "down": "act"}
    for n, (f, r, c, _) in spec.items():
        x = xs[inp[n]][None]
        got = y[n].cpu().numpy()[None]
        err = oracle.rel_err_rows(got, oracle.mv_deq(f, raw[n], r, c, x)).max()
        assert err <= 1e-3, (n, err)
        err_i = oracle.rel_err_rows(got, oracle.mv_int(f, raw[n], r, c, *oracle.quant_q8(x))).max()
        assert err_i <= 2e-5, (n, err_i)


def test_gguf_upload_and_matvec(nmq, oracle, tmp_path):
    """A GGUF file with Llama-named Q4_K / Q6_K / F32 tensors (the library's writer and encoder): the
    Uploader moves each tensor's bytes through its ring of pinned buffers unchanged (chunks of 300 KB,
    so the ring of 4 wraps), and the mat-vecs on the uploaded blocks match the oracle on the file's
    bytes."""
    from ggufengine_amd import encode, gguf as G, mmvq
    rng = np.random.default_rng(131)
    gate = encode.encode("Q4_K", (rng.standard_normal(512 * 4096) * 0.02).astype(np.float32), threads=8)
    down = encode.encode("Q6_K", (rng.standard_normal(256 * 1024) * 0.02).astype(np.float32), threads=8)
    norm = rng.standard_normal(4096).astype(np.float32)
    path = tmp_path / "blk.gguf"
    G.write_gguf(path, {"general.architecture": (G.T_STRING, "llama"), "llama.block_count": (G.T_UINT32, 1)},
                 [("blk.0.attn_norm.weight", (4096,), 0, norm.tobytes()),
                  ("blk.0.ffn_gate.weight", (4096, 512), 12, gate.tobytes()),
                  ("blk.0.ffn_down.weight", (1024, 256), 14, down.tobytes())])
    say("gguf upload")
    up = G.Uploader("cuda")
    up.CHUNK = 300_000
    with G.GGUFFile(path) as gf:
        g_dev = G.load_raw(gf, "blk.0.ffn_gate.weight", "cuda", up)
        d_dev = G.load_raw(gf, "blk.0.ffn_down.weight", "cuda", up)
        n_dev = G.load_raw(gf, "blk.0.attn_norm.weight", "cuda", up)
        torch.cuda.synchronize()
        assert np.array_equal(g_dev.cpu().numpy(), gate) and np.array_equal(d_dev.cpu().numpy(), down)
        assert np.array_equal(n_dev.cpu().numpy().view(np.float32), norm)
        for raw, raw_np, fmt, n_out, n_in in ((g_dev, gate, "Q4_K", 512, 4096), (d_dev, down, "Q6_K", 256, 1024)):
            x = rng.standard_normal(n_in).astype(np.float32)
            y = mmvq.mv(fmt, raw, torch.from_numpy(x).cuda(), n_out, n_in).cpu().numpy()
            err = oracle.rel_err_rows(y[None], oracle.mv_deq(fmt, raw_np, n_out, n_in, x[None]))
            assert err.max() <= 1e-3, (fmt, float(err.max()))
        cpu = G.load_raw(gf, "blk.0.ffn_gate.weight", "cpu")
        assert np.array_equal(cpu.numpy(), gate)
        del cpu


def test_experts_in_pinned_ram_with_vram_slots(nmq, oracle):
    """Experts kept in pinned RAM (hostmem.empty + abbilden: hipHostMalloc, mapped at the same address)
    are read by the gathered kernels over PCIe; ExpertenLager puts the most used ones into VRAM slots
    behind an address table.  Every result equals the same experts in VRAM bit for bit: directly from
    RAM, through the slots before and after re-sorting, and from a HIP graph replayed across
    re-sorts (the graph reads the table on the device)."""
    from ggufengine_amd import experts, hostmem
    n_exp, n_out, n_in = 16, 256, 1024
    raw = random_blocks("Q4_K", n_exp * n_out * n_in // 256, seed=141)
    say("experts in pinned RAM")
    host = hostmem.empty(raw.size, "cuda")
    host.numpy()[:] = raw
    mapped = hostmem.abbilden(host, "cuda")
    assert mapped.is_cuda and mapped.data_ptr() == host.data_ptr() and hostmem.abgebildet(mapped)
    in_ram = experts.PackedExperts(mapped, 12, n_exp, n_out, n_in)
    in_vram = experts.PackedExperts(dev(raw), 12, n_exp, n_out, n_in)
    rng = np.random.default_rng(142)
    x = torch.from_numpy(rng.standard_normal(n_in).astype(np.float32)).cuda()
    ids = torch.tensor([3, 7, 0, 15, 9, 9, 1, 12], dtype=torch.int64, device="cuda")
    want = in_vram.matvec(ids, x)
    assert torch.equal(in_ram.matvec(ids, x), want)
    ref = oracle.mv_deq("Q4_K", raw.reshape(n_exp, -1)[ids.cpu().numpy()].ravel(), 8 * n_out, n_in,
                        oracle.round_bf16(x.cpu().numpy())[None])
    err = oracle.rel_err_rows(want.cpu().numpy(), ref.reshape(8, n_out))
    assert err.max() <= 1e-3
    lager = experts.ExpertenLager([in_ram], plaetze=4, device="cuda")
    assert lager.belegt == [0, 1, 2, 3]
    assert torch.equal(in_ram.matvec(ids, x), want)
    for _ in range(3):
        lager.zaehlen(torch.tensor([9, 12, 15, 7, 9], device="cuda"))
    assert lager.umsortieren() == 4 and sorted(lager.belegt) == [7, 9, 12, 15]
    assert lager.treffer() == 1.0
    assert torch.equal(in_ram.matvec(ids, x), want)
    # a graph of the gathered launch, replayed across re-sorts
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        in_ram.matvec(ids, x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = in_ram.matvec(ids, x)
    for hot in ([0, 1, 2, 3], [3, 7, 0, 15], [12, 1, 9, 0]):
        for _ in range(2):
            lager.zaehlen(torch.tensor(hot, device="cuda"))
        lager.umsortieren()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), hot
        assert torch.equal(in_ram.matvec(ids, x), want)   # eager work between replays
    del g, out, lager, in_ram, mapped, host
    import gc
    gc.collect()
    assert hostmem.pending() >= 1
    hostmem.flush()
    assert hostmem.pending() == 0


def test_band_refuses_to_overwrite_a_matrix_in_use():
    """A copy into a slot whose matrix holen() handed out and fertig() has not released raises instead
    of racing with that matrix's computation: within a pass (the ring wraps onto it) and at the start
    of the next pass.  After fertig() the same calls go through and return the right bytes."""
    from ggufengine_amd import band
    fl = band.Fliessband("cuda")
    src = [torch.full((1000 + i,), i, dtype=torch.uint8, device="cuda") for i in range(6)]
    for t in src:
        fl.anmelden(t)
    say("band guard")
    a = fl.holen(0)
    with pytest.raises(RuntimeError, match="overwrite matrix 0"):
        fl.holen(1)                          # queues matrix 4 into slot 0
    fl.fertig(0)
    for nr in range(1, 6):
        got = fl.holen(nr)
        assert got.numel() == 1000 + nr and bool((got == nr).all())
        if nr < 5:
            fl.fertig(nr)
    with pytest.raises(RuntimeError, match=r"handed out"):
        fl.holen(0)                          # a new pass while matrix 5 is still out
    fl.fertig(5)
    assert bool((fl.holen(0) == 0).all()) and a.numel() == 1000
    fl.fertig(0)
    torch.cuda.synchronize()


def test_packed_linear_band_from_pinned_ram(nmq):
    """Layers whose weights live in pinned RAM, computed through a Fliessband (4 VRAM slots filled by
    whole-matrix copies a few layers ahead on a copy stream, ordered by events only): over several
    passes, eagerly and as a HIP graph replayed with eager passes between the replays, every output
    equals the same layers held in VRAM bit for bit.  Seven layers of two formats and sizes, so the
    ring wraps within a pass."""
    from ggufengine_amd import band, hostmem, packed
    specs = [("Q4_K", 12, 512, 1024), ("Q6_K", 14, 256, 2048), ("Q4_K", 12, 768, 1024), ("Q8_0", 8, 256, 1024),
             ("Q4_K", 12, 512, 2048), ("Q6_K", 14, 512, 1024), ("Q4_K", 12, 256, 1024)]
    fl = band.Fliessband("cuda")
    vram, ram, xs = [], [], []
    rng = np.random.default_rng(171)
    say("band layers", len(specs))
    for i, (fmt, tid, n_out, n_in) in enumerate(specs):
        raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=172 + i)
        vram.append(packed.PackedLinear(dev(raw), tid, n_out, n_in, dtype=torch.float32))
        host = hostmem.empty(raw.size, "cuda")
        host.numpy()[:] = raw
        lay = packed.PackedLinear(hostmem.abbilden(host, "cuda"), tid, n_out, n_in, dtype=torch.float32)
        assert lay.im_ram
        lay.band, lay.nr = fl, fl.anmelden(host)
        ram.append(lay)
        xs.append(dev(rng.standard_normal((1, n_in)).astype(np.float32)))
    want = [lay(x) for lay, x in zip(vram, xs)]

    def one_pass():
        return [lay(x) for lay, x in zip(ram, xs)]

    for _ in range(3):
        got = one_pass()
        torch.cuda.synchronize()
        for i, (g, w) in enumerate(zip(got, want)):
            assert torch.equal(g, w), i
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        one_pass()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = one_pass()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), (rep, i)
        got = one_pass()                          # eager work between the replays
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(got, want)):
            assert torch.equal(o, w), ("eager", rep, i)


@pytest.mark.parametrize("L", [1, 4])
def test_expert_layer_with_experts_in_pinned_ram(nmq, L):
    """The whole expert layer (Experten: gate and up in one launch, down, combine) with all three parts'
    experts in pinned RAM behind one ExpertenLager (4 VRAM slots per part, address tables read by the
    kernels): equal bit for bit to the layer on VRAM experts, before and after the slots are re-sorted."""
    from ggufengine_amd import experts, hostmem
    n_exp, k, E, FF = 16, 4, 1024, 512
    raws = [random_blocks("Q4_K", n_exp * FF * E // 256, seed=181), random_blocks("Q4_K", n_exp * FF * E // 256, seed=182),
            random_blocks("Q6_K", n_exp * E * FF // 256, seed=183)]
    shapes = [(12, FF, E), (12, FF, E), (14, E, FF)]

    def part(raw, shape, in_ram):
        t, n_out, n_in = shape
        if not in_ram:
            return experts.PackedExperts(dev(raw), t, n_exp, n_out, n_in)
        host = hostmem.empty(raw.size, "cuda")
        host.numpy()[:] = raw
        return experts.PackedExperts(hostmem.abbilden(host, "cuda"), t, n_exp, n_out, n_in)

    vram = experts.Experten(*[part(r, s, False) for r, s in zip(raws, shapes)])
    ram_parts = [part(r, s, True) for r, s in zip(raws, shapes)]
    ram = experts.Experten(*ram_parts)
    lager = experts.ExpertenLager(ram_parts, plaetze=4, device="cuda")
    rng = np.random.default_rng(184 + L)
    x = dev(rng.standard_normal((L, E)).astype(np.float32))
    idx, w = experts.auswahl(dev(rng.standard_normal((L, n_exp)).astype(np.float32)), k)
    say("expert layer in RAM", L)
    want = vram(x, idx, w)
    assert torch.equal(ram(x, idx, w), want)
    lager.zaehlen(idx)
    lager.umsortieren()
    assert torch.equal(ram(x, idx, w), want)


# ---- QuantLinear (the reference's "QLinear forward", qlinear.py:222-239) ------------------------------------

@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_0", "Q4_K", "Q6_K"])
@pytest.mark.parametrize("M", [1, 8, 64, 300])
def test_quant_linear_call(nmq, oracle, fmt, M):
    """QuantLinear.__call__: x cast to bf16, the route for M rows (mat-vec kernels, matrix cores, or the
    unpack to bf16 + GEMM at 300 rows), the result in bf16, the bias added in bf16.  Against dequantise +
    matmul in fp64 on the bf16-rounded x, with the bias: the bf16 output rounding (2^-9 relative) bounds
    the difference; tolerance 8e-3 of the row maximum."""
    from ggufengine_amd import qlinear
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = 320, 1024
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=201 + M)
    rng = np.random.default_rng(202 + M)
    x = rng.standard_normal((M, n_in)).astype(np.float32)
    b = (rng.standard_normal(n_out) * 0.5).astype(np.float32)
    say("QuantLinear", fmt, M)
    ql = qlinear.build_quant_linear(dev(raw), TYPE_ID[fmt], n_out, n_in, bias=dev(b))
    y = ql(dev(x).view(M, 1, n_in))
    assert y.dtype == torch.bfloat16 and y.shape == (M, 1, n_out)
    got = y.float().reshape(M, n_out).cpu().numpy()
    xb = oracle.round_bf16(x)
    ref = oracle.mv_deq(fmt, raw, n_out, n_in, xb) + oracle.round_bf16(b).astype(np.float64)
    err = oracle.rel_err_rows(got, ref)
    assert err.max() <= 8e-3, (fmt, M, ql.route(M), float(err.max()))
    # before the bf16 cast: the kernels' fp32 result on the same bf16 x within the mat-vec bar
    kind = ql.route(M)
    assert kind == {1: "mmvq.mv" if fmt in ("Q4_K", "Q6_K") else "cudakern.mv"}.get(M, kind)
    if kind != "unpack":
        f32 = ql._layer.forward_raw(dev(xb), ql._layer.raw, torch.float32).cpu().numpy()
        assert oracle.rel_err_rows(f32, ref - oracle.round_bf16(b)).max() <= 1e-3
    assert ql.bf16_weight().shape == (n_out, n_in)


def test_quant_linear_experts_as_packed_experts(nmq, oracle):
    """QuantLinear experts cut back to back out of one tensor (the reference loader's way) become one
    PackedExperts in place; the gathered kernel on them equals each expert's own QuantLinear call on the
    same bf16 input."""
    from ggufengine_amd import experts, qlinear
    n_exp, n_out, n_in = 6, 128, 1024
    raw = random_blocks("Q4_K", n_exp * n_out * n_in // 256, seed=211)
    whole = dev(raw)
    per = raw.size // n_exp
    qls = [qlinear.build_quant_linear(whole[e * per:(e + 1) * per], 12, n_out, n_in) for e in range(n_exp)]
    pe = experts.PackedExperts.aus_quantlinear(qls)
    assert pe.raw.data_ptr() == whole.data_ptr() and pe.n_exp == n_exp
    x = dev(np.random.default_rng(212).standard_normal(n_in).astype(np.float32))
    ids = torch.tensor([5, 0, 3, 3], device="cuda")
    say("QuantLinear experts")
    y = pe.matvec(ids, x)
    for j, e in enumerate(ids.tolist()):
        one = qls[e]._layer.forward_raw(x.to(torch.bfloat16).view(1, -1), qls[e]._layer.raw, torch.float32)
        assert torch.allclose(y[j], one[0], rtol=1e-6, atol=1e-6 * float(one.abs().max())), (j, e)
    # copied together when the experts are separate allocations
    pe2 = experts.PackedExperts.aus_quantlinear([qlinear.build_quant_linear(whole[e * per:(e + 1) * per].clone(), 12,
                                                                             n_out, n_in) for e in range(n_exp)])
    assert pe2.raw.data_ptr() != whole.data_ptr() and torch.equal(pe2.matvec(ids, x), y)
    # unpacked experts and one expert as a layer
    w = pe.weights(ids[:2])
    assert w.shape == (2, n_out, n_in)
    ref = oracle.round_bf16(oracle.dequant("Q4_K", raw.reshape(n_exp, -1)[5])).reshape(n_out, n_in)
    assert np.array_equal(w[0].float().cpu().numpy(), ref)
    one5 = pe[5](x.view(1, -1)).float().view(-1)
    assert torch.allclose(one5, y[0].to(torch.bfloat16).float(), rtol=1e-2, atol=1e-2 * float(y[0].abs().max()))


def test_band_slots_aligned_for_any_largest_source(nmq):
    """The largest source is a 5-row TQ2_0 matrix of 1320 bytes (not a multiple of 16); Q4_K matrices after
    it land in slots 1..3, which start at 256-byte multiples, and compute the VRAM results bit for bit."""
    from ggufengine_amd import band, hostmem, packed
    specs = [("TQ2_0", 35, 5, 1024), ("Q4_K", 12, 8, 256), ("Q4_K", 12, 4, 512), ("Q4_K", 12, 2, 1024),
             ("Q6_K", 14, 3, 512), ("Q4_K", 12, 6, 256)]
    fl = band.Fliessband("cuda")
    vram, ram, xs = [], [], []
    rng = np.random.default_rng(221)
    say("band alignment")
    for i, (fmt, tid, n_out, n_in) in enumerate(specs):
        raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=222 + i)
        vram.append(packed.PackedLinear(dev(raw), tid, n_out, n_in, dtype=torch.float32))
        host = hostmem.empty(raw.size, "cuda")
        host.numpy()[:] = raw
        lay = packed.PackedLinear(hostmem.abbilden(host, "cuda"), tid, n_out, n_in, dtype=torch.float32)
        lay.band, lay.nr = fl, fl.anmelden(host)
        ram.append(lay)
        xs.append(dev(rng.standard_normal((1, n_in)).astype(np.float32)))
    for _ in range(2):
        for i, (a, b, x) in enumerate(zip(ram, vram, xs)):
            assert torch.equal(a(x), b(x)), i
    torch.cuda.synchronize()
    assert all(s.data.data_ptr() % 256 == 0 for s in fl._slots)


def test_band_refuses_a_pass_split_across_a_capture(nmq):
    """A pass begun by eager calls cannot continue inside a graph capture (its queued copies are not part
    of the capture): holen raises before touching any stream, and the pass then finishes eagerly."""
    from ggufengine_amd import band
    fl = band.Fliessband("cuda")
    src = [torch.full((512,), i, dtype=torch.uint8, device="cuda") for i in range(3)]
    for t in src:
        fl.anmelden(t)
    say("band split pass")
    fl.holen(0)
    fl.fertig(0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="whole passes"):
        with torch.cuda.graph(g, stream=s):
            fl.holen(1)
    torch.cuda.current_stream().wait_stream(s)
    got = fl.holen(1)
    assert bool((got == 1).all())
    fl.fertig(1)
    torch.cuda.synchronize()



# ---- gate and up with the activation in one launch (nmq_moe_gate_up), down on its two-stage input ----------

def _gate_up_case(fmt, n_exp, FF, E, L, k, seed):
    from ggufengine_amd.gguf_types import TYPE_ID
    A = dev(random_blocks(fmt, n_exp * FF * E // BV[fmt], seed=seed))
    B = dev(random_blocks(fmt, n_exp * FF * E // BV[fmt], seed=seed + 1))
    rng = np.random.default_rng(seed + 2)
    ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
    x = dev(rng.standard_normal((L, E)).astype(np.float32))
    return TYPE_ID[fmt], A, B, A.numel() // n_exp, ids, x, rng


def _gate_up_two_launches(nmq, t, A, B, ids, per, x, mode, L, k, FF, E):
    """nmq_mv_experts_x (gate and up of every slot) followed by nmq_silu_mul_quant."""
    from ggufengine_amd import mmvq
    n = L * k
    gu = torch.full((2 * n, FF), float("nan"), device="cuda")
    Lb = nmq.lib()
    nmq.check(Lb.nmq_mv_experts_x(t, A.data_ptr(), B.data_ptr(), ids.data_ptr(), n, per, x.data_ptr(), mode, None, k,
                                  gu.data_ptr(), FF, E, nmq.stream_ptr()))
    a = mmvq.Eingang(n=n * FF, device=torch.device("cuda"))
    nmq.check(Lb.nmq_silu_mul_quant(gu.data_ptr(), gu[n:].data_ptr(), a.xq.data_ptr(), a.xq2.data_ptr(),
                                    a.xd.data_ptr(), a.xs.data_ptr(), n * FF, nmq.stream_ptr()))
    return a, gu


def _gate_up_fused(nmq, t, A, B, ids, per, x, mode, L, k, FF, E, a=None):
    from ggufengine_amd import mmvq
    n = L * k
    if a is None:
        a = mmvq.Eingang(n=n * FF, device=torch.device("cuda"))
        for b in (a.xq, a.xq2):
            b.fill_(77)
        for b in (a.xd, a.xs):
            b.fill_(float("nan"))
    nmq.check(nmq.lib().nmq_moe_gate_up(t, A.data_ptr(), B.data_ptr(), ids.data_ptr(), L, k, per, x.data_ptr(), mode,
                                        a.xq.data_ptr(), a.xq2.data_ptr(), a.xd.data_ptr(), a.xs.data_ptr(), FF, E,
                                        nmq.stream_ptr()))
    return a


def _same_input(a, b):
    return all(torch.equal(getattr(a, f), getattr(b, f)) for f in ("xq", "xq2", "xd", "xs"))


# (format, FF rows, E values per row, tokens L, slots k): T = 16, 32 and 64 lanes per row, every format
GATE_UP = [("Q4_K", 768, 2048, 1, 8), ("Q4_K", 768, 2048, 4, 8), ("Q4_K", 256, 1024, 3, 4), ("Q6_K", 512, 4096, 2, 2),
           ("Q8_0", 320, 2080, 2, 3), ("TQ2_0", 256, 1536, 1, 8), ("IQ2_XXS", 256, 2048, 2, 4), ("Q4_0", 288, 864, 5, 2)]


@pytest.mark.parametrize("rows", ["default", "fewer", "more"])
@pytest.mark.parametrize("fmt,FF,E,L,k", GATE_UP)
def test_moe_gate_up_equals_gathered_launch_and_activation(nmq, tune, fmt, FF, E, L, k, rows):
    """nmq_moe_gate_up (each workgroup: 32 rows of a slot's gate and up, then the activation and its
    two-stage input) equals nmq_mv_experts_x followed by nmq_silu_mul_quant bit for bit (xq, xq2, xd, xs),
    with either number of rows per team (the planner's choice, 2 or 4 -- 4 or 8 for rows over 2048 values)."""
    if rows != "default":
        tune(MOE_GU_RW=(2 if rows == "fewer" else 4) * (2 if E > 2048 else 1))
    t, A, B, per, ids, x, rng = _gate_up_case(fmt, 12, FF, E, L, k, 261 + FF + L)
    say("moe_gate_up", fmt, FF, E, L, k, rows)
    for mode in (nmq.X_F32_BF16, nmq.X_F32):
        want, _ = _gate_up_two_launches(nmq, t, A, B, ids, per, x, mode, L, k, FF, E)
        got = _gate_up_fused(nmq, t, A, B, ids, per, x, mode, L, k, FF, E)
        torch.cuda.synchronize()
        assert _same_input(got, want), (fmt, mode)
    xb = x.to(torch.bfloat16).contiguous()
    want, _ = _gate_up_two_launches(nmq, t, A, B, ids, per, xb, nmq.X_BF16, L, k, FF, E)
    got = _gate_up_fused(nmq, t, A, B, ids, per, xb, nmq.X_BF16, L, k, FF, E)
    torch.cuda.synchronize()
    assert _same_input(got, want), (fmt, "bf16")


def test_moe_gate_up_against_oracle(nmq, oracle):
    """nmq_moe_gate_up against the oracle: g and u of every slot from the oracle's integer path on the
    token's two-stage bf16 input, act = silu(g) * u in fp64; the launch's xd * (xq + xq2 / 254) is act
    within the bf16 rounding of the activation (2^-8 relative) plus the second stage's step (xd / 254)."""
    fmt, FF, E, L, k, n_exp = "Q4_K", 256, 2048, 2, 4, 6
    t, A, B, per, ids, x, rng = _gate_up_case(fmt, n_exp, FF, E, L, k, 271)
    say("moe_gate_up oracle")
    a = _gate_up_fused(nmq, t, A, B, ids, per, x, nmq.X_F32_BF16, L, k, FF, E)
    torch.cuda.synchronize()
    Ac, Bc, idc = A.cpu().numpy(), B.cpu().numpy(), ids.cpu().numpy()
    xd = a.xd.cpu().numpy().astype(np.float64)
    got = (np.repeat(xd, 32) * (a.xq.cpu().numpy() + a.xq2.cpu().numpy() / 254.0)).reshape(L * k, FF)
    step = np.repeat(xd, 32).reshape(L * k, FF) / 254.0
    for s in range(L * k):
        e = int(idc[s])
        q = oracle.quant_q8(oracle.round_bf16(x[s // k].cpu().numpy()))
        g = oracle.mv_int(fmt, _expert_rows(Ac, fmt, n_exp, FF, E, e), FF, E, *q)[0]
        u = oracle.mv_int(fmt, _expert_rows(Bc, fmt, n_exp, FF, E, e), FF, E, *q)[0]
        want = oracle.akt(g, u)
        tol = 2.0 ** -8 * np.abs(want) + step[s] + 1e-5 * np.abs(want).max()
        assert np.all(np.abs(got[s] - want) <= tol), s


def test_moe_down_q8_equals_value_input(nmq):
    """nmq_moe_down_q8 on the two-stage input of bf16(silu(g) * u) equals nmq_moe_down on g and u (the
    activation formed in its staging) bit for bit: one launch (rows of 768 values) and the workspace form
    (5120)."""
    from ggufengine_amd import mmvq
    for fmt, L, k, E, FF in [("Q6_K", 1, 8, 2048, 768), ("Q6_K", 4, 8, 2048, 768), ("Q4_K", 2, 8, 256, 5120)]:
        t, w, per, gu, rng = _moe_down_case(nmq, fmt, L, k, E, FF, 16, 281 + L)
        n = L * k
        work = _moe_down_work(nmq, t, L, k, E, FF)
        ids = torch.from_numpy(rng.integers(0, 16, n)).cuda()
        wts = dev(rng.random((L, k)).astype(np.float32))
        say("moe_down_q8", fmt, L, k, E, FF)
        want = _moe_down_fused(nmq, t, w, per, ids, gu, wts, L, k, E, FF, work)
        a = mmvq.Eingang(n=n * FF, device=torch.device("cuda"))
        Lb = nmq.lib()
        nmq.check(Lb.nmq_silu_mul_quant(gu.data_ptr(), gu[n:].data_ptr(), a.xq.data_ptr(), a.xq2.data_ptr(),
                                        a.xd.data_ptr(), a.xs.data_ptr(), n * FF, nmq.stream_ptr()))
        got = torch.full((L, E), float("nan"), device="cuda")
        nmq.check(Lb.nmq_moe_down_q8(t, w.data_ptr(), ids.data_ptr(), L, k, per, a.xq.data_ptr(), a.xq2.data_ptr(),
                                     a.xd.data_ptr(), a.xs.data_ptr(), wts.data_ptr(), got.data_ptr(), E, FF,
                                     work.data_ptr(), work.numel(), nmq.stream_ptr()))
        torch.cuda.synchronize()
        assert torch.equal(got, want), (fmt, L, k, FF)


def test_moe_gate_up_graph_replays(nmq):
    """nmq_moe_gate_up + nmq_moe_down_q8 captured in one HIP graph, replayed with new ids and weights written
    between replays (eager work in between): every replay equals the eager calls."""
    from ggufengine_amd import mmvq
    fmt, FF, E, L, k = "Q4_K", 768, 2048, 1, 8
    t, A, B, per, ids, x, rng = _gate_up_case(fmt, 16, FF, E, L, k, 291)
    D = dev(random_blocks("Q6_K", 16 * E * FF // 256, seed=292))
    perd = D.numel() // 16
    wts = dev(rng.random((L, k)).astype(np.float32))
    a = mmvq.Eingang(n=L * k * FF, device=torch.device("cuda"))
    out = torch.empty(L, E, device="cuda")
    Lb = nmq.lib()

    def layer(a, out):
        _gate_up_fused(nmq, t, A, B, ids, per, x, nmq.X_F32_BF16, L, k, FF, E, a)
        nmq.check(Lb.nmq_moe_down_q8(14, D.data_ptr(), ids.data_ptr(), L, k, perd, a.xq.data_ptr(), a.xq2.data_ptr(),
                                     a.xd.data_ptr(), a.xs.data_ptr(), wts.data_ptr(), out.data_ptr(), E, FF, None, 0,
                                     nmq.stream_ptr()))
        return out
    say("moe_gate_up graph")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer(a, out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer(a, out)
    for rep in range(4):
        ids.copy_(torch.from_numpy(rng.integers(0, 16, L * k)))
        wts.copy_(torch.from_numpy(rng.random((L, k)).astype(np.float32)))
        x.copy_(torch.from_numpy(rng.standard_normal((L, E)).astype(np.float32)))
        g.replay()
        torch.cuda.synchronize()
        a2 = mmvq.Eingang(n=L * k * FF, device=torch.device("cuda"))
        want = layer(a2, torch.empty(L, E, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep




@pytest.mark.parametrize("fmt,n_out,n_in,gelu", [("Q4_K", 14336, 4096, False), ("Q4_K", 1024, 2048, True),
                                                 ("Q6_K", 1024, 2048, False)])
def test_gate_up_akt_equals_mv_and_akt(nmq, fmt, n_out, n_in, gelu):
    """mmvq.gate_up_akt (one launch for Q4_K; Q6_K through mv_mehrere + akt_q8) gives the Eingang of
    mv_mehrere on gate and up followed by akt_q8, bit for bit."""
    from ggufengine_amd import mmvq
    A = dev(random_blocks(fmt, n_out * n_in // 256, seed=501 + n_in))
    B = dev(random_blocks(fmt, n_out * n_in // 256, seed=502 + n_in))
    x = dev(np.random.default_rng(503).standard_normal(n_in).astype(np.float32))
    say("gate_up_akt", fmt, n_out, n_in, gelu)
    got = mmvq.gate_up_akt(fmt, A, B, x, n_out, n_in, gelu)
    g, u = mmvq.mv_mehrere(fmt, [A, B], x, [n_out, n_out], n_in)
    want = mmvq.akt_q8(g, u, gelu)[1]
    torch.cuda.synchronize()
    for f in ("xq", "xq2", "xd", "xs"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f

# ---- the whole expert layer (nmq_moe_layer) ------------------------------------------------------------------

def _layer_case(fg, fd, n_exp, E, FF, seed):
    from ggufengine_amd.gguf_types import TYPE_ID
    A = dev(random_blocks(fg, n_exp * FF * E // BV[fg], seed=seed))
    B = dev(random_blocks(fg, n_exp * FF * E // BV[fg], seed=seed + 1))
    D = dev(random_blocks(fd, n_exp * E * FF // BV[fd], seed=seed + 2))
    return TYPE_ID[fg], TYPE_ID[fd], A, B, D, A.numel() // n_exp, D.numel() // n_exp


def _layer_launch_by_launch(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF):
    """nmq_mv_experts_x (gate and up) -> nmq_silu_mul_quant -> nmq_mv_experts (down) -> nmq_moe_combine."""
    n = L * k
    a, _ = _gate_up_two_launches(nmq, tg, A, B, ids, per, x, nmq.X_F32_BF16, L, k, FF, E)
    y = torch.empty(n, E, device="cuda")
    out = torch.empty(L, E, device="cuda")
    Lb = nmq.lib()
    nmq.check(Lb.nmq_mv_experts(td, D.data_ptr(), ids.data_ptr(), n, perd, a.xq.data_ptr(), a.xq2.data_ptr(),
                                a.xd.data_ptr(), a.xs.data_ptr(), 1, y.data_ptr(), E, FF, nmq.stream_ptr()))
    nmq.check(Lb.nmq_moe_combine(y.data_ptr(), wts.data_ptr(), L, k, E, out.data_ptr(), nmq.stream_ptr()))
    return out


def _layer_work(nmq, L, k, E, FF):
    import ctypes
    need = ctypes.c_int64(0)
    nmq.check(nmq.lib().nmq_moe_layer_work_bytes(L, k, E, FF, ctypes.byref(need)))
    return torch.zeros(need.value, dtype=torch.uint8, device="cuda")


def _layer_call(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF, work, out=None):
    out = torch.full((L, E), float("nan"), device="cuda") if out is None else out
    nmq.check(nmq.lib().nmq_moe_layer(tg, A.data_ptr(), B.data_ptr(), per, td, D.data_ptr(), perd, ids.data_ptr(),
                                      wts.data_ptr(), L, k, x.data_ptr(), nmq.X_F32_BF16, out.data_ptr(), E, FF,
                                      work.data_ptr(), work.numel(), nmq.stream_ptr()))
    return out


# (gate|up format, down format, E, FF, tokens L, slots k, path): "gu" = gate|up kernel + down launch on its
# two-stage input (the default for these shapes), "gathered" = the gathered gate|up launch + down forming the
# activation (the default for many tokens)
LAYER = [("Q4_K", "Q6_K", 2048, 768, 1, 8, "gu"), ("Q4_K", "Q4_K", 4096, 1024, 1, 4, "gu"),
         ("Q4_K", "Q6_K", 2048, 1536, 1, 4, "gu"), ("Q4_K", "Q6_K", 2048, 768, 1, 3, "gu"),
         ("Q4_K", "Q6_K", 2048, 768, 4, 8, "gathered"), ("Q8_0", "Q8_0", 1024, 512, 1, 8, "gu"),
         ("Q6_K", "Q4_K", 2048, 768, 2, 4, "gathered"), ("Q4_K", "Q6_K", 2048, 768, 1, 8, "gathered"),
         ("Q4_K", "Q6_K", 256, 5120, 2, 8, "gu")]


@pytest.mark.parametrize("fg,fd,E,FF,L,k,path", LAYER)
def test_moe_layer_equals_launch_by_launch(nmq, tune, fg, fd, E, FF, L, k, path):
    """nmq_moe_layer equals the gathered gate|up launch, the activation's quantisation, the gathered down
    launch and the combine, bit for bit, over three calls in a row on one workspace with new routings,
    weights and inputs (FF 5120: the down launch through its workspace)."""
    if path == "gathered":
        tune(MOE_GU_WGS=0)
    n_exp = 12
    tg, td, A, B, D, per, perd = _layer_case(fg, fd, n_exp, E, FF, 301 + E + FF + L * k)
    work = _layer_work(nmq, L, k, E, FF)
    rng = np.random.default_rng(311 + L * k)
    say("moe_layer", fg, fd, E, FF, L, k, path)
    for call in range(3):
        ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
        wts = dev(rng.random((L, k)).astype(np.float32))
        x = dev(rng.standard_normal((L, E)).astype(np.float32))
        want = _layer_launch_by_launch(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF)
        got = _layer_call(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF, work)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (call, path)


def test_moe_layer_graph_replays(nmq):
    """One nmq_moe_layer call captured in a HIP graph and replayed with new ids, weights and inputs written
    between replays (eager work in between): every replay equals the launch-by-launch layer."""
    E, FF, L, k, n_exp = 2048, 768, 1, 8, 16
    tg, td, A, B, D, per, perd = _layer_case("Q4_K", "Q6_K", n_exp, E, FF, 321)
    work = _layer_work(nmq, L, k, E, FF)
    rng = np.random.default_rng(322)
    ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
    wts = dev(rng.random((L, k)).astype(np.float32))
    x = dev(rng.standard_normal((L, E)).astype(np.float32))
    out = torch.empty(L, E, device="cuda")
    say("moe_layer graph")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _layer_call(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF, work, out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _layer_call(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF, work, out)
    for rep in range(4):
        ids.copy_(torch.from_numpy(rng.integers(0, n_exp, L * k)))
        wts.copy_(torch.from_numpy(rng.random((L, k)).astype(np.float32)))
        x.copy_(torch.from_numpy(rng.standard_normal((L, E)).astype(np.float32)))
        g.replay()
        torch.cuda.synchronize()
        want = _layer_launch_by_launch(nmq, tg, td, A, B, D, per, perd, ids, wts, x, L, k, E, FF)
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep


# ---- down projection fused with the weighted combine (nmq_moe_down) ----------------------------------------

def _moe_down_case(nmq, fmt, L, k, E, FF, n_exp, seed):
    from ggufengine_amd.gguf_types import TYPE_ID
    raw = random_blocks(fmt, n_exp * E * FF // BV[fmt], seed=seed)
    w = dev(raw)
    rng = np.random.default_rng(seed + 1)
    gu = dev(rng.standard_normal((2 * L * k, FF)).astype(np.float32))
    return TYPE_ID[fmt], w, raw.size // n_exp, gu, rng


def _moe_down_unfused(nmq, t, w, per, ids, gu, wts, L, k, E, FF):
    n = L * k
    y = torch.empty(n, E, dtype=torch.float32, device="cuda")
    out = torch.empty(L, E, dtype=torch.float32, device="cuda")
    Lb = nmq.lib()
    nmq.check(Lb.nmq_mv_experts_x(t, w.data_ptr(), None, ids.data_ptr(), n, per, gu.data_ptr(), nmq.X_SILU_MUL_BF16,
                                  gu[n:].data_ptr(), 1, y.data_ptr(), E, FF, nmq.stream_ptr()))
    nmq.check(Lb.nmq_moe_combine(y.data_ptr(), wts.data_ptr(), L, k, E, out.data_ptr(), nmq.stream_ptr()))
    return out


def _moe_down_work(nmq, t, L, k, E, FF):
    import ctypes
    need = ctypes.c_int64(0)
    nmq.check(nmq.lib().nmq_moe_down_work_bytes(t, L, k, E, FF, ctypes.byref(need)))
    return torch.zeros(max(need.value, 0), dtype=torch.uint8, device="cuda")


def _moe_down_fused(nmq, t, w, per, ids, gu, wts, L, k, E, FF, work, out=None):
    n = L * k
    out = torch.empty(L, E, dtype=torch.float32, device="cuda") if out is None else out
    nmq.check(nmq.lib().nmq_moe_down(t, w.data_ptr(), ids.data_ptr(), L, k, per, gu.data_ptr(), nmq.X_SILU_MUL_BF16,
                                     gu[n:].data_ptr(), wts.data_ptr(), out.data_ptr(), E, FF, work.data_ptr(),
                                     work.numel(), nmq.stream_ptr()))
    return out


@pytest.mark.parametrize("fmt,L,k,E,FF", [("Q6_K", 1, 8, 2048, 768), ("Q6_K", 4, 8, 2048, 768),
                                          ("Q4_K", 3, 2, 1024, 512), ("Q8_0", 2, 8, 640, 1024),
                                          ("IQ2_XXS", 5, 4, 512, 1024), ("TQ2_0", 1, 8, 2048, 768),
                                          ("Q6_K", 2, 8, 256, 5120)])
def test_moe_down_fused_equals_unfused(nmq, fmt, L, k, E, FF):
    """nmq_moe_down (each workgroup computes a row block of all k slots of one token and sums them in LDS;
    n_in 5120: the plain gathered launch into the workspace + the combine launch) equals nmq_mv_experts_x +
    nmq_moe_combine bit for bit, over three calls in a row with new routings."""
    n_exp = 16
    t, w, per, gu, rng = _moe_down_case(nmq, fmt, L, k, E, FF, n_exp, 231 + L * k)
    work = _moe_down_work(nmq, t, L, k, E, FF)
    say("moe_down", fmt, L, k, E, FF, work.numel())
    for call in range(3):
        ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
        wts = dev(rng.random((L, k)).astype(np.float32))
        want = _moe_down_unfused(nmq, t, w, per, ids, gu, wts, L, k, E, FF)
        got = _moe_down_fused(nmq, t, w, per, ids, gu, wts, L, k, E, FF, work)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (fmt, L, k, call)
    assert (work.numel() == 0) == (FF <= 4096)      # a workspace only where the one-launch kernel does not fit


def test_moe_down_refuses_a_small_workspace(nmq):
    t, w, per, gu, rng = _moe_down_case(nmq, "Q6_K", 2, 8, 512, 5120, 4, 241)
    work = _moe_down_work(nmq, t, 2, 8, 512, 5120)
    assert work.numel() == 2 * 8 * 512 * 4
    ids = torch.zeros(16, dtype=torch.int64, device="cuda")
    wts = torch.ones(2, 8, device="cuda")
    with pytest.raises(ValueError):
        _moe_down_fused(nmq, t, w, per, ids, gu, wts, 2, 8, 512, 5120, work[:work.numel() - 256])


def test_moe_down_graph_replays(nmq):
    """One nmq_moe_down call captured in a HIP graph and replayed with new ids and weights written into its
    input tensors between replays (eager work in between): every replay equals the unfused launches."""
    L, k, E, FF, n_exp = 2, 8, 2048, 768, 16
    t, w, per, gu, rng = _moe_down_case(nmq, "Q6_K", L, k, E, FF, n_exp, 251)
    work = _moe_down_work(nmq, t, L, k, E, FF)
    ids = torch.from_numpy(rng.integers(0, n_exp, L * k)).cuda()
    wts = dev(rng.random((L, k)).astype(np.float32))
    out = torch.empty(L, E, device="cuda")
    say("moe_down graph")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _moe_down_fused(nmq, t, w, per, ids, gu, wts, L, k, E, FF, work, out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _moe_down_fused(nmq, t, w, per, ids, gu, wts, L, k, E, FF, work, out)
    for rep in range(4):
        ids.copy_(torch.from_numpy(rng.integers(0, n_exp, L * k)))
        wts.copy_(torch.from_numpy(rng.random((L, k)).astype(np.float32)))
        g.replay()
        torch.cuda.synchronize()
        want = _moe_down_unfused(nmq, t, w, per, ids, gu, wts, L, k, E, FF)
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
