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

BV = {"Q8_0": 32, "Q4_K": 256, "Q6_K": 256, "TQ2_0": 256, "IQ2_XXS": 256}


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
DISPATCH = [("Q4_K", 1, "mmvq.mv"), ("Q4_K", 9, "mmvq.mv"), ("Q4_K", 16, "mmvq.mv"), ("Q4_K", 40, "mmvq.mm"),
            ("Q4_K", 120, "unpack"), ("Q6_K", 3, "mmvq.mv"), ("Q6_K", 17, "mmvq.mm"),
            ("TQ2_0", 1, "cudakern.mv"), ("TQ2_0", 5, "cudakern.mm"), ("TQ2_0", 17, "unpack"),
            ("IQ2_XXS", 1, "cudakern.mv"), ("IQ2_XXS", 16, "cudakern.mm"), ("Q8_0", 1, "cudakern.mv"),
            ("Q8_0", 8, "cudakern.mm"), ("Q8_0", 24, "unpack")]


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
    # stage 3: the weighted combine of the layer, against the same slot outputs in fp64
    comb = (y.astype(np.float64).reshape(L, k, E) * wts[:, :, None]).sum(1)
    assert oracle.rel_err_rows(out, comb).max() <= 1e-5
    # end to end against the oracle chain (dequantised weights all the way)
    g_o, u_o = g_ref, u_ref
    act_o = g_o / (1.0 + np.exp(-g_o)) * u_o
    y_o = np.stack([oracle.mv_deq("Q6_K", _expert_rows(d_raw, "Q6_K", n_exp, E, FF, e), E, FF,
                                  oracle.round_bf16(act_o[i:i + 1].astype(np.float32)))[0]
                    for i, (_, _, e) in enumerate(pairs)])
    full = (y_o.reshape(L, k, E) * wts[:, :, None]).sum(1)
    assert oracle.rel_err_rows(out, full).max() <= 1e-2
