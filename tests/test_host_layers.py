"""Host-side logic of the layer mirrors (no GPU): the softmax router against a restatement, and the
loud failure of the block-format layers where libnmq cannot run."""
import numpy as np
import pytest
import torch

from ggufengine_amd import experts, packed
from ggufengine_amd.gguf_types import GGUFError, TYPE_ID


def _router_restated(logits: np.ndarray, k: int):
    """softmax, the k largest (ties: lower index first), renormalised (reference baukasten.py:171-190)."""
    z = logits.astype(np.float64)
    p = np.exp(z - z.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    idx = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(p, idx, -1)
    return idx, w / (w.sum(-1, keepdims=True) + 1e-20)


@pytest.mark.parametrize("L", [1, 4])
def test_router_matches_restatement(L):
    logits = np.random.Generator(np.random.PCG64(42)).standard_normal((L, 128)).astype(np.float32)
    idx, w = experts.auswahl(torch.from_numpy(logits), 8)
    ridx, rw = _router_restated(logits, 8)
    assert np.array_equal(np.sort(idx.numpy(), -1), np.sort(ridx, -1))
    # same experts, same weights (order of equal-probability slots aside)
    for t in range(L):
        a = dict(zip(idx[t].tolist(), w[t].tolist()))
        b = dict(zip(ridx[t].tolist(), rw[t].tolist()))
        for e in a:
            assert abs(a[e] - b[e]) <= 1e-6
    assert torch.allclose(w.sum(-1), torch.ones(L), atol=1e-6)


def test_router_scale_and_no_renormalisation():
    logits = torch.tensor([[3.0, 1.0, 2.0, 0.0]])
    idx, w = experts.auswahl(logits, 2, normieren=False, scale=2.5)
    p = torch.softmax(logits, -1)
    assert idx.tolist() == [[0, 2]]
    assert torch.allclose(w, 2.5 * p[:, [0, 2]])


def _router_variant_restated(logits: np.ndarray, k: int, sigmoid: bool, bias, n_group: int, group_used: int):
    """The router's variants written out per token with numpy: p = sigmoid or softmax; the choice on p + bias;
    groups scored by their largest choice value (sigmoid: the sum of the two largest), the group_used best
    kept; the k largest kept choices; weights p there, renormalised."""
    z = logits.astype(np.float64)
    if sigmoid:
        p = 1.0 / (1.0 + np.exp(-z))
    else:
        p = np.exp(z - z.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
    choice = p + (0.0 if bias is None else bias.astype(np.float64))
    ids, ws = [], []
    for t in range(z.shape[0]):
        c = choice[t].copy()
        if n_group > 1:
            je = c.size // n_group
            score = [np.sort(c[g * je:(g + 1) * je])[::-1][:min(2, je)].sum() if sigmoid else c[g * je:(g + 1) * je].max()
                     for g in range(n_group)]
            keep = set(np.argsort(-np.array(score), kind="stable")[:group_used].tolist())
            for g in range(n_group):
                if g not in keep:
                    c[g * je:(g + 1) * je] = -np.inf
        sel = np.argsort(-c, kind="stable")[:k]
        wt = p[t, sel]
        ids.append(sel)
        ws.append(wt / (wt.sum() + 1e-20))
    return np.array(ids), np.array(ws)


@pytest.mark.parametrize("sigmoid,use_bias,n_group,group_used", [(True, True, 8, 4), (False, False, 4, 2),
                                                                   (True, False, 1, 1), (False, True, 1, 1)])
def test_router_variants(sigmoid, use_bias, n_group, group_used):
    """Sigmoid gating, a selection bias the weights do not see, grouped selection (reference
    baukasten.py:171-190) against the per-token restatement: the same experts, weights within 1e-6."""
    rng = np.random.default_rng(7 + n_group)
    logits = rng.standard_normal((5, 64)).astype(np.float32)
    bias = (rng.standard_normal(64) * 0.3).astype(np.float32) if use_bias else None
    idx, w = experts.auswahl(torch.from_numpy(logits), 6, sigmoid=sigmoid,
                             wahl_bias=None if bias is None else torch.from_numpy(bias), n_group=n_group,
                             group_used=group_used)
    ridx, rw = _router_variant_restated(logits, 6, sigmoid, bias, n_group, group_used)
    for t in range(5):
        a = dict(zip(idx[t].tolist(), w[t].tolist()))
        b = dict(zip(ridx[t].tolist(), rw[t].tolist()))
        assert set(a) == set(b), t
        assert all(abs(a[e] - b[e]) <= 1e-6 for e in a)
    if n_group > 1:  # every chosen expert lies in one of group_used groups
        je = 64 // n_group
        assert all(len({e // je for e in row}) <= group_used for row in idx.tolist())


def test_router_softmax_after_selection():
    logits = torch.tensor([[0.5, 3.0, -1.0, 2.0, 1.0]])
    idx, w = experts.auswahl(logits, 3, nach_auswahl=True)
    assert idx.tolist() == [[1, 3, 4]]
    assert torch.allclose(w, torch.softmax(torch.tensor([[3.0, 2.0, 1.0]]), -1))


def test_block_layers_refuse_cpu_tensors():
    raw = torch.zeros(4 * 16 * 144, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        packed.PackedLinear(raw, TYPE_ID["Q4_K"], 4, 4096)
    with pytest.raises(RuntimeError):
        experts.PackedExperts(raw, TYPE_ID["Q4_K"], 1, 4, 4096)


def test_block_layers_check_sizes():
    raw = torch.zeros(100, dtype=torch.uint8)
    with pytest.raises(GGUFError):
        packed.PackedLinear(raw, TYPE_ID["Q4_K"], 4, 4096)
    with pytest.raises(GGUFError):
        experts.PackedExperts(raw, TYPE_ID["Q6_K"], 2, 4, 4096)
    with pytest.raises(GGUFError):
        packed.PackedLinear(raw, 9, 1, 32)   # Q8_1 is not a weight format of this library


def test_hostmem_without_gpu():
    """hostmem imports and answers without a device: ordinary tensors are not pinned blocks, nothing is
    pending, flush() is a no-op, and abbilden() refuses memory that is not from hostmem.empty()."""
    import torch
    from ggufengine_amd import hostmem
    t = torch.zeros(16, dtype=torch.uint8)
    assert not hostmem.abgebildet(t)
    assert hostmem.pending() == 0
    hostmem.flush()
    with pytest.raises(ValueError):
        hostmem.abbilden(t, "cpu")
    assert hostmem.ram_reicht(0) in (True, False)


def test_mat_vec_bound_by_row_length():
    """Where PackedLinear switches from the int8 mat-vec kernels to the fp16 matrix cores: 8 tokens for
    rows the dense-read kernel takes (up to 4096 values, or a multiple of 2048 up to 32768 over K
    ranges), for other rows 1 (Q4_K) and 4 (Q6_K, the few-token long-row kernel)."""
    from ggufengine_amd import mmvq
    assert mmvq.mv_bis("Q4_K", 4096) == 8 and mmvq.mv_bis("Q6_K", 4096) == 8
    assert mmvq.mv_bis("Q4_K", 1024) == 8 and mmvq.mv_bis("Q6_K", 2048) == 8
    assert mmvq.mv_bis("Q4_K", 14336) == 8 and mmvq.mv_bis("Q6_K", 14336) == 8
    assert mmvq.mv_bis("Q4_K", 28672) == 8 and mmvq.mv_bis("Q6_K", 6144) == 8
    assert mmvq.mv_bis("Q4_K", 11008) == 1 and mmvq.mv_bis("Q6_K", 11008) == 4
    assert mmvq.mv_bis("Q4_K", 4352) == 1 and mmvq.mv_bis("Q6_K", 4352) == 4
    assert mmvq.mv_bis("Q4_K", 36864) == 1 and mmvq.mv_bis("Q6_K", 36864) == 4
