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
