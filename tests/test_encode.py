"""The library's own block encoders (nmq_encode, host code): the bytes they write are valid blocks
of the format, and their dequantisation (by the oracle) stays close to the input weights."""
import numpy as np
import pytest

from ggufengine_amd import encode as E


def _w(n, seed=0):
    return (np.random.default_rng(seed).standard_normal(n) * 0.02).astype(np.float32)


@pytest.mark.parametrize("fmt,rel", [("Q4_0", 0.12), ("Q8_0", 0.01), ("Q4_K", 0.12), ("Q6_K", 0.03), ("IQ2_XXS", 0.45)])
def test_encode_dequant_close(oracle, fmt, rel):
    w = _w(256 * 64)
    raw = E.encode(fmt, w, threads=4)
    back = oracle.dequant(fmt, raw)
    err = np.linalg.norm(back - w) / np.linalg.norm(w)
    assert err < rel, err


def test_q8_0_follows_the_config_rule(oracle):
    w = _w(32 * 50, seed=3)
    raw = E.encode("Q8_0", w).reshape(-1, 34)
    d = np.abs(w.reshape(-1, 32)).max(1) / np.float32(127)
    assert np.array_equal(raw[:, :2].copy().view(np.float16).ravel(), d.astype(np.float16))
    q = raw[:, 2:].view(np.int8).astype(np.int32)
    assert np.all(np.abs(q - np.round(w.reshape(-1, 32) / d[:, None])) <= 1)


def test_q4_0_follows_ggml_rule(oracle):
    """d = -m / 8 for the value m of largest magnitude (which lands on nibble 0); every nibble within one
    step of x / d + 8."""
    w = _w(32 * 50, seed=5)
    raw = E.encode("Q4_0", w).reshape(-1, 18)
    blk = w.reshape(-1, 32)
    m = blk[np.arange(blk.shape[0]), np.abs(blk).argmax(1)]
    d = m / np.float32(-8)
    assert np.array_equal(raw[:, :2].copy().view(np.float16).ravel(), d.astype(np.float16))
    qs = raw[:, 2:].astype(np.int32)
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    assert np.all(q[np.arange(blk.shape[0]), np.abs(blk).argmax(1)] == 0)
    assert np.all(np.abs(q - (blk / d[:, None] + 8)) <= 1)


def test_tq2_0_ternary_lossless(oracle):
    rng = np.random.default_rng(4)
    codes = rng.choice(3, size=(4, 256), p=[0.3, 0.4, 0.3])
    d = np.abs(rng.standard_normal(4) * 0.02).astype(np.float16).astype(np.float32)
    d[d == 0] = 0.01
    codes[:, 0] = 2  # max |w| = d in every block
    w = ((codes - 1) * d[:, None]).astype(np.float32)
    assert np.array_equal(oracle.dequant("TQ2_0", E.encode("TQ2_0", w)), w.ravel())
    assert np.array_equal(oracle.dequant("TQ2_0", E.pack_ternary(codes, d)), w.ravel())


def test_iq2_xxs_sign_parity(oracle):
    raw = E.encode("IQ2_XXS", _w(256 * 8, seed=5)).reshape(-1, 66)
    aux1 = raw[:, 2:].reshape(-1, 8, 8)[:, :, 4:].copy().view(np.uint32)
    for l in range(4):
        s7 = (aux1 >> (7 * l)) & 127
        assert s7.max() <= 127
    assert np.all((aux1 >> 28) <= 15)


def test_encoders_reject_bad_sizes():
    with pytest.raises(ValueError):
        E.encode("Q4_K", np.zeros(100, np.float32))
