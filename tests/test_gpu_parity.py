"""GPU parity of the HIP kernels (libnmq.so, called through ctypes) against the CPU oracle.

Bars (from the task's parity definition):
  - two-stage activation (xq, xq2, xd, xs): bit-exact;
  - int32 sums per 16 weights: bit-exact;
  - fp32 outputs: per output row-vector max|y - ref| / max|ref| <= 1e-3 against the dequantise +
    matmul oracle (fp64 accumulation) on the same x (rounded to bf16 first where the reference's
    entry point does); and <= 2e-5 against the oracle of the same integer decomposition.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import random_blocks

pytestmark = pytest.mark.gpu

FMTS = ["Q4_0", "Q8_0", "Q4_K", "Q6_K", "TQ2_0", "IQ2_XXS"]
BV = {"Q4_0": 32, "Q8_0": 32, "Q4_K": 256, "Q6_K": 256, "TQ2_0": 256, "IQ2_XXS": 256}
TOL_DEQ = 1e-3
TOL_INT = 2e-5


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


def quant_dev(x: torch.Tensor):
    from ggufengine_amd import mmvq
    e = mmvq.Eingang(x)
    return e


def host(t):
    return t.detach().cpu().numpy()


# ---- activation ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quant_q8_bitexact(nmq, oracle, dtype):
    rng = np.random.default_rng(11)
    n = 32 * 3000
    x = (rng.standard_normal(n) * np.repeat(10.0 ** rng.uniform(-4, 3, n // 32), 32)).astype(np.float32)
    x[:32] = 0.0                 # an all-zero group
    x[32:64] = -1.5              # all equal
    xt = torch.from_numpy(x).to(dtype).cuda()
    say("quant_q8", dtype, n)
    e = quant_dev(xt)
    torch.cuda.synchronize()
    xin = xt.float().cpu().numpy()
    ref = oracle.quant_q8(xin)
    for name, g, r in zip(("xq", "xq2", "xd", "xs"), (e.xq, e.xq2, e.xd, e.xs), ref):
        assert np.array_equal(host(g).view(np.uint8), np.ascontiguousarray(r).view(np.uint8)), name


def test_quant_q8_ties_and_tiny_scales(nmq, oracle):
    """Groups whose quotients v / d fall exactly on half-integers (d = 2^k: max = 127 * 2^k), within an ulp
    of them, and groups with a scale below 2^-100 (the reciprocal-product shortcut does not apply there):
    the two-stage input equals the oracle's (IEEE division, round half to even) bit for bit, from
    nmq_quant_q8 and from the value staging of a mat-vec (nmq_mv_x against nmq_mv on that input)."""
    from ggufengine_amd.gguf_types import TYPE_ID
    rng = np.random.default_rng(17)
    groups = []
    for k in range(-6, 7):
        d = np.float32(2.0 ** k)
        half = (rng.integers(-126, 126, 31) + 0.5).astype(np.float32) * d
        g = np.concatenate([[np.float32(127) * d], half]).astype(np.float32)
        groups += [g, np.nextafter(g, np.float32(np.inf)), np.nextafter(g, np.float32(-np.inf))]
    for sc in (1e-38, 1e-33, 2.0 ** -110):
        groups.append((rng.standard_normal(32) * sc).astype(np.float32))
    x = np.concatenate(groups).astype(np.float32)
    n = (x.size + 255) // 256 * 256
    x = np.concatenate([x, (rng.standard_normal(n - x.size) * 3).astype(np.float32)])
    say("quant_q8 ties", n)
    e = quant_dev(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    for name, g, r in zip(("xq", "xq2", "xd", "xs"), (e.xq, e.xq2, e.xd, e.xs), oracle.quant_q8(x)):
        assert np.array_equal(host(g).view(np.uint8), np.ascontiguousarray(r).view(np.uint8)), name
    raw = random_blocks("Q4_K", 64 * n // 256, seed=18)
    w = dev(raw)
    y1 = torch.full((64,), float("nan"), device="cuda")
    y2 = torch.full((64,), float("nan"), device="cuda")
    L = nmq.lib()
    xd_ = dev(x)
    nmq.check(L.nmq_mv_x(TYPE_ID["Q4_K"], 1, (ctypes.c_void_p * 1)(w.data_ptr()), (ctypes.c_int * 1)(64),
                         (ctypes.c_void_p * 1)(y1.data_ptr()), xd_.data_ptr(), nmq.X_F32, None, n, nmq.stream_ptr()))
    nmq.check(L.nmq_mv(TYPE_ID["Q4_K"], w.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                       e.xs.data_ptr(), y2.data_ptr(), 64, n, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


# ---- integer sums --------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", FMTS)
def test_block_sums_bitexact(nmq, oracle, fmt):
    n_out = 37
    n_in = 1056 if BV[fmt] == 32 else 1280      # Q4_0 / Q8_0: 33 blocks, the last unit half full
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=21)
    rng = np.random.default_rng(22)
    xq = rng.integers(-127, 128, n_in).astype(np.int8)
    xq2 = rng.integers(-127, 128, n_in).astype(np.int8)
    s1 = torch.empty(n_out, n_in // 16, dtype=torch.int32, device="cuda")
    s2 = torch.empty_like(s1)
    w, q1, q2 = dev(raw), dev(xq), dev(xq2)
    say("block_sums", fmt, n_out, n_in)
    from ggufengine_amd.gguf_types import TYPE_ID
    nmq.check(nmq.lib().nmq_block_sums(TYPE_ID[fmt], w.data_ptr(), q1.data_ptr(), q2.data_ptr(), s1.data_ptr(),
                                       s2.data_ptr(), n_out, n_in, nmq.stream_ptr()))
    torch.cuda.synchronize()
    r1, r2 = oracle.block_sums(fmt, raw, n_out, n_in, xq, xq2)
    assert np.array_equal(host(s1), r1)
    assert np.array_equal(host(s2), r2)


# ---- mat-vec --------------------------------------------------------------------------------------------

def _check_mv(oracle, fmt, raw, n_out, n_in, x_np, y, tol_deq=TOL_DEQ):
    y = host(y).reshape(-1, n_out)
    ref = oracle.mv_deq(fmt, raw, n_out, n_in, x_np)
    err = oracle.rel_err_rows(y, ref)
    assert err.max() <= tol_deq, (fmt, n_out, n_in, float(err.max()))
    xq, xq2, xd, xs = oracle.quant_q8(x_np)
    ref_i = oracle.mv_int(fmt, raw, n_out, n_in, xq, xq2, xd, xs, ncols=x_np.shape[0])
    err_i = oracle.rel_err_rows(y, ref_i)
    assert err_i.max() <= TOL_INT, (fmt, n_out, n_in, float(err_i.max()))
    return float(err.max())


SHAPES = [(256, 512), (300, 1280), (1024, 4096), (37, 768)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_mv_one_token(nmq, oracle, fmt, shape):
    from ggufengine_amd import cudakern
    n_out, n_in = shape
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=31)
    x = np.random.default_rng(32).standard_normal((1, n_in)).astype(np.float32)
    say("mv", fmt, shape)
    e = quant_dev(dev(x))
    y = torch.empty(1, n_out, device="cuda")
    from ggufengine_amd.gguf_types import TYPE_ID
    raw_d = dev(raw)  # kept alive until the launch has run
    nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                               e.xs.data_ptr(), y.data_ptr(), n_out, n_in, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    _check_mv(oracle, fmt, raw, n_out, n_in, x, y)
    assert cudakern.verfuegbar("cuda", fmt, n_in)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n_in", [8448, 10240, 14336, 16384])
@pytest.mark.parametrize("kernel", ["ksplit", "ksplit_compiler_reads", "longrow", "longrow_pipelined"])
def test_mv_one_token_long_rows(nmq, oracle, tune, fmt, n_in, kernel):
    """One token on rows of 132..256 units of 64 values (the Llama down projection has 224): the K-split
    kernel (3 or 4 waves per row, input slices from global memory; reads issued by hand for Q4_K, TQ2_0,
    Q6_K, and the compiler-scheduled variant; IQ2_XXS always takes the long-row kernel), and the long-row
    kernel with one row per wave and (with fewer resident waves than rows) the variant that cycles two row
    buffers."""
    n_out = 300
    if kernel == "ksplit_compiler_reads":
        tune(MVK_HR=0)
    if kernel.startswith("longrow"):
        tune(MVK=0)
    if kernel == "longrow_pipelined":
        tune(MVL_WPC=1)   # 1 wave per CU: fewer waves than rows
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=81)
    x = np.random.default_rng(82).standard_normal((1, n_in)).astype(np.float32)
    x[0, 5] = 25.0
    say("mv long rows", fmt, n_in, kernel)
    e = quant_dev(dev(x))
    y = torch.full((1, n_out), float("nan"), device="cuda")
    from ggufengine_amd.gguf_types import TYPE_ID
    raw_d = dev(raw)  # kept alive until the launch has run
    nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                               e.xs.data_ptr(), y.data_ptr(), n_out, n_in, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "TQ2_0", "Q8_0"])
@pytest.mark.parametrize("hr", [1, 0, 4])
def test_mv_one_token_long_rows_batches(nmq, oracle, tune, fmt, hr):
    """The K-split kernel with more than 64 rows per workgroup (1 resident wave per CU: 85 workgroups of 3
    waves for 5600 rows of 8448 values, 65-66 rows each), so that its row batches are added and written in
    the middle of the row loop as well as at the end, with hand-issued reads (hr = 1; Q8_0 has none) and
    compiler-scheduled ones."""
    n_out, n_in = 5600, 8448
    tune(MVK_WPC=1)
    tune(MVK_HR=1 if hr else 0)
    tune(MVK_NBUF=4 if hr == 4 else 3)   # hr = 4: hand-issued reads with 4 row buffers
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=83)
    x = np.random.default_rng(84).standard_normal((1, n_in)).astype(np.float32)
    say("mv long rows batches", fmt, hr)
    e = quant_dev(dev(x))
    y = torch.full((1, n_out), float("nan"), device="cuda")
    from ggufengine_amd.gguf_types import TYPE_ID
    raw_d = dev(raw)
    nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                               e.xs.data_ptr(), y.data_ptr(), n_out, n_in, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("nc", [2, 3, 4, 5, 8, 9, 16])
def test_mv_tokens(nmq, oracle, fmt, nc):
    n_out, n_in = (300, 1280) if BV[fmt] != 32 else (300, 1056)
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=41 + nc)
    x = np.random.default_rng(42 + nc).standard_normal((nc, n_in)).astype(np.float32)
    x[:, 7] = 30.0   # an outlier column (test_mmvq.py:71)
    say("mv tokens", fmt, nc)
    from ggufengine_amd import mmvq, cudakern
    if fmt in mmvq.FORMATE:
        y = mmvq.mv(fmt, dev(raw), dev(x), n_out, n_in)
    elif 2 <= nc <= 16:
        xb = oracle.round_bf16(x)
        y = cudakern.mm(fmt, dev(raw), dev(x), n_out, n_in)
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, xb, y)
        return
    torch.cuda.synchronize()
    assert tuple(y.shape) == (nc, n_out)
    _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("split", [(1, 16), (1, 8), (1, 4), (1, 2), (1, 1), (2, 4), (4, 4), (3, 2)])
def test_mv_tokens_matrix_core_splits(nmq, oracle, tune, fmt, split):
    """2..16 tokens on the matrix cores (one or two groups of 8 per launch) with every (tiles per
    workgroup, K slices) split: slices of 16, 8, 4, 2 and 1 blocks (held whole or cycled through
    buffers), a partial last tile, and workgroups whose last tiles lie past the matrix."""
    tpw, ks = split
    n_out, n_in = 200, 4096
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=61 + ks)
    from ggufengine_amd.gguf_types import TYPE_ID
    tune(MVM=2)   # the matrix-core path from 2 tokens on, whatever the format
    tune(MVT_MAX=1)   # (not the few-token Q4_K kernel)
    tune(MVD=0)   # (nor the dense-read Q4_K kernel)
    tune(MVM_TPW=tpw)
    tune(MVM_KS=ks)
    for nc in (2, 7, 8, 12, 16):
        x = np.random.default_rng(62 + nc).standard_normal((nc, n_in)).astype(np.float32)
        x[:, 7] = 30.0
        e = quant_dev(dev(x))
        y = torch.full((nc, n_out), float("nan"), device="cuda")
        say("mv tokens mfma", fmt, split, nc)
        raw_d = dev(raw)  # kept alive until the launch has run
        nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                   e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                   nmq.stream_ptr()))
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", ["Q4_K", "Q4_0", "Q8_0", "Q6_K", "TQ2_0", "IQ2_XXS"])
@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 4096), (200, 4096), (1000, 2048), (333, 1024),
                                   (130, 512)])
@pytest.mark.parametrize("split", [None, (1, 4), (2, 8), (4, 2)])
def test_mv_tokens_dense_mfma(nmq, oracle, tune, fmt, shape, split):
    """2..8 tokens on the dense-read matrix-core kernel (weights and input moved into LDS by
    global_load_lds; the default for Q4_K at 5..8 tokens, the other formats at 2..8): the planner's split
    and forced (tiles per workgroup, K slices) splits, slices of 1 and 2 chunks (Q4_K, Q4_0, TQ2_0,
    IQ2_XXS: chunks of 2 blocks of 256 values; Q8_0, Q6_K: 1 block), chunk windows starting off a 16-byte
    boundary (Q6_K, TQ2_0, IQ2_XXS), partial last tiles and tiles past the matrix.  Rows whose bytes are not
    a multiple of 16 (Q6_K, TQ2_0, IQ2_XXS below 2048 values) take the other kernels."""
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = shape
    nblk = n_in // 256
    chb = 1 if fmt in ("Q8_0", "Q6_K") else 2
    if split is not None:
        tpw, ks = split
        if nblk % ks or (nblk // ks) % chb or (nblk // ks) // chb not in (1, 2) or tpw * ks < 4:
            pytest.skip("split outside the kernel's slices")
        tune(MVD_TPW=tpw)
        tune(MVD_KS=ks)
    elif n_out < 16 * 4:
        pytest.skip("planner keeps small matrices elsewhere")
    tune(MVD_MIN=2)
    tune(MVT_MAX=1)
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=71 + n_out % 97)
    raw_d = dev(raw)
    for nc in (2, 5, 8) if n_out > 5000 else (2, 3, 4, 5, 6, 7, 8):
        x = np.random.default_rng(72 + nc).standard_normal((nc, n_in)).astype(np.float32)
        x[:, 3] = -25.0
        e = quant_dev(dev(x))
        y = torch.full((nc, n_out), float("nan"), device="cuda")
        say("mv tokens dense mfma", fmt, shape, split, nc)
        nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                   e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                   nmq.stream_ptr()))
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", [(1000, 4096), (300, 14336)])
def test_mv_9_to_16_tokens_dense_pairs(nmq, oracle, fmt, shape):
    """9..16 tokens where the dense-read kernel takes 8 (rows of 4096 values, and 14336 over K ranges):
    two launches (8 and the rest, the rest on its own kernel: one-token, few-token or dense), against the
    oracle."""
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = shape
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=77)
    raw_d = dev(raw)
    for nc in (9, 10, 12, 13, 16):
        x = np.random.default_rng(78 + nc).standard_normal((nc, n_in)).astype(np.float32)
        x[nc - 1, 11] = 40.0
        e = quant_dev(dev(x))
        y = torch.full((nc, n_out), float("nan"), device="cuda")
        say("mv 9..16 tokens dense pairs", fmt, shape, nc)
        nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                   e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                   nmq.stream_ptr()))
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", [(4096, 14336), (300, 8192), (130, 6144), (64, 28672)])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_mv_tokens_long_rows_k_ranges(nmq, oracle, tune, fmt, shape, mode):
    """2..8 tokens on rows beyond 4096 values on the dense-read kernel over K ranges: one launch staging
    the ranges one after another (mode 1, the default: equal ranges, or ranges of 16 blocks and a shorter
    last one; mode 3: equal ranges only), or one launch per range of 4096 values (the last shorter),
    each adding its sums to y in range order (mode 2); against the oracle, and two calls bit for bit
    equal.  Q6_K 2..4 tokens take the few-token long-row kernel by default, so the
    ranges are forced on with that kernel off."""
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = shape
    tune(MVD_LONG=min(mode, 2))
    if mode == 3:
        tune(MVD_UNEQ=0)   # equal ranges only
    if fmt == "Q6_K":
        tune(MVLT_MAX=1)
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=79 + n_in % 89)
    raw_d = dev(raw)
    for nc in ((2, 5, 8) if n_out > 1000 else (2, 3, 4, 5, 6, 7, 8)):
        x = np.random.default_rng(80 + nc).standard_normal((nc, n_in)).astype(np.float32)
        x[:, 5000 % n_in] = -30.0
        e = quant_dev(dev(x))
        ys = []
        for rep in range(2):
            y = torch.full((nc, n_out), float("nan"), device="cuda")
            say("mv tokens long rows", fmt, shape, mode, nc, rep)
            nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                       e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                       nmq.stream_ptr()))
            torch.cuda.synchronize()
            ys.append(y)
        assert torch.equal(ys[0], ys[1])
        _check_mv(oracle, fmt, raw, n_out, n_in, x, ys[0])


@pytest.mark.parametrize("fmt", ["Q4_0", "Q8_0", "Q6_K", "TQ2_0", "IQ2_XXS"])
def test_mv_tokens_weights_off_16_bytes(nmq, oracle, fmt):
    """Weights 2 bytes past a 16-byte boundary (allowed for every format but Q4_K): the dense-read
    kernel needs 16-byte aligned rows, so 2..8 tokens take the other kernels, with the same results."""
    from ggufengine_amd.gguf_types import TYPE_ID
    n_out, n_in = 1000, 2048
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=75)
    buf = torch.zeros(raw.nbytes + 64, dtype=torch.uint8, device="cuda")
    off = (16 - buf.data_ptr() % 16) % 16 + 2
    buf[off:off + raw.nbytes] = dev(raw)
    for nc in (2, 5, 8):
        x = np.random.default_rng(76 + nc).standard_normal((nc, n_in)).astype(np.float32)
        e = quant_dev(dev(x))
        y = torch.full((nc, n_out), float("nan"), device="cuda")
        say("mv tokens weights off 16 bytes", fmt, nc)
        nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], buf.data_ptr() + off, e.xq.data_ptr(), e.xq2.data_ptr(),
                                   e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                   nmq.stream_ptr()))
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", FMTS)
def test_mv_tokens_17_to_112(nmq, oracle, fmt):
    """17..112 tokens through nmq_mv (launches of 16 on the matrix cores, or 8 on the dot4 kernels).
    200 rows: partial tiles; Q8_0 / Q4_0 also on 1056 values (not whole 256-value blocks)."""
    from ggufengine_amd.gguf_types import TYPE_ID
    for n_in in ((1280, 1056) if BV[fmt] == 32 else (1280,)):
        n_out = 200
        raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=91)
        raw_d = dev(raw)  # kept alive until the launches have run
        for nc in (17, 24, 33, 64, 65, 112):
            x = np.random.default_rng(92 + nc).standard_normal((nc, n_in)).astype(np.float32)
            x[:, 7] = 30.0
            x[nc // 2, :] *= 1e-3   # a token of much smaller scale next to the others
            e = quant_dev(dev(x))
            y = torch.full((nc, n_out), float("nan"), device="cuda")
            say("mv 17..112 tokens", fmt, n_in, nc)
            nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                       e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                       nmq.stream_ptr()))
            torch.cuda.synchronize()
            _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


# ---- several tokens on the fp16 matrix cores (nmq_mm) ---------------------------------------------------

MM_TOL = 2e-5   # against the dequantised weights times the exact x (fp64)


@pytest.mark.parametrize("f32", [True, False])
@pytest.mark.parametrize("n_in", [4096 + 32, 14336, 16384 + 32])
def test_mm_input_bitexact(nmq, oracle, f32, n_in):
    """nmq_mm_input equals the oracle's two-stage fp16 input value for value (the sign of a zero aside):
    rows of very different scales, a zero row, an all-equal row, a row of subnormal-range values (bf16:
    some round to -0); rows held in registers in one or two rounds, and longer rows read twice."""
    rng = np.random.default_rng(101)
    nc = 19
    x = (rng.standard_normal((nc, n_in)) * 10.0 ** rng.uniform(-5, 5, (nc, 1))).astype(np.float32)
    x[2] = 0.0
    x[3] = 0.75
    x[4] *= 1e-35
    if not f32:
        x = oracle.round_bf16(x)
    xd = dev(x) if f32 else dev(x).to(torch.bfloat16)
    xh = torch.full(((nc + 15) // 16 * 16, n_in), float("nan"), dtype=torch.float16, device="cuda")
    xl = torch.full_like(xh, float("nan"))
    xsum = torch.full((xh.shape[0], n_in // 32), float("nan"), dtype=torch.float32, device="cuda")
    xs = torch.empty(nc, dtype=torch.float32, device="cuda")
    say("mm input", f32, n_in)
    nmq.check(nmq.lib().nmq_mm_input(xd.data_ptr(), int(f32), xh.data_ptr(), xl.data_ptr(), xsum.data_ptr(),
                                     xs.data_ptr(), n_in, nc, nmq.stream_ptr()))
    torch.cuda.synchronize()
    rh, rl, rsum, rs = oracle.mm_input(x)
    pad = (nc + 15) // 16 * 16 - nc
    for got, ref in ((xh, rh), (xl, rl)):
        ref = np.concatenate([ref, np.zeros((pad, n_in), np.float16)])
        got = _operand_order(host(got), n_in)
        # exact values; the sign of a zero is not specified (-0 input may come out as xh = +0, xl = -0)
        assert not np.isnan(got).any() and np.array_equal(got, ref)
    g = xh.shape[0] // 16
    got = host(xsum).reshape(g, n_in // 32, 16).transpose(0, 2, 1).reshape(16 * g, n_in // 32)
    ref = np.concatenate([rsum, np.zeros((pad, n_in // 32), np.float32)])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(host(xs), rs)


def _operand_order(a: np.ndarray, n_in: int) -> np.ndarray:
    """nmq_mm_input's operand order back to token-major rows: value k of token t sits at
    ((t/16 * n_in/32 + k/32) * 64 + (k%32)/8 * 16 + t%16) * 8 + k%8."""
    g = a.size // (16 * n_in)
    return a.reshape(g, n_in // 32, 4, 16, 8).transpose(0, 3, 1, 2, 4).reshape(16 * g, n_in)


def _mm_run(nmq, fmt, raw_d, x_np, n_out, n_in):
    from ggufengine_amd.gguf_types import TYPE_ID
    nc = x_np.shape[0]
    xd = dev(x_np)
    xh = torch.empty((nc + 15) // 16 * 16, n_in, dtype=torch.float16, device="cuda")
    xl = torch.empty_like(xh)
    xsum = torch.empty(xh.shape[0], n_in // 32, dtype=torch.float32, device="cuda")
    xs = torch.empty(nc, dtype=torch.float32, device="cuda")
    y = torch.full((nc, n_out), float("nan"), device="cuda")
    L = nmq.lib()
    nmq.check(L.nmq_mm_input(xd.data_ptr(), 1, xh.data_ptr(), xl.data_ptr(), xsum.data_ptr(), xs.data_ptr(), n_in, nc,
                             nmq.stream_ptr()))
    nmq.check(L.nmq_mm(TYPE_ID[fmt], raw_d.data_ptr(), xh.data_ptr(), xl.data_ptr(), xsum.data_ptr(), xs.data_ptr(),
                       y.data_ptr(), n_out, n_in, nc, nmq.stream_ptr()))
    torch.cuda.synchronize()
    return host(y)


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("tiles,groups", [("1", "0"), ("2", "0"), ("4", "0"), ("4", "1"), ("2", "3")])
def test_mm_tokens(nmq, oracle, tune, fmt, tiles, groups):
    """1..112 tokens (1..4 groups of 16 per launch, launches of 64) with 1, 2 and 4 row tiles per
    workgroup and all, one or three token groups per workgroup (three: the last workgroup of 4 groups
    repeats the last one, unstored): against the dequantised weights times the same two-stage input
    (only the order of the fp32 sums differs) and times the exact input.  Shapes: partial tiles and
    workgroups whose tiles lie past the matrix (200, 37 rows), one block per row (256: three of the
    four K quarters empty), an odd number of blocks per quarter (1280)."""
    tune(MMH_T=int(tiles))
    tune(MMH_G=int(groups))
    for n_out, n_in in ((200, 1280), (37, 256), (64, 4096)):
        raw = random_blocks(fmt, n_out * n_in // 256, seed=103)
        raw_d = dev(raw)
        for nc in (1, 5, 16, 17, 33, 64, 65, 112):
            x = np.random.default_rng(104 + nc).standard_normal((nc, n_in)).astype(np.float32)
            x[:, 7] = 30.0
            x[nc // 2, :] *= 1e-3
            say("mm", fmt, tiles, groups, n_out, n_in, nc)
            y = _mm_run(nmq, fmt, raw_d, x, n_out, n_in)
            ref_same = oracle.mv_deq(fmt, raw, n_out, n_in, oracle.mm_x(x).astype(np.float32))
            assert oracle.rel_err_rows(y, ref_same).max() <= 1e-5, (fmt, n_out, n_in, nc)
            err = oracle.rel_err_rows(y, oracle.mv_deq(fmt, raw, n_out, n_in, x))
            assert err.max() <= MM_TOL, (fmt, n_out, n_in, nc, float(err.max()))


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K"])
def test_mm_mirror_112_tokens(nmq, oracle, fmt):
    """mmvq.mm over the reference's MMQ range (17..112 tokens, MMQ_BIS) on a Llama-width matrix, fp32
    and bf16 input, and its input shared inside eingang_teilen()."""
    from ggufengine_amd import mmvq
    n_out, n_in, nc = 512, 4096, 112
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=95)
    x = np.random.default_rng(96).standard_normal((nc, n_in)).astype(np.float32)
    say("mm mirror", fmt, nc)
    raw_d = dev(raw)
    y = mmvq.mm(fmt, raw_d, dev(x), n_out, n_in)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (nc, n_out)
    assert oracle.rel_err_rows(host(y), oracle.mv_deq(fmt, raw, n_out, n_in, x)).max() <= MM_TOL
    xb = dev(x).to(torch.bfloat16)
    with mmvq.eingang_teilen():
        y1 = mmvq.mm(fmt, raw_d, xb, n_out, n_in)
        y2 = mmvq.mm(fmt, raw_d, xb, n_out, n_in)
    torch.cuda.synchronize()
    ref = oracle.mv_deq(fmt, raw, n_out, n_in, oracle.round_bf16(x))
    assert oracle.rel_err_rows(host(y1), ref).max() <= MM_TOL
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("fmt", FMTS)
def test_mv_tokens_dot4_kernel(nmq, oracle, tune, fmt):
    """2..8 tokens on the dot4 kernel (the path below each format's matrix-core threshold), forced for
    every token count."""
    n_out, n_in = 200, 4096
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=71)
    from ggufengine_amd.gguf_types import TYPE_ID
    tune(MVM=0)
    tune(MVT_MAX=1)
    for nc in (2, 5, 8, 13):                   # 13: launches of 8 and 5
        x = np.random.default_rng(72 + nc).standard_normal((nc, n_in)).astype(np.float32)
        e = quant_dev(dev(x))
        y = torch.full((nc, n_out), float("nan"), device="cuda")
        say("mv tokens dot4", fmt, nc)
        raw_d = dev(raw)  # kept alive until the launch has run
        nmq.check(nmq.lib().nmq_mv(TYPE_ID[fmt], raw_d.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                                   e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, nc,
                                   nmq.stream_ptr()))
        torch.cuda.synchronize()
        _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "Q8_0", "Q4_0"])
def test_mv_long_rows_several_tiles(nmq, oracle, fmt):
    """8 tokens of 14336 values exceed the LDS budget: the input goes through in K tiles."""
    n_out, n_in, nc = 96, 14336, 8
    raw = random_blocks(fmt, n_out * n_in // BV[fmt], seed=51)
    x = np.random.default_rng(52).standard_normal((nc, n_in)).astype(np.float32)
    from ggufengine_amd import mmvq, qlinear
    from ggufengine_amd.gguf_types import TYPE_ID
    say("mv tiles", fmt)
    if fmt in mmvq.FORMATE:
        y = mmvq.mv(fmt, dev(raw), dev(x), n_out, n_in)
    else:
        y = qlinear.build_quant_linear(dev(raw), TYPE_ID[fmt], n_out, n_in).forward_f32(dev(x))
    torch.cuda.synchronize()
    _check_mv(oracle, fmt, raw, n_out, n_in, x, y)


# ---- expert gather --------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", FMTS)
def test_experts_shared_and_own_input(nmq, oracle, fmt):
    """5 experts of 12 x 768 (the reference's test_alle_formate shape, test_gguf_iq.py:207-221):
    ids [4, 0, 2], one shared input and one input per expert."""
    from ggufengine_amd import cudakern
    n_exp, n_out, n_in = 5, 12, 768
    raw = random_blocks(fmt, n_exp * n_out * n_in // BV[fmt], seed=61)
    per = raw.size // n_exp
    rawd = dev(raw).view(n_exp, per)
    ids = torch.tensor([4, 0, 2], device="cuda")
    rng = np.random.default_rng(62)
    x = rng.standard_normal(n_in).astype(np.float32)
    a = rng.standard_normal((3, n_in)).astype(np.float32)
    say("experts", fmt)
    y1 = cudakern.mv(fmt, rawd, ids, dev(x), n_out, n_in)
    y2 = cudakern.mv(fmt, rawd, ids, dev(a), n_out, n_in)
    # address-table form: each expert's bytes somewhere else, raw not read
    copies = [dev(raw[e * per:(e + 1) * per]) for e in range(n_exp)]
    adressen = torch.tensor([c.data_ptr() for c in copies], dtype=torch.int64, device="cuda")
    y3 = cudakern.mv(fmt, None, ids, dev(a), n_out, n_in, adressen=adressen)
    torch.cuda.synchronize()
    xb, ab = oracle.round_bf16(x), oracle.round_bf16(a)
    for j, e in enumerate([4, 0, 2]):
        re = raw[e * per:(e + 1) * per]
        _check_mv(oracle, fmt, re, n_out, n_in, xb[None], y1[j:j + 1])
        _check_mv(oracle, fmt, re, n_out, n_in, ab[j:j + 1], y2[j:j + 1])
        _check_mv(oracle, fmt, re, n_out, n_in, ab[j:j + 1], y3[j:j + 1])


# ---- unpack ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bf16_exact(nmq, oracle, fmt):
    small = BV[fmt] == 32                             # odd Q4_0 / Q8_0 count: last pair half
    n_blocks = 25 if small else 5
    raw = random_blocks(fmt, n_blocks, seed=71)
    out = torch.empty(n_blocks * BV[fmt], dtype=torch.bfloat16, device="cuda")
    from ggufengine_amd.gguf_types import TYPE_ID
    say("dequant", fmt, n_blocks)
    raw_d = dev(raw)  # kept alive until the launch has run
    nmq.check(nmq.lib().nmq_dequant_bf16(TYPE_ID[fmt], raw_d.data_ptr(), out.data_ptr(), n_blocks,
                                         nmq.stream_ptr()))
    torch.cuda.synchronize()
    ref = oracle.round_bf16(oracle.dequant(fmt, raw))
    assert np.array_equal(out.float().cpu().numpy().view(np.uint32), ref.view(np.uint32))


# ---- graph capture ---------------------------------------------------------------------------------------

def test_graph_capture_replays(nmq, oracle):
    """Quantise + mat-vec + expert gather captured once, replayed with new inputs and new expert ids
    (the reference's test_im_cuda_graph, test_gguf_iq.py:240-256); each replay equals the eager result."""
    from ggufengine_amd import cudakern, mmvq
    n_out, n_in = 512, 1024
    raw = random_blocks("Q4_K", n_out * n_in // 256, seed=81)
    rawd = dev(raw)
    xraw = random_blocks("IQ2_XXS", 3 * 8 * 512 // 256, seed=82)
    xrawd = dev(xraw).view(3, -1)
    x = torch.zeros(n_in, device="cuda")
    xe = torch.zeros(512, device="cuda")
    ids = torch.tensor([2, 1], device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mmvq.mv("Q4_K", rawd, x, n_out, n_in)
        cudakern.mv("IQ2_XXS", xrawd, ids, xe, 8, 512)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    say("graph capture")
    with torch.cuda.graph(g):
        y = mmvq.mv("Q4_K", rawd, x, n_out, n_in)
        ye = cudakern.mv("IQ2_XXS", xrawd, ids, xe, 8, 512)
    rng = np.random.default_rng(83)
    for rep in range(4):
        xv = rng.standard_normal(n_in).astype(np.float32)
        xev = rng.standard_normal(512).astype(np.float32)
        x.copy_(torch.from_numpy(xv))
        xe.copy_(torch.from_numpy(xev))
        sel = [rep % 3, (rep + 1) % 3]
        ids.copy_(torch.tensor(sel))
        g.replay()
        torch.cuda.synchronize()
        eager = mmvq.mv("Q4_K", rawd, x, n_out, n_in)
        eager_e = cudakern.mv("IQ2_XXS", xrawd, ids, xe, 8, 512)
        torch.cuda.synchronize()
        assert torch.equal(y, eager), rep
        assert torch.equal(ye, eager_e), rep
        _check_mv(oracle, "Q4_K", raw, n_out, n_in, xv[None], y[None])


# ---- several matrices on one input in one launch ---------------------------------------------------------

# (format, n_in, rows of each matrix): chunk kernel, persistent kernel, long rows, a half Q8_0 unit,
# four matrices, and rows too long for the one-token kernels (one launch per matrix then)
MULTI = [("Q4_K", 4096, (4096, 1024, 1024)), ("Q4_K", 4096, (7000, 7000)), ("Q6_K", 14336, (300, 200)),
         ("Q8_0", 1056, (37, 100, 5, 64)), ("IQ2_XXS", 2048, (500, 700, 900)), ("Q4_0", 4096, (1000, 3000)),
         ("Q4_K", 32768, (50, 70))]


@pytest.mark.parametrize("fmt,n_in,rows", MULTI)
def test_mv_multi_equals_single_launches(nmq, oracle, fmt, n_in, rows):
    """nmq_mv_multi: every matrix's output bit for bit what nmq_mv gives for it alone, and within the
    parity bar of the oracle."""
    import ctypes
    from ggufengine_amd.gguf_types import TYPE_ID
    raws = [random_blocks(fmt, r * n_in // BV[fmt], seed=90 + i) for i, r in enumerate(rows)]
    x = np.random.default_rng(95).standard_normal((1, n_in)).astype(np.float32)
    e = quant_dev(dev(x))
    ws = [dev(r) for r in raws]
    ys = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    alone = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    k = len(rows)
    say("mv multi", fmt, n_in, rows)
    L = nmq.lib()
    args = (e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr())
    nmq.check(L.nmq_mv_multi(TYPE_ID[fmt], k, (ctypes.c_void_p * k)(*[w.data_ptr() for w in ws]),
                             (ctypes.c_int * k)(*rows), (ctypes.c_void_p * k)(*[y.data_ptr() for y in ys]),
                             *args, n_in, nmq.stream_ptr()))
    for w, y, r in zip(ws, alone, rows):
        nmq.check(L.nmq_mv(TYPE_ID[fmt], w.data_ptr(), *args, y.data_ptr(), r, n_in, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    for y, ya in zip(ys, alone):
        assert torch.equal(y, ya)
    _check_mv(oracle, fmt, raws[-1], rows[-1], n_in, x, ys[-1])


def test_mv_mehrere_mirror(nmq, oracle):
    """mmvq.mv_mehrere: q, k, v of one Eingang, and more matrices than one launch takes."""
    from ggufengine_amd import mmvq
    n_in = 1024
    rows = (256, 64, 64, 128, 32)
    raws = [random_blocks("Q4_K", r * n_in // 256, seed=97 + i) for i, r in enumerate(rows)]
    x = np.random.default_rng(98).standard_normal(n_in).astype(np.float32)
    say("mv_mehrere")
    ws = [dev(r) for r in raws]
    xt = dev(x)
    ys = mmvq.mv_mehrere("Q4_K", ws, xt, rows, n_in)
    single = [mmvq.mv("Q4_K", w, xt, r, n_in) for w, r in zip(ws, rows)]
    torch.cuda.synchronize()
    for y, s in zip(ys, single):
        assert torch.equal(y, s)
    with pytest.raises(ValueError):
        mmvq.mv_mehrere("Q4_K", ws[:2], xt, rows[:1], n_in)


# ---- input given as values: the launch quantises it itself ---------------------------------------------

# (format, n_in, rows of each matrix): chunk kernel, persistent kernel, long rows (several staging
# rounds), a half Q8_0 unit with a padded staging tail, strided formats, segments
VALUES = [("Q4_K", 4096, (4096,)), ("Q4_K", 4096, (7000, 7000)), ("Q6_K", 14336, (300,)), ("Q8_0", 1056, (37, 100)),
          ("TQ2_0", 2048, (500,)), ("IQ2_XXS", 4096, (300, 200, 100)), ("Q4_0", 768, (2048,)),
          ("Q6_K", 4096, (4096, 1024))]


@pytest.mark.parametrize("fmt,n_in,rows", VALUES)
@pytest.mark.parametrize("mode", ["f32", "f32_bf16", "bf16"])
def test_mv_values_equal_quant_then_mv(nmq, oracle, fmt, n_in, rows, mode):
    """nmq_mv_x: each output bit for bit what nmq_quant_q8 followed by nmq_mv gives (the staging
    quantises with the same arithmetic), within the parity bar of the oracle."""
    import ctypes
    from ggufengine_amd.gguf_types import TYPE_ID
    raws = [random_blocks(fmt, r * n_in // BV[fmt], seed=110 + i) for i, r in enumerate(rows)]
    rng = np.random.default_rng(111)
    x = (rng.standard_normal(n_in) * np.repeat(10.0 ** rng.uniform(-3, 2, n_in // 32), 32)).astype(np.float32)
    x[32:64] = 0.0                                     # a zero group
    xt = dev(x)
    xin = xt.to(torch.bfloat16) if mode == "bf16" else xt
    xm = {"f32": nmq.X_F32, "f32_bf16": nmq.X_F32_BF16, "bf16": nmq.X_BF16}[mode]
    ws = [dev(r) for r in raws]
    k = len(rows)
    ys = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    ref = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    say("mv values", fmt, n_in, rows, mode)
    L = nmq.lib()
    nmq.check(L.nmq_mv_x(TYPE_ID[fmt], k, (ctypes.c_void_p * k)(*[w.data_ptr() for w in ws]), (ctypes.c_int * k)(*rows),
                         (ctypes.c_void_p * k)(*[y.data_ptr() for y in ys]), xin.data_ptr(), xm, None, n_in,
                         nmq.stream_ptr()))
    from ggufengine_amd import mmvq
    e = mmvq.Eingang(n=n_in, device=torch.device("cuda"))
    qmode = {"f32": 1, "f32_bf16": 2, "bf16": 0}[mode]
    nmq.check(L.nmq_quant_q8(xin.data_ptr(), qmode, e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                             e.xs.data_ptr(), n_in, nmq.stream_ptr()))
    for w, y, r in zip(ws, ref, rows):
        nmq.check(L.nmq_mv(TYPE_ID[fmt], w.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
                           e.xs.data_ptr(), y.data_ptr(), r, n_in, 1, nmq.stream_ptr()))
    torch.cuda.synchronize()
    for y, yr in zip(ys, ref):
        assert torch.equal(y, yr)
    xr = oracle.round_bf16(x) if mode != "f32" else x
    _check_mv(oracle, fmt, raws[0], rows[0], n_in, xr[None], ys[0])


@pytest.mark.parametrize("two", [False, True])
def test_experts_values(nmq, oracle, two):
    """nmq_mv_experts_x: fp32 tokens rounded to bf16 (the gate/up call) and bf16(silu(g) * u) (the down
    call) against the quantisation launches followed by the gathered launches, bit for bit."""
    from ggufengine_amd.gguf_types import TYPE_ID
    n_exp, n_out, n_in, Lt, k = 10, 256, 2048, 3, 4
    A = dev(random_blocks("Q4_K", n_exp * n_out * n_in // 256, seed=121))
    B = dev(random_blocks("Q4_K", n_exp * n_out * n_in // 256, seed=122))
    per = A.numel() // n_exp
    ids = torch.tensor(np.random.default_rng(123).integers(0, n_exp, Lt * k), dtype=torch.int64, device="cuda")
    rng = np.random.default_rng(124)
    x = dev(rng.standard_normal((Lt, n_in)).astype(np.float32))
    n_inst = (2 if two else 1) * Lt * k
    y = torch.full((n_inst, n_out), float("nan"), device="cuda")
    say("experts values", two)
    L = nmq.lib()
    nmq.check(L.nmq_mv_experts_x(TYPE_ID["Q4_K"], A.data_ptr(), B.data_ptr() if two else None, ids.data_ptr(),
                                 Lt * k, per, x.data_ptr(), nmq.X_F32_BF16, None, k, y.data_ptr(), n_out, n_in,
                                 nmq.stream_ptr()))
    from ggufengine_amd import mmvq
    e = mmvq.eingang_bf16(x)
    yr = torch.full_like(y, float("nan"))
    nmq.check(L.nmq_mv_experts(TYPE_ID["Q4_K"], A.data_ptr(), ids.data_ptr(), Lt * k, per, e.xq.data_ptr(),
                               e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k, yr.data_ptr(), n_out, n_in,
                               nmq.stream_ptr()))
    if two:
        nmq.check(L.nmq_mv_experts(TYPE_ID["Q4_K"], B.data_ptr(), ids.data_ptr(), Lt * k, per, e.xq.data_ptr(),
                                   e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k, yr[Lt * k:].data_ptr(),
                                   n_out, n_in, nmq.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(y, yr)
    # the down call: input bf16(silu(g) * u) of each slot's own rows (x_group 1), from fp32 g and u
    D = dev(random_blocks("Q6_K", n_exp * n_in * n_out // 256, seed=125))      # n_out -> n_in
    g = dev((rng.standard_normal((Lt * k, n_out)) * 3).astype(np.float32))
    u = dev(rng.standard_normal((Lt * k, n_out)).astype(np.float32))
    yd = torch.full((Lt * k, n_in), float("nan"), device="cuda")
    perd = D.numel() // n_exp
    nmq.check(L.nmq_mv_experts_x(TYPE_ID["Q6_K"], D.data_ptr(), None, ids.data_ptr(), Lt * k, perd, g.data_ptr(),
                                 nmq.X_SILU_MUL_BF16, u.data_ptr(), 1, yd.data_ptr(), n_in, n_out, nmq.stream_ptr()))
    a = mmvq.Eingang(n=Lt * k * n_out, device=torch.device("cuda"))
    nmq.check(L.nmq_silu_mul_quant(g.data_ptr(), u.data_ptr(), a.xq.data_ptr(), a.xq2.data_ptr(), a.xd.data_ptr(),
                                   a.xs.data_ptr(), Lt * k * n_out, nmq.stream_ptr()))
    ydr = torch.full_like(yd, float("nan"))
    nmq.check(L.nmq_mv_experts(TYPE_ID["Q6_K"], D.data_ptr(), ids.data_ptr(), Lt * k, perd, a.xq.data_ptr(),
                               a.xq2.data_ptr(), a.xd.data_ptr(), a.xs.data_ptr(), 1, ydr.data_ptr(), n_in, n_out,
                               nmq.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(yd, ydr)


@pytest.mark.parametrize("nc", [2, 3, 4])
@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 4096), (1000, 2048), (513, 1024), (37, 256)])
def test_few_tokens_equal_one_by_one(nmq, oracle, tune, shape, nc):
    """2..4 tokens of Q4_K (speculative verification) in one launch of the few-token kernel (enabled up to
    4 tokens here): each token's output equals the one-token launch on that token bit for bit (the same
    decode and combine expression, one weight read for all), and the oracle within tolerance.  Covers
    64, 32 and 16 lanes per row and row counts that leave the last steps partial."""
    tune(MVT_MAX=4)
    n_out, n_in = shape
    raw = random_blocks("Q4_K", n_out * n_in // 256, seed=131 + n_in)
    x = np.random.default_rng(132 + n_out + nc).standard_normal((nc, n_in)).astype(np.float32)
    x[1, 5] = -25.0
    say("few tokens", shape, nc)
    e = quant_dev(dev(x))
    w = dev(raw)
    L = nmq.lib()
    y2 = torch.empty(nc, n_out, dtype=torch.float32, device="cuda")
    nmq.check(L.nmq_mv(12, w.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(),
                       y2.data_ptr(), n_out, n_in, nc, nmq.stream_ptr()))
    ys = []
    for t in range(nc):
        y1 = torch.empty(n_out, dtype=torch.float32, device="cuda")
        g = n_in // 32
        nmq.check(L.nmq_mv(12, w.data_ptr(), e.xq[t * n_in:].data_ptr(), e.xq2[t * n_in:].data_ptr(),
                           e.xd[t * g:].data_ptr(), e.xs[t * g:].data_ptr(), y1.data_ptr(), n_out, n_in, 1,
                           nmq.stream_ptr()))
        ys.append(y1)
    torch.cuda.synchronize()
    for t in range(nc):
        assert torch.equal(y2[t], ys[t]), (shape, nc, t)
    _check_mv(oracle, "Q4_K", raw, n_out, n_in, x, y2)


@pytest.mark.parametrize("nc", [2, 3, 4])
@pytest.mark.parametrize("shape", [(4096, 14336), (1000, 8448), (37, 16384)])
def test_few_tokens_long_rows_equal_one_by_one(nmq, oracle, shape, nc):
    """2..4 tokens of Q6_K with long rows (the layer's down projection) in one launch of the few-token
    long-row kernel: each token's output equals the one-token launch on that token bit for bit, and the
    oracle within tolerance.  Covers 3 and 4 units per lane and a last workgroup with idle waves."""
    n_out, n_in = shape
    raw = random_blocks("Q6_K", n_out * n_in // 256, seed=141 + n_in)
    x = np.random.default_rng(142 + n_out + nc).standard_normal((nc, n_in)).astype(np.float32)
    x[nc - 1, 9] = 40.0
    say("few tokens long rows", shape, nc)
    e = quant_dev(dev(x))
    w = dev(raw)
    L = nmq.lib()
    yn = torch.empty(nc, n_out, dtype=torch.float32, device="cuda")
    nmq.check(L.nmq_mv(14, w.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(),
                       yn.data_ptr(), n_out, n_in, nc, nmq.stream_ptr()))
    g = n_in // 32
    ys = []
    for t in range(nc):
        y1 = torch.empty(n_out, dtype=torch.float32, device="cuda")
        nmq.check(L.nmq_mv(14, w.data_ptr(), e.xq[t * n_in:].data_ptr(), e.xq2[t * n_in:].data_ptr(),
                           e.xd[t * g:].data_ptr(), e.xs[t * g:].data_ptr(), y1.data_ptr(), n_out, n_in, 1,
                           nmq.stream_ptr()))
        ys.append(y1)
    torch.cuda.synchronize()
    for t in range(nc):
        assert torch.equal(yn[t], ys[t]), (shape, nc, t)
    _check_mv(oracle, "Q6_K", raw, n_out, n_in, x, yn)


# ---- dense gate|up with the activation (nmq_mv_gate_up_act) ----------------------------------------------------

# (format, n_out, n_in, knobs): the Llama-3-8B shape, 8 and 4 rows per wave, several groups per workgroup
GATE_UP_ACT = [("Q4_K", 14336, 4096, {}), ("Q4_K", 14336, 4096, {"MVP_RPW": 4}),
               ("Q4_K", 14336, 4096, {"MVP_WGS": 7}), ("Q4_K", 1024, 2048, {}), ("Q4_K", 320, 1024, {"MVP_WGS": 3}),
               ("TQ2_0", 4096, 4096, {}), ("TQ2_0", 2048, 1536, {"MVP_RPW": 4, "MVP_WGS": 9}),
               ("IQ2_XXS", 4096, 4096, {}), ("IQ2_XXS", 1536, 2048, {"MVP_WGS": 11})]


@pytest.mark.parametrize("fmt,n_out,n_in,knobs", GATE_UP_ACT)
def test_gate_up_act_equals_two_launches(nmq, oracle, tune, fmt, n_out, n_in, knobs):
    """nmq_mv_gate_up_act (gate and up rows of 32-row groups in one workgroup, the activation and its
    two-stage input in the same launch) equals nmq_mv_x on both matrices followed by nmq_akt_q8 (silu, gelu)
    or nmq_silu_mul_quant (silu rounded to bf16), bit for bit, for fp32 input with and without the bf16
    rounding; and the activation against the oracle."""
    from ggufengine_amd import mmvq
    from ggufengine_amd.gguf_types import TYPE_ID
    tune(**knobs)
    Lb = nmq.lib()
    rawg = random_blocks(fmt, n_out * n_in // BV[fmt], seed=401 + n_out)
    rawu = random_blocks(fmt, n_out * n_in // BV[fmt], seed=402 + n_out)
    A, B = dev(rawg), dev(rawu)
    rng = np.random.default_rng(403 + n_in)
    x = dev(rng.standard_normal(n_in).astype(np.float32))
    t = TYPE_ID[fmt]
    a = torch.empty(n_out, device="cuda")
    say("gate_up_act", fmt, n_out, n_in, knobs)
    for mode, act in ((nmq.X_F32, nmq.ACT_SILU), (nmq.X_F32_BF16, nmq.ACT_SILU), (nmq.X_F32, nmq.ACT_GELU),
                      (nmq.X_F32_BF16, nmq.ACT_SILU | nmq.ACT_BF16)):
        y = torch.full((2, n_out), float("nan"), device="cuda")
        nmq.check(Lb.nmq_mv_x(t, 2, (ctypes.c_void_p * 2)(A.data_ptr(), B.data_ptr()), (ctypes.c_int * 2)(n_out, n_out),
                              (ctypes.c_void_p * 2)(y[0].data_ptr(), y[1].data_ptr()), x.data_ptr(), mode, None, n_in,
                              nmq.stream_ptr()))
        want = mmvq.Eingang(n=n_out, device=torch.device("cuda"))
        wp = (want.xq.data_ptr(), want.xq2.data_ptr(), want.xd.data_ptr(), want.xs.data_ptr())
        if act & nmq.ACT_BF16:
            nmq.check(Lb.nmq_silu_mul_quant(y[0].data_ptr(), y[1].data_ptr(), *wp, n_out, nmq.stream_ptr()))
        else:
            nmq.check(Lb.nmq_akt_q8(y[0].data_ptr(), y[1].data_ptr(), act & nmq.ACT_GELU, a.data_ptr(), *wp, n_out,
                                    nmq.stream_ptr()))
        got = mmvq.Eingang(n=n_out, device=torch.device("cuda"))
        for b in (got.xq, got.xq2):
            b.fill_(77)
        for b in (got.xd, got.xs):
            b.fill_(float("nan"))
        nmq.check(Lb.nmq_mv_gate_up_act(t, A.data_ptr(), B.data_ptr(), x.data_ptr(), mode, act, got.xq.data_ptr(),
                                        got.xq2.data_ptr(), got.xd.data_ptr(), got.xs.data_ptr(), n_out, n_in,
                                        nmq.stream_ptr()))
        torch.cuda.synchronize()
        for f in ("xq", "xq2", "xd", "xs"):
            assert torch.equal(getattr(got, f), getattr(want, f)), (f, mode, act)
        if mode == nmq.X_F32 and act == nmq.ACT_SILU:
            # the activation against the oracle's products
            g = oracle.mv_deq(fmt, rawg, n_out, n_in, x.cpu().numpy()[None])[0]
            u = oracle.mv_deq(fmt, rawu, n_out, n_in, x.cpu().numpy()[None])[0]
            ref = oracle.akt(g, u)
            xd = np.repeat(got.xd.cpu().numpy().astype(np.float64), 32)
            rec = xd * (got.xq.cpu().numpy() + got.xq2.cpu().numpy() / 254.0)
            assert np.max(np.abs(rec - ref)) <= 2e-3 * np.abs(ref).max()


def test_gate_up_act_refuses_what_it_does_not_take(nmq):
    from ggufengine_amd.gguf_types import TYPE_ID
    Lb = nmq.lib()
    a = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(4096, device="cuda")
    q = torch.zeros(4096, dtype=torch.int8, device="cuda")
    f = torch.zeros(128, device="cuda")

    def call(fmt, n_out, n_in, mode, act=0):
        return Lb.nmq_mv_gate_up_act(fmt, a.data_ptr(), a.data_ptr(), x.data_ptr(), mode, act, q.data_ptr(),
                                     q.data_ptr(), f.data_ptr(), f.data_ptr(), n_out, n_in, nmq.stream_ptr())
    assert call(TYPE_ID["Q6_K"], 64, 1024, nmq.X_F32) == nmq.NMQ_ERR_SHAPE   # not a hand-read format
    assert call(TYPE_ID["Q4_K"], 48, 1024, nmq.X_F32) == nmq.NMQ_ERR_SHAPE   # groups of 32 rows
    assert call(TYPE_ID["Q4_K"], 64, 8192, nmq.X_F32) == nmq.NMQ_ERR_SHAPE   # rows over 4096 values
    assert call(TYPE_ID["Q4_K"], 64, 1024, nmq.X_BF16) == nmq.NMQ_ERR_SHAPE  # fp32 input only
    assert call(TYPE_ID["Q4_K"], 64, 1024, nmq.X_F32, 4) == nmq.NMQ_ERR_ARG  # unknown activation
    torch.cuda.synchronize()
