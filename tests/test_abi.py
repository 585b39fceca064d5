"""libnmq.so on the CPU: it loads, exports every entry point include/nmq.h declares, and rejects bad
arguments before anything reaches a device (no compute call is made here)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "nmq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nmq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from ggufengine_amd import _native
    return _native.lib()


def test_exports_every_declared_symbol(L):
    names = declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(L, n), n


def test_format_table(L):
    bv, bb = ctypes.c_int(), ctypes.c_int()
    from ggufengine_amd.gguf_types import GGML_TYPES
    for t, (name, v, b) in GGML_TYPES.items():
        assert L.nmq_format_info(t, ctypes.byref(bv), ctypes.byref(bb)) == 0, name
        assert (bv.value, bb.value) == (v, b), name
    assert L.nmq_format_info(3, None, None) == -1          # Q4_1: not served
    from ggufengine_amd import _native
    assert L.nmq_abi_version() == _native.ABI_VERSION == 2


def test_rejects_bad_arguments_without_launching(L):
    from ggufengine_amd import _native
    buf = ctypes.create_string_buffer(4096)
    a16 = (ctypes.addressof(buf) + 15) // 16 * 16
    # NULL weight pointer, bad n_in, bad format, bad token count: all rejected before a launch
    assert L.nmq_mv(12, None, a16, a16, a16, a16, a16, 4, 256, 1, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv(12, a16, a16, a16, a16, a16, a16, 4, 300, 1, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mv(13, a16, a16, a16, a16, a16, a16, 4, 256, 1, None) == _native.NMQ_ERR_FORMAT
    assert L.nmq_mv(12, a16, a16, a16, a16, a16, a16, 4, 256, 0, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv(12, a16 + 2, a16, a16, a16, a16, a16, 4, 256, 1, None) == _native.NMQ_ERR_ARG  # Q4_K needs 16 B
    assert L.nmq_mv(14, a16, a16 + 1, a16, a16, a16, a16, 4, 256, 1, None) == _native.NMQ_ERR_ARG  # xq alignment
    assert L.nmq_quant_q8(a16, 1, a16, a16, a16, a16, 33, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mv_experts(12, a16, None, 2, 0, a16, a16, a16, a16, 1, a16, 4, 256, None) == _native.NMQ_ERR_ARG
    # per-expert stride smaller than one matrix
    assert L.nmq_mv_experts(12, a16, a16, 2, 144, a16, a16, a16, a16, 1, a16, 4, 256, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_dequant_bf16(12, a16, a16, 0, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_encode(12, None, 256, a16, 1) == _native.NMQ_ERR_ARG
    assert b"block format" in L.nmq_strerror(-1)
    # quantisation modes: 0 bf16, 1 fp32, 2 fp32 rounded to bf16; anything else is refused
    assert L.nmq_quant_q8(a16, 3, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_quant_q8(a16, -1, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    # fused expert entry points
    assert L.nmq_silu_mul_quant(None, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_silu_mul_quant(a16, a16 + 2, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_silu_mul_quant(a16, a16, a16, a16, a16, a16, 48, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mv_experts2(12, a16, None, a16, 2, 0, a16, a16, a16, a16, 1, a16, 4, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_experts2(12, a16, a16, None, 2, 0, a16, a16, a16, a16, 1, a16, 4, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_experts2(12, a16, a16, a16, 40000, 4 * 144, a16, a16, a16, a16, 1, a16, 4, 256,
                             None) == _native.NMQ_ERR_ARG      # 2 x 40000 instances exceed the grid
    assert L.nmq_mv_experts2(12, a16, a16, a16, 2, 144, a16, a16, a16, a16, 1, a16, 4, 256,
                             None) == _native.NMQ_ERR_SHAPE    # stride smaller than one matrix
    assert L.nmq_moe_combine(None, a16, 1, 8, 64, a16, None) == _native.NMQ_ERR_ARG
    assert L.nmq_moe_combine(a16, a16, 0, 8, 64, a16, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_moe_combine(a16, a16, 1, 8, 64, a16 + 1, None) == _native.NMQ_ERR_ARG
    # several matrices in one launch: 1..4 matrices, host arrays present, sizes in range
    W = (ctypes.c_void_p * 5)(*([a16] * 5))
    N = (ctypes.c_int * 5)(*([4] * 5))
    Y = (ctypes.c_void_p * 5)(*([a16] * 5))
    assert L.nmq_mv_multi(12, 0, W, N, Y, a16, a16, a16, a16, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_multi(12, 5, W, N, Y, a16, a16, a16, a16, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_multi(12, 2, None, N, Y, a16, a16, a16, a16, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_multi(12, 2, W, N, Y, a16, a16, a16, a16, 300, None) == _native.NMQ_ERR_SHAPE
    N0 = (ctypes.c_int * 2)(4, 0)
    assert L.nmq_mv_multi(12, 2, W, N0, Y, a16, a16, a16, a16, 256, None) == _native.NMQ_ERR_SHAPE
    # input given as values: mode range, alignment, second operand, row length
    W1 = (ctypes.c_void_p * 1)(a16)
    N1 = (ctypes.c_int * 1)(4)
    Y1 = (ctypes.c_void_p * 1)(a16)
    assert L.nmq_mv_x(12, 1, W1, N1, Y1, None, 1, None, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_x(12, 1, W1, N1, Y1, a16, 4, None, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_x(12, 1, W1, N1, Y1, a16 + 8, 1, None, 256, None) == _native.NMQ_ERR_ARG  # fp32: 16 B
    assert L.nmq_mv_x(12, 1, W1, N1, Y1, a16, 3, None, 256, None) == _native.NMQ_ERR_ARG      # silu: x2
    assert L.nmq_mv_x(12, 1, W1, N1, Y1, a16, 1, None, 16384 + 256, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mv_experts_x(12, a16, None, None, 2, 0, a16, 1, None, 1, a16, 4, 256, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_experts_x(12, a16, a16, a16, 40000, 4 * 144, a16, 1, None, 1, a16, 4, 256,
                              None) == _native.NMQ_ERR_ARG
    assert L.nmq_mv_experts_x(12, a16, None, a16, 2, 144, a16, 1, None, 1, a16, 4, 256,
                              None) == _native.NMQ_ERR_SHAPE
    # fused producers of the one-token step
    h, r, o = a16, a16 + 1024, a16 + 2048
    assert L.nmq_norm_q8(None, None, 1.0, None, a16, 1e-6, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_norm_q8(h, r, 1.0, None, a16, 1e-6, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_norm_q8(h, r, 1.0, h + 64, a16, 1e-6, a16, a16, a16, a16, a16, 32,
                         None) == _native.NMQ_ERR_ARG          # hout overlaps h
    assert L.nmq_norm_q8(h, r, 1.0, r, a16, 1e-6, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_norm_q8(h, r, 1.0, o, a16, 1e-6, a16, a16, a16, a16, a16, 48, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_norm_q8(h, None, 1.0, None, a16, 1e-6, a16, a16, a16, a16, a16, 65536 + 32,
                         None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_akt_q8(None, None, 0, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_akt_q8(a16, None, 2, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_akt_q8(a16, a16 + 2, 1, a16, a16, a16, a16, a16, 32, None) == _native.NMQ_ERR_ARG
    assert L.nmq_akt_q8(a16, None, 1, a16, a16, a16, a16, a16, 40, None) == _native.NMQ_ERR_SHAPE
    # several tokens on the fp16 matrix cores: Q4_K and Q6_K only, whole 256-value blocks
    assert L.nmq_mm_input(None, 1, a16, a16, a16, a16, 256, 2, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mm_input(a16, 2, a16, a16, a16, a16, 256, 2, None) == _native.NMQ_ERR_ARG      # x kind
    assert L.nmq_mm_input(a16, 1, a16 + 2, a16, a16, a16, 256, 2, None) == _native.NMQ_ERR_ARG  # xh alignment
    assert L.nmq_mm_input(a16, 1, a16, a16, None, a16, 256, 2, None) == _native.NMQ_ERR_ARG     # xsum
    assert L.nmq_mm_input(a16, 1, a16, a16, a16, a16, 260, 2, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mm_input(a16, 1, a16, a16, a16, a16, 256, 0, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mm(8, a16, a16, a16, a16, a16, a16, 4, 256, 2, None) == _native.NMQ_ERR_FORMAT   # Q8_0
    assert L.nmq_mm(12, a16, a16, a16, a16, a16, a16, 4, 288, 2, None) == _native.NMQ_ERR_SHAPE
    assert L.nmq_mm(12, a16, None, a16, a16, a16, a16, 4, 256, 2, None) == _native.NMQ_ERR_ARG
    assert L.nmq_mm(14, a16, a16, a16 + 8, a16, a16, a16, 4, 256, 2, None) == _native.NMQ_ERR_ARG  # xl alignment
    assert L.nmq_mm(12, a16, a16, a16, a16, a16, a16, 4, 256, 0, None) == _native.NMQ_ERR_ARG


def test_python_api_without_gpu():
    import torch
    from ggufengine_amd import cudakern, mmvq, qlinear
    from ggufengine_amd.gguf_types import GGUFError
    if torch.cuda.is_available():
        pytest.skip("CPU-only behaviour")
    assert not mmvq.verfuegbar("cpu", "Q4_K", 4096)
    assert not cudakern.verfuegbar("cpu", "IQ2_XXS", 4096)
    assert not qlinear.kernel_available(torch.device("cpu"))
    assert cudakern.mm_bis("cpu") == 1
    with pytest.raises(ValueError):
        cudakern.mm("Q8_0", torch.zeros(34, dtype=torch.uint8), torch.zeros(2, 32), 1, 32)
    with pytest.raises(GGUFError):
        qlinear.build_quant_linear(torch.zeros(100, dtype=torch.uint8), 12, 2, 256)
    with pytest.raises(ValueError):
        mmvq.Eingang(n=33, device="cpu")
    assert qlinear.quantizable(12, 4096, 4096) and not qlinear.quantizable(16, 4096, 4096)
    assert not mmvq.schritt_moeglich("cpu", 32, 8, 128)


def test_tuning_knobs_set_get_and_reset(L):
    """Launch-plan overrides go through nmq_set_tuning only (no environment variable is read): a value
    set is read back, NMQ_TUNE_DEFAULT restores the default, unknown names are refused."""
    from ggufengine_amd import _native
    assert _native.get_tuning("MVM") is None
    with _native.tuning(MVM=2, NMQ_MVT_MAX=1):
        assert _native.get_tuning("MVM") == 2 and _native.get_tuning("MVT_MAX") == 1
        assert _native.get_tuning("NMQ_MVM") == 2
    assert _native.get_tuning("MVM") is None and _native.get_tuning("MVT_MAX") is None
    with pytest.raises(ValueError):
        _native.set_tuning("NOT_A_KNOB", 1)
    assert L.nmq_set_tuning(None, 1) == _native.NMQ_ERR_ARG
    os.environ["NMQ_MVM"] = "0"
    try:
        assert _native.get_tuning("MVM") is None      # the environment changes nothing
    finally:
        del os.environ["NMQ_MVM"]


def test_quantlinear_has_no_int4_planes_and_every_format_stays_packed():
    """models/moe.py `_StapelTeil` stacks QuantLinear.mats for torch's int4 kernel: this library's
    QuantLinear has none and says so; its expert tensors take the gathered path instead, because every
    format is in cudakern.IMMER_GEPACKT (the reference loader's `packed_type`)."""
    from ggufengine_amd import cudakern, qlinear
    with pytest.raises(TypeError, match="aus_quantlinear"):
        qlinear.QuantLinear.mats.fget(object())
    assert cudakern.IMMER_GEPACKT == frozenset(cudakern.FORMATE)


def test_moe_down_checks_without_launching(L):
    """nmq_moe_down sizes its workspace and refuses bad arguments before anything is launched."""
    from ggufengine_amd import _native
    need = ctypes.c_int64(0)
    assert L.nmq_moe_down_work_bytes(14, 4, 8, 2048, 768, ctypes.byref(need)) == 0
    assert need.value == 0                                       # one launch, the sums in LDS
    assert L.nmq_moe_down_work_bytes(14, 4, 8, 2048, 5120, ctypes.byref(need)) == 0
    assert need.value == 4 * 8 * 2048 * 4                        # rows too long: slots through a workspace
    assert L.nmq_moe_down_work_bytes(14, 0, 8, 2048, 768, ctypes.byref(need)) == _native.NMQ_ERR_ARG
    assert L.nmq_moe_down_work_bytes(13, 1, 8, 2048, 768, ctypes.byref(need)) == _native.NMQ_ERR_FORMAT
    buf = ctypes.create_string_buffer(1 << 16)
    a = (ctypes.addressof(buf) + 255) // 256 * 256
    args = dict(fmt=14, w=a, ids=a, L=1, k=8, per=2048 * 3 * 210, x=a, mode=_native.X_SILU_MUL_BF16, x2=a, wts=a,
                out=a, n_out=2048, n_in=768, work=a, work_bytes=1 << 14)

    def call(**kw):
        v = {**args, **kw}
        return L.nmq_moe_down(v["fmt"], v["w"], v["ids"], v["L"], v["k"], v["per"], v["x"], v["mode"], v["x2"],
                              v["wts"], v["out"], v["n_out"], v["n_in"], v["work"], v["work_bytes"], None)
    assert call(ids=None) == _native.NMQ_ERR_ARG
    assert call(wts=None) == _native.NMQ_ERR_ARG
    assert call(k=0) == _native.NMQ_ERR_ARG
    long = dict(n_in=5120, per=2048 * 20 * 210)
    assert call(work=a + 16, **long) == _native.NMQ_ERR_ARG       # not 256-byte aligned
    assert call(work_bytes=16, **long) == _native.NMQ_ERR_SHAPE   # too small
    assert call(n_in=700) == _native.NMQ_ERR_SHAPE                # not whole blocks


def test_moe_gate_up_and_down_q8_check_without_launching(L):
    """nmq_moe_gate_up and nmq_moe_down_q8 refuse bad arguments before anything is launched."""
    from ggufengine_amd import _native
    buf = ctypes.create_string_buffer(1 << 16)
    a = (ctypes.addressof(buf) + 255) // 256 * 256
    gu = dict(fmt=12, wg=a, wu=a, ids=a, L=1, k=8, per=768 * 8 * 144, x=a, mode=_native.X_F32_BF16, xq=a, xq2=a,
              xd=a, xs=a, n_out=768, n_in=2048)

    def gate_up(**kw):
        v = {**gu, **kw}
        return L.nmq_moe_gate_up(v["fmt"], v["wg"], v["wu"], v["ids"], v["L"], v["k"], v["per"], v["x"], v["mode"],
                                 v["xq"], v["xq2"], v["xd"], v["xs"], v["n_out"], v["n_in"], None)
    assert gate_up(ids=None) == _native.NMQ_ERR_ARG
    assert gate_up(wu=None) == _native.NMQ_ERR_ARG
    assert gate_up(xq=a + 1) == _native.NMQ_ERR_ARG                     # two-stage output: 16-byte aligned
    assert gate_up(mode=_native.X_SILU_MUL_BF16) == _native.NMQ_ERR_ARG  # no second operand taken
    assert gate_up(L=4096, k=16) == _native.NMQ_ERR_ARG                  # more than 32767 slots
    assert gate_up(n_out=760, per=760 * 8 * 144) == _native.NMQ_ERR_SHAPE  # groups of 32 rows
    assert gate_up(per=100) == _native.NMQ_ERR_SHAPE                     # experts overlap
    assert gate_up(fmt=13) == _native.NMQ_ERR_FORMAT
    dn = dict(fmt=14, w=a, ids=a, L=1, k=8, per=2048 * 20 * 210, xq=a, xq2=a, xd=a, xs=a, wts=a, out=a, n_out=2048,
              n_in=5120, work=a, work_bytes=1 << 14)

    def down(**kw):
        v = {**dn, **kw}
        return L.nmq_moe_down_q8(v["fmt"], v["w"], v["ids"], v["L"], v["k"], v["per"], v["xq"], v["xq2"], v["xd"],
                                 v["xs"], v["wts"], v["out"], v["n_out"], v["n_in"], v["work"], v["work_bytes"], None)
    assert down(ids=None) == _native.NMQ_ERR_ARG
    assert down(xs=None) == _native.NMQ_ERR_ARG
    assert down(wts=a + 2) == _native.NMQ_ERR_ARG
    assert down(work=a + 16) == _native.NMQ_ERR_ARG      # rows too long for one launch: a workspace, 256-aligned
    assert down(work_bytes=16) == _native.NMQ_ERR_SHAPE  # too small
    assert down(n_in=5000) == _native.NMQ_ERR_SHAPE      # not whole blocks


def test_moe_layer_checks_without_launching(L):
    """nmq_moe_layer sizes its workspace and refuses bad arguments before anything is launched."""
    from ggufengine_amd import _native
    need = ctypes.c_int64(0)
    assert L.nmq_moe_layer_work_bytes(1, 8, 2048, 768, ctypes.byref(need)) == 0
    n = 8 * 768
    assert need.value >= 2 * n + 2 * (n // 32 * 4) + 2 * n * 4            # activation, fp32 gate|up
    assert L.nmq_moe_layer_work_bytes(0, 8, 2048, 768, ctypes.byref(need)) == _native.NMQ_ERR_ARG
    buf = ctypes.create_string_buffer(1 << 16)
    a = (ctypes.addressof(buf) + 255) // 256 * 256
    args = dict(fg=12, wg=a, wu=a, per=768 * 8 * 144, fd=14, wd=a, perd=2048 * 3 * 210, ids=a, wts=a, L=1, k=8, x=a,
                mode=_native.X_F32_BF16, out=a, E=2048, FF=768, work=a, work_bytes=1 << 30)

    def call(**kw):
        v = {**args, **kw}
        return L.nmq_moe_layer(v["fg"], v["wg"], v["wu"], v["per"], v["fd"], v["wd"], v["perd"], v["ids"], v["wts"],
                               v["L"], v["k"], v["x"], v["mode"], v["out"], v["E"], v["FF"], v["work"],
                               v["work_bytes"], None)
    assert call(ids=None) == _native.NMQ_ERR_ARG
    assert call(wd=None) == _native.NMQ_ERR_ARG
    assert call(mode=_native.X_SILU_MUL_BF16) == _native.NMQ_ERR_ARG
    assert call(work=None) == _native.NMQ_ERR_ARG
    assert call(work=a + 64) == _native.NMQ_ERR_ARG                 # 256-byte aligned
    assert call(work_bytes=1024) == _native.NMQ_ERR_SHAPE           # too small
    assert call(FF=760, per=760 * 8 * 144) == _native.NMQ_ERR_SHAPE  # groups of 32 rows
    assert call(perd=100) == _native.NMQ_ERR_SHAPE                   # down experts overlap
    assert call(fd=13) == _native.NMQ_ERR_FORMAT
