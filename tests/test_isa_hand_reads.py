"""The one-token kernels with hand-issued reads (mv1_kernel<..., HR = 1 or 2>, mvt_kernel, mvp_kernel: Q4_K, TQ2_0,
IQ2_XXS; mvk_kernel, mvd_kernel) rely on the
compiler never touching a register whose read is still outstanding: the compiler does not see those
reads, so a copy of such a register (which it could place at a branch join or to split a live range)
would silently take a stale value.  This test compiles the sources to gfx950 assembly and checks,
for every such kernel, that between a hand-issued read and the wait that covers it no instruction
reads or writes the read's destination registers.  (CPU only: hipcc cross-compiles the three sources
in parallel.)"""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "nemicli-terminal_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HAND_KERNEL = re.compile(r"^(_ZN3nmq10mv1_kernel\w*Li[12]EEEvNS_8MvParamsE|_ZN3nmq10mvt_kernel\w*EEEvNS_8MvParamsE):", re.M)
# the dense gate|up kernel with the activation (fp32 input, 8 or 4 rows per wave and group)
PAIR_KERNEL = re.compile(r"^(_ZN3nmq10mvp_kernel\w*EEEvNS_8MvParamsENS_8QuantOutE):", re.M)


def _vregs(op):
    m = re.match(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def hazards(asm: str, name: str):
    """(kernel, instruction, load) for every access to a register of a hand-issued read before a wait
    covers it.  A hand wait vmcnt(N) (inside the inline-assembly markers) completes all but the last N
    hand-issued reads; the compiler's own vmcnt(0) completes all of them."""
    body = asm[asm.index(name + ":"):]
    body = body[:body.index("s_endpgm")]
    ins, hand = [], False
    for line in body.split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            hand = True
            continue
        if t.startswith(";;#ASMEND"):
            hand = False
            continue
        if not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        ins.append((hand, t))
    found, pend = [], []
    for hand, t in ins:
        op = t.split()[0]
        args = [a.strip() for a in t[len(op):].split(",")]
        if hand and op.startswith("global_load_lds"):
            pend.append((set(), t))   # counted by vmcnt, no register written
            continue
        if hand and op.startswith("global_load"):
            pend.append((_vregs(args[0]), t))
            continue
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", t)
            if m:
                n = int(m.group(1))
                if hand:
                    pend = pend[len(pend) - n:] if 0 < n < len(pend) else ([] if n == 0 else pend)
                elif n == 0:
                    pend = []
            continue
        if op.startswith("s_"):
            continue
        store = op.startswith(("global_store", "ds_write", "buffer_store"))
        srcs = set()
        for a in (args if store else args[1:]):
            if a:
                srcs |= _vregs(a.split()[0])
        dst = set() if store or not args else _vregs(args[0])
        for regs, load in pend:
            if (srcs | dst) & regs:
                found.append((name, t, load))
    return found


SOURCES = ("nmq_mv_q4_k.hip", "nmq_mv_tq2_0.hip", "nmq_mv_iq2_xxs.hip", "nmq_mv_q6_k.hip", "nmq_mv_q4_0.hip",
           "nmq_mv_q8_0.hip")
# the sources with the dense-read matrix-core kernel (all of them)
DMA_SOURCES = SOURCES
# the K-split long-row kernel with hand-issued reads (mvk_kernel<..., HR = true>): Q4_K, TQ2_0, Q6_K
KSPLIT_KERNEL = re.compile(r"^(_ZN3nmq10mvk_kernel\w*Lb1EEEvNS_8MvParamsE):", re.M)


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    out = tmp_path_factory.mktemp("isa")
    procs = {}
    for src in SOURCES:
        cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops", "-fno-fast-math", "--cuda-device-only", "-S", os.path.join(CSRC, src),
               "-o", str(out / (src + ".s"))]
        procs[src] = subprocess.Popen(cmd, cwd=CSRC, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    for src, pr in procs.items():
        assert pr.wait(timeout=900) == 0, src
    return {src: (out / (src + ".s")).read_text() for src in SOURCES}


@pytest.mark.parametrize("src", SOURCES[:3])
def test_hand_read_kernels_exist(asm, src):
    names = HAND_KERNEL.findall(asm[src])
    one = [n for n in names if "mv1_kernel" in n]
    two = [n for n in names if "mvt_kernel" in n]
    # one token: T = 16/32/64 x (one unit per lane with 3 or 4 step buffers, two units with 3) x (two-stage
    # plain, two-stage ext, fp32 values); 2..4 tokens (Q4_K): T = 16/32/64 x NC = 2, 3, 4
    assert len(one) == 27, one
    assert len(two) == (9 if "q4_k" in src else 0), two


@pytest.mark.parametrize("src", SOURCES)
def test_no_access_to_registers_of_outstanding_reads(asm, src):
    names = HAND_KERNEL.findall(asm[src]) + KSPLIT_KERNEL.findall(asm[src]) + PAIR_KERNEL.findall(asm[src])
    bad = [h for n in names for h in hazards(asm[src], n)]
    assert not bad, bad[:5]


@pytest.mark.parametrize("src", SOURCES[:3])
def test_pair_kernels_exist(asm, src):
    assert len(PAIR_KERNEL.findall(asm[src])) == 2, PAIR_KERNEL.findall(asm[src])


@pytest.mark.parametrize("src", ["nmq_mv_q4_k.hip", "nmq_mv_tq2_0.hip", "nmq_mv_q6_k.hip"])
def test_ksplit_hand_read_kernels_exist(asm, src):
    # KS = 2, 3, 4 slices x 3 or 4 row buffers, without segments (the segment variant keeps
    # compiler-scheduled reads)
    assert len(KSPLIT_KERNEL.findall(asm[src])) == 6, KSPLIT_KERNEL.findall(asm[src])


def test_checker_finds_a_planted_read(asm):
    """The check itself: a copy of a pending register placed right after a hand-issued read is found."""
    text = asm[SOURCES[0]]
    name = HAND_KERNEL.findall(text)[0]
    start = text.index(name + ":")
    m = re.compile(r"global_load_dwordx4 v\[(\d+):\d+\]").search(text, text.index(";;#ASMSTART", start))
    end = text.index(";;#ASMEND", m.end()) + len(";;#ASMEND")
    planted = text[:end] + f"\n\tv_mov_b32_e32 v250, v{m.group(1)}\n" + text[end:]
    assert hazards(planted, name)


DMA_KERNEL = re.compile(r"^(_ZN3nmq10mvd_kernel\w*EEEvNS_9MvmParamsE):", re.M)


def m0_outside_hand_code(asm: str, name: str):
    """Instructions outside the inline-assembly blocks that name M0: the dense-read kernel sets M0 for
    its hand-issued global_load_lds inside those blocks and relies on nothing else using it."""
    body = asm[asm.index(name + ":"):]
    body = body[:body.index("s_endpgm")]
    bad, hand = [], False
    for line in body.split("\n"):
        t = line.split(";")[0].strip() if not line.strip().startswith(";;#ASM") else line.strip()
        if t.startswith(";;#ASMSTART"):
            hand = True
        elif t.startswith(";;#ASMEND"):
            hand = False
        elif t and not hand and re.search(r"\bm0\b", t):
            bad.append(t)
    return bad


@pytest.mark.parametrize("src", DMA_SOURCES)
def test_dense_read_kernels_touch_no_outstanding_register(asm, src):
    """mvd_kernel reads (xd, xs) by hand (global_load_dwordx4) with its chunk reads (global_load_lds, no
    destination register) in flight: no instruction may touch those registers before the wait."""
    names = DMA_KERNEL.findall(asm[src])
    assert names
    bad = [h for n in names for h in hazards(asm[src], n)]
    assert not bad, bad[:5]


@pytest.mark.parametrize("src", DMA_SOURCES)
def test_dense_read_kernels_keep_m0_to_themselves(asm, src):
    names = DMA_KERNEL.findall(asm[src])
    assert len(names) == 4, names   # 1 or 2 chunks per slice, with and without K ranges
    bad = [(n, t) for n in names for t in m0_outside_hand_code(asm[src], n)]
    assert not bad, bad[:5]
    # and every hand block that writes M0 issues its LDS load right after
    text = asm[src]
    for n in names:
        body = text[text.index(n + ":"):]
        body = body[:body.index("s_endpgm")]
        for blk in re.findall(r";;#ASMSTART(.*?);;#ASMEND", body, re.S):
            ops = [l.strip() for l in blk.split("\n") if l.strip()]
            if any("m0" in o for o in ops):
                assert len(ops) == 2 and ops[0].startswith("s_mov_b32 m0") and \
                    ops[1].startswith("global_load_lds_dwordx4"), ops


@pytest.mark.parametrize("src", SOURCES)
def test_hand_read_kernels_use_no_scratch(asm, src):
    """Kernels with hand-issued reads keep everything in registers: a value the compiler parks in scratch
    memory comes back through reads and waits of its own among the hand-issued ones."""
    text = asm[src]
    names = HAND_KERNEL.findall(text) + KSPLIT_KERNEL.findall(text) + DMA_KERNEL.findall(text) + PAIR_KERNEL.findall(text)
    bad = []
    for n in names:
        body = text[text.index(n + ":"):]
        body = body[:body.index("s_endpgm")]
        if re.search(r"\bscratch_", body):
            bad.append(n)
    assert not bad, bad
