#!/usr/bin/env python3
"""Benchmark of the GGUF quantized mat-vec path on one MI355X.

Headline (one JSON line on stdout): Q4_K 14336x4096 mat-vec at batch 1 (the gate/up projection of a
Llama-3-8B decoder layer) -- GB/s of algorithmic bytes, % of the 8 TB/s HBM peak, us per mat-vec --
plus us per Llama-3-8B layer: the 7 mat-vecs in 4 launches (q, k, v in one nmq_mv_x launch and o in
another, each quantising its fp32 4096-value input itself; gate and up in one nmq_mv_gate_up_act launch
that also forms the activation silu(gate) * up and quantises it as the down input; down), checked
against the oracle.  Beside it: the layer with the down input given and quantised by its own launch
(us_per_layer_values, 5 launches), with 4 quantisation launches and nmq_mv_multi (us_per_layer_multi),
and with one launch per matrix (us_per_layer_separate); the layer and the layer with its inputs formed
(us_per_layer_fused_inputs) also as HIP graphs of 1 and 32 layers, replayed (us_per_layer_graph*).

A "step" is one launch of the mat-vec kernel over one token whose two-stage int8 input (Eingang) is
already resident in HBM.  The weight matrix of each step is one of several identical copies whose
total exceeds twice the 256 MB last-level cache, so every step streams its weights from HBM.
Timing: HIP events on the launch stream around K back-to-back launches (after W warm-up launches).

Weights: ~N(0, 0.02) fp32 (numpy PCG64, fixed seeds) quantised by this library's encoders;
x ~N(0, 1).  The CPU baseline (reported, not the target) times the oracle's restatement of the
reference's CPU path on this host: the matrix dequantised once, then an fp32 GEMV per call.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "nemicli-terminal_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "Q4_K matvec GB/s (% of HBM peak) + µs/layer, Llama-3-8B shapes, batch 1"
HBM_PEAK_GBS = 8000.0
LLC_BYTES = 256 << 20
BLOCK = {"Q4_0": (32, 18), "Q8_0": (32, 34), "Q4_K": (256, 144), "Q6_K": (256, 210), "TQ2_0": (256, 66), "IQ2_XXS": (256, 66)}
TYPE = {"Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ2_XXS": 16, "TQ2_0": 35}
# Llama-3-8B decoder layer (Q4_K_M mix): name, format, rows, n_in, weight seed, input
LAYER = [("q", "Q4_K", 4096, 4096, 21, "x_attn"), ("k", "Q4_K", 1024, 4096, 22, "x_attn"),
         ("v", "Q4_K", 1024, 4096, 23, "x_attn"), ("o", "Q4_K", 4096, 4096, 24, "attn_out"),
         ("gate", "Q4_K", 14336, 4096, 25, "x_ffn"), ("up", "Q4_K", 14336, 4096, 26, "x_ffn"),
         ("down", "Q6_K", 4096, 14336, 27, "act")]
INPUTS = {"x_attn": (4096, 28), "attn_out": (4096, 30), "x_ffn": (4096, 31), "act": (14336, 29)}
# longest input a layer launch takes as fp32 values (measured: staging 14336 fp32 values in the long-row
# kernel costs more than a separate quantisation launch)
VALUES_MAX_N_IN = 8192


def weight_bytes(fmt, rows, n_in):
    bv, bb = BLOCK[fmt]
    return rows * (n_in // bv) * bb


def alg_bytes(fmt, rows, n_in, n=1):
    """Weights + two-stage int8 input (xq, xq2: 2 B/value; xd, xs: 8 B per 32) + fp32 output."""
    return weight_bytes(fmt, rows, n_in) + n * (2 * n_in + 8 * n_in // 32) + n * 4 * rows


def make_weights(fmt, rows, n_in, seed):
    import numpy as np
    from ggufengine_amd import encode
    w = np.random.Generator(np.random.PCG64(seed)).standard_normal(rows * n_in, dtype=np.float32)
    w *= np.float32(0.02)
    return encode.encode(fmt, w, threads=min(16, len(os.sched_getaffinity(0))))


def traffic_bytes():
    """HBM bytes per launch of the headline kernel, from the committed FETCH_SIZE / WRITE_SIZE counter
    runs (profiles/q4k_14336x4096_batch1_traffic.md), or None when they are absent."""
    path = os.path.join(ROOT, "profiles", "q4k_14336x4096_batch1_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def host_threads():
    """(threads, reason): every host core this process may use -- its CPU affinity, capped by
    OMP_NUM_THREADS where the machine sets one (the share of the host that belongs to one GPU)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and 0 < int(cap) < n:
        return int(cap), f"all {cap} host threads of this GPU's share (OMP_NUM_THREADS; affinity {n})"
    return n, f"all {n} host threads in the process's affinity"


def cpu_baseline(raw, fmt, rows, n_in, x, budget_s):
    """The oracle's restatement of the reference CPU path (models/common.py:190, 526-527): dequantise
    once, then fp32 GEMV per call, timed for about budget_s seconds."""
    import oracle
    threads, why = host_threads()
    w = oracle.dequant(fmt, raw).reshape(rows, n_in)
    oracle.gemv_f32(w, x, threads)  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.gemv_f32(w, x, threads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s or calls >= 100000:
            break
    per = el / calls
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(alg_bytes(fmt, rows, n_in) / per / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{fmt} {rows}x{n_in} dequantised once by the oracle, fp32 GEMV (F.linear path) timed over "
                      f"{calls} calls ({el:.1f} s, {per * 1e6:.0f} us/call) on {threads} threads of {cpu}: {why}"}


# ---- the other configurations: one JSON record per case on stdout ---------------------------------

_CLOCKS_PER_US = None


def _hold_gpu(us):
    """Keep the current stream busy for about `us` microseconds (torch.cuda._sleep: a one-wave kernel
    counting shader clocks, bounded), so launches queued meanwhile by the host run back to back on the
    GPU instead of at the host's launch rate."""
    import torch
    global _CLOCKS_PER_US
    if _CLOCKS_PER_US is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        a.record()
        torch.cuda._sleep(2_000_000)
        b.record()
        torch.cuda.synchronize()
        _CLOCKS_PER_US = 2_000_000 / max(1.0, a.elapsed_time(b) * 1e3)
    torch.cuda._sleep(int(us * _CLOCKS_PER_US))


def _timed(fn, steps, warmup, pairs=False, chunk=200):
    """fn(i) queues step i on the current stream.  W untimed steps, then `steps` timed ones in chunks of at
    most `chunk`; before each chunk the GPU is held (spin kernel) longer than the host takes to queue it, so
    the chunk runs back to back on the GPU.  Returns the us per step between events around each chunk
    (back to back: the launch gaps between kernels included, the host's launch rate not) and, with
    pairs=True, from a second timed pass with events recorded around every step, their mean (the step's
    own duration on the stream, as a kernel trace sees it)."""
    import time
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    probe = min(steps, 20)
    t = time.perf_counter()
    for i in range(probe):
        fn(i)
    host_us = (time.perf_counter() - t) / probe * 1e6
    torch.cuda.synchronize()

    def timed_pass(with_pairs):
        total_ms, pair_ms, done = 0.0, [], 0
        while done < steps:
            n = min(chunk, steps - done)
            _hold_gpu(3 * host_us * n + 300)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(n if with_pairs else 0)]
            a.record()
            for j in range(n):
                if with_pairs:
                    ev[j][0].record()
                fn(done + j)
                if with_pairs:
                    ev[j][1].record()
            b.record()
            torch.cuda.synchronize()
            total_ms += a.elapsed_time(b)
            pair_ms += [e0.elapsed_time(e1) for e0, e1 in ev]
            done += n
        return total_ms / steps * 1e3, (sum(pair_ms) / len(pair_ms) * 1e3 if pair_ms else None)

    out = {"us_back_to_back": timed_pass(False)[0], "host_us_per_step": host_us}
    if pairs:
        out["us_event_pairs"] = timed_pass(True)[1]
    return out


def _events_us(fn, steps, warmup):
    """us per call of fn(i) (launches on the current stream), run back to back on the GPU (see _timed)."""
    return _timed(fn, steps, warmup)["us_back_to_back"]


def _copies(t, total_bytes=None):
    """t and clones of it, together more than twice the last-level cache."""
    n = max(2, -(-2 * LLC_BYTES // (total_bytes or t.numel() * t.element_size())))
    return [t] + [t.clone() for _ in range(n - 1)]


def _record(config, case, fmt, us, ab, err, **extra):
    gbs = ab / (us * 1e-6) / 1e9
    rec = {"config": config, "case": case, "format": fmt, "us": round(us, 3), "algorithmic_bytes": ab,
           "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
    if err is not None:
        rec["max_rel_err_vs_oracle"] = err
    rec.update(extra)
    print(json.dumps(rec), flush=True)


def _mv_case(L, stream, fmt, ws, raw_np, rows, n_in, x_np, steps, warmup, knobs=None):
    """Time nmq_mv on n = x_np.shape[0] tokens rotating over the weight copies ws; parity of the last
    output against the oracle.  knobs: launch-plan overrides (nmq_set_tuning) for this case only."""
    import torch
    import oracle
    from ggufengine_amd import _native, mmvq
    with _native.tuning(**(knobs or {})):
        dev = ws[0].device
        n = x_np.shape[0]
        e = mmvq.Eingang(torch.from_numpy(x_np).to(dev))
        y = torch.empty(n, rows, dtype=torch.float32, device=dev)
        ep = [e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr()]

        def go(i):
            rc = L.nmq_mv(TYPE[fmt], ws[i % len(ws)].data_ptr(), *ep, y.data_ptr(), rows, n_in, n, stream)
            if rc:
                _native.check(rc)
        us = _events_us(go, steps, warmup)
        err = float(oracle.rel_err_rows(y.cpu().numpy(), oracle.mv_deq(fmt, raw_np, rows, n_in, x_np)).max())
        return us, err


def _x(seed, shape):
    import numpy as np
    return np.random.Generator(np.random.PCG64(seed)).standard_normal(shape, dtype=np.float32)


def run_configs(which, steps, warmup):
    import numpy as np
    import torch
    from ggufengine_amd import _native, encode
    if not _native.available("cuda"):
        raise SystemExit("libnmq.so not loaded or device is not gfx950")
    L = _native.lib()
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream().cuda_stream
    threads = min(16, len(os.sched_getaffinity(0)))

    if which in ("q8_0", "all"):
        # Q8_0 4096x4096, W ~N(0,0.02) (seed 11), x ~N(0,1) (seed 12), batch 1
        raw = make_weights("Q8_0", 4096, 4096, 11)
        ws = _copies(torch.from_numpy(raw).cuda())
        us, err = _mv_case(L, stream, "Q8_0", ws, raw, 4096, 4096, _x(12, (1, 4096)), steps, warmup)
        del ws
        _record("q8_0", "Q8_0 4096x4096 batch 1", "Q8_0", us, alg_bytes("Q8_0", 4096, 4096), err)

    if which in ("speculative", "all"):
        # speculative verification: Q4_K 14336x4096 (seed 31) and 4096x4096 (seed 32), n in 1,2,4,8 (seed 33)
        for rows, seed in ((14336, 31), (4096, 32)):
            raw = make_weights("Q4_K", rows, 4096, seed)
            ws = _copies(torch.from_numpy(raw).cuda())
            X = _x(33, (8, 4096))
            for n in (1, 2, 4, 8):
                us, err = _mv_case(L, stream, "Q4_K", ws, raw, rows, 4096, X[:n], steps, warmup)
                extra = {}
                if n > 1:
                    us4, _ = _mv_case(L, stream, "Q4_K", ws, raw, rows, 4096, X[:n], steps, warmup,
                                      {"MVM": 0, "MVT_MAX": 1, "MVD": 0})
                    usm, _ = _mv_case(L, stream, "Q4_K", ws, raw, rows, 4096, X[:n], steps, warmup,
                                      {"MVM": 2, "MVT_MAX": 1, "MVD": 0})
                    usd, _ = _mv_case(L, stream, "Q4_K", ws, raw, rows, 4096, X[:n], steps, warmup,
                                      {"MVD_MIN": 2, "MVT_MAX": 1})
                    extra = {"us_dot4_kernel": round(us4, 3), "us_matrix_core_kernel": round(usm, 3),
                             "us_dense_matrix_core_kernel": round(usd, 3)}
                _record("speculative", f"Q4_K {rows}x4096 n={n}", "Q4_K", us, alg_bytes("Q4_K", rows, 4096, n), err,
                        **extra)
            del ws
        # the layer's down projection under the same verification: Q6_K 4096x14336 (seed 27), n in 1..4
        # (the few-token long-row kernel) and 8 (the dense-read kernel over K ranges)
        raw = make_weights("Q6_K", 4096, 14336, 27)
        ws = _copies(torch.from_numpy(raw).cuda())
        X = _x(29, (8, 14336))
        for n in (1, 2, 3, 4, 8):
            us, err = _mv_case(L, stream, "Q6_K", ws, raw, 4096, 14336, X[:n], steps, warmup)
            extra = {}
            if 1 < n <= 4:
                usg, _ = _mv_case(L, stream, "Q6_K", ws, raw, 4096, 14336, X[:n], steps, warmup, {"MVLT_MAX": 1})
                extra = {"us_without_few_token_kernel": round(usg, 3)}
            elif n > 4:
                usg, _ = _mv_case(L, stream, "Q6_K", ws, raw, 4096, 14336, X[:n], steps, warmup, {"MVD_LONG": 0})
                extra = {"us_without_dense_kernel": round(usg, 3)}
            _record("speculative", f"Q6_K 4096x14336 n={n}", "Q6_K", us, alg_bytes("Q6_K", 4096, 14336, n), err, **extra)
        del ws

    if which in ("q4_0", "all"):
        # Q4_0 (no workload of its own among the headline configurations): W ~N(0,0.02) (seed 61),
        # 4096x4096 and 14336x4096, x ~N(0,1) (seed 62), n in 1, 2, 4, 8 with both small-batch kernels
        for rows in (4096, 14336):
            raw = make_weights("Q4_0", rows, 4096, 61)
            ws = _copies(torch.from_numpy(raw).cuda())
            X = _x(62, (8, 4096))
            for n in (1, 2, 4, 8):
                us, err = _mv_case(L, stream, "Q4_0", ws, raw, rows, 4096, X[:n], steps, warmup)
                extra = {}
                if n > 1:
                    us4, _ = _mv_case(L, stream, "Q4_0", ws, raw, rows, 4096, X[:n], steps, warmup,
                                      {"MVM": 0, "MVD": 0})
                    usm, _ = _mv_case(L, stream, "Q4_0", ws, raw, rows, 4096, X[:n], steps, warmup,
                                      {"MVM": 2, "MVD": 0})
                    extra = {"us_dot4_kernel": round(us4, 3), "us_matrix_core_kernel": round(usm, 3)}
                _record("q4_0", f"Q4_0 {rows}x4096 n={n}", "Q4_0", us, alg_bytes("Q4_0", rows, 4096, n), err, **extra)
            del ws

    if which in ("fewtoken", "all"):
        # 2..16 tokens of the other formats (speculative verification, small batches) on the dense-read
        # matrix-core kernel: 14336x4096 and 4096x4096, W ~N(0,0.02) (seed 81), x ~N(0,1) (seed 82); beside
        # each, the launch plan without that kernel (the other matrix-core kernel or dot4); then every
        # format on rows of 14336 values (4096x14336, the down projection's shape: K ranges)
        for rows, n_in, fmts in ((14336, 4096, ("Q4_0", "Q8_0", "Q6_K", "TQ2_0", "IQ2_XXS")),
                                 (4096, 4096, ("Q4_0", "Q8_0", "Q6_K", "TQ2_0", "IQ2_XXS")),
                                 (4096, 14336, ("Q4_K", "Q6_K", "Q4_0", "Q8_0", "TQ2_0", "IQ2_XXS"))):
            for fmt in fmts:
                raw = make_weights(fmt, rows, n_in, 81)
                ws = _copies(torch.from_numpy(raw).cuda())
                X = _x(82, (16, n_in))
                for n in (2, 4, 8, 16):
                    us, err = _mv_case(L, stream, fmt, ws, raw, rows, n_in, X[:n], steps, warmup)
                    uso, _ = _mv_case(L, stream, fmt, ws, raw, rows, n_in, X[:n], steps, warmup, {"MVD": 0})
                    _record("fewtoken", f"{fmt} {rows}x{n_in} n={n}", fmt, us, alg_bytes(fmt, rows, n_in, n), err,
                            us_without_dense_kernel=round(uso, 3))
                del ws

    if which in ("lowbit", "all"):
        # TQ2_0: codes i.i.d. P(0)=0.4, P(+-1)=0.3, d = fp16(|N(0,0.02)|) (seed 51); IQ2_XXS from N(0,0.02)
        # (seed 52); x seed 53
        for rows in (4096, 12288):
            g = np.random.Generator(np.random.PCG64(51))
            nb = rows * 4096 // 256
            codes = g.choice(np.array([0, 1, 2], dtype=np.uint8), size=(nb, 256), p=[0.3, 0.4, 0.3])
            d16 = np.abs(g.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
            raws = {"TQ2_0": encode.pack_ternary(codes, d16), "IQ2_XXS": make_weights("IQ2_XXS", rows, 4096, 52)}
            for fmt, raw in raws.items():
                ws = _copies(torch.from_numpy(raw).cuda())
                us, err = _mv_case(L, stream, fmt, ws, raw, rows, 4096, _x(53, (1, 4096)), steps, warmup)
                _record("lowbit", f"{fmt} {rows}x4096 batch 1", fmt, us, alg_bytes(fmt, rows, 4096), err)
                del ws

    if which in ("prefill", "all"):
        run_prefill(L, stream, steps, warmup)

    if which in ("offload",):
        run_offload(steps, warmup, len(os.sched_getaffinity(0)))

    if which in ("moe", "all"):
        run_moe(steps, warmup, threads)

    if which in ("ceiling", "all"):
        run_ceiling(steps, warmup)


CEILING_SHAPES = [(wpc, wgw, u) for wpc in (4, 8, 16, 32) for wgw in (4, 8, 16) for u in (2, 4, 8)
                  if wpc % wgw == 0]


def read_ceiling(n_bytes, steps, warmup, shapes=None):
    """The pure streaming read (nmq_stream_read) of n_bytes in one launch, rotating over copies larger than
    twice the last-level cache, for each launch shape (resident waves per CU, waves per workgroup, loads in
    flight per thread); us per launch back to back (see _timed).  Returns the best shape's
    record and all timings."""
    import torch
    from ggufengine_amd import _native
    L = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream
    n_copies = max(2, -(-2 * LLC_BYTES // n_bytes))
    bufs = [torch.randint(0, 255, (n_bytes,), dtype=torch.uint8, device="cuda") for _ in range(n_copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    table = []
    for wpc, wgw, u in shapes or CEILING_SHAPES:
        def go(i, wpc=wpc, wgw=wgw, u=u):
            rc = L.nmq_stream_read(bufs[i % n_copies].data_ptr(), n_bytes, sink.data_ptr(), wpc, wgw, u, stream)
            if rc:
                _native.check(rc)
        table.append({"waves_per_cu": wpc, "wg_waves": wgw, "unroll": u, "us": round(_events_us(go, steps, warmup), 3)})
    del bufs
    best = min(table, key=lambda r: r["us"])
    gbs = n_bytes / (best["us"] * 1e-6) / 1e9
    return {"bytes": n_bytes, **best, "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}, table


def run_ceiling(steps, warmup):
    """Pure-read reference points: the headline's weight bytes (33 MB) and sizes up to 1 GB, every launch
    shape; one record per size."""
    sizes = (weight_bytes("TQ2_0", 4096, 4096), weight_bytes("Q4_K", 4096, 4096), weight_bytes("TQ2_0", 12288, 4096),
             weight_bytes("Q4_K", 14336, 4096), weight_bytes("Q6_K", 4096, 14336), 128 << 20, 512 << 20, 1 << 30)
    for n in sizes:
        best, table = read_ceiling(n, steps, warmup)
        print(json.dumps({"config": "ceiling", "case": f"pure read of {n} bytes in one launch", "best": best,
                          "shapes": table}), flush=True)


def run_prefill(L, stream, steps, warmup):
    """Several tokens per call (the reference's mmvq.mm range, 17..112, and 16): the fp16 matrix-core
    path (nmq_mm_input + nmq_mm) against the int8 mat-vec path (nmq_mv in launches of 16) on the Llama
    matrices, W ~N(0,0.02) (seeds 31, 32, 27), x ~N(0,1) (seed 34).  `us` is nmq_mm alone,
    `us_with_input` adds the input launch; algorithmic bytes as for nmq_mv (weights once, fp32 x read
    once, y written)."""
    import torch
    import oracle
    from ggufengine_amd import _native
    for fmt, rows, n_in, seed in (("Q4_K", 14336, 4096, 31), ("Q4_K", 4096, 4096, 32), ("Q6_K", 4096, 14336, 27)):
        raw = make_weights(fmt, rows, n_in, seed)
        ws = _copies(torch.from_numpy(raw).cuda())
        X = _x(34, (112, n_in))
        for n in (16, 64, 112):
            xd = torch.from_numpy(X[:n]).cuda()
            pad = (n + 15) // 16 * 16
            xh = torch.empty(pad, n_in, dtype=torch.float16, device="cuda")
            xl = torch.empty_like(xh)
            xsum = torch.empty(pad, n_in // 32, dtype=torch.float32, device="cuda")
            xs = torch.empty(n, dtype=torch.float32, device="cuda")
            y = torch.empty(n, rows, dtype=torch.float32, device="cuda")

            def prep(i):
                _native.check(L.nmq_mm_input(xd.data_ptr(), 1, xh.data_ptr(), xl.data_ptr(), xsum.data_ptr(),
                                             xs.data_ptr(), n_in, n, stream))

            def go(i):
                _native.check(L.nmq_mm(TYPE[fmt], ws[i % len(ws)].data_ptr(), xh.data_ptr(), xl.data_ptr(),
                                       xsum.data_ptr(), xs.data_ptr(), y.data_ptr(), rows, n_in, n, stream))
            prep(0)
            us = _events_us(go, steps, warmup)
            us_in = _events_us(prep, steps, warmup)
            go(0)
            torch.cuda.synchronize()
            err = float(oracle.rel_err_rows(y.cpu().numpy(), oracle.mv_deq(fmt, raw, rows, n_in, X[:n])).max())
            us_int8, _ = _mv_case(L, stream, fmt, ws, raw, rows, n_in, X[:n], steps, warmup)
            ab = weight_bytes(fmt, rows, n_in) + n * (4 * n_in + 4 * rows)
            _record("prefill", f"{fmt} {rows}x{n_in} n={n}", fmt, us, ab, err, us_with_input=round(us + us_in, 3),
                    us_int8_path=round(us_int8, 3), tokens_per_s=round(n / ((us + us_in) * 1e-6)))
        del ws


def run_offload(steps, warmup, threads):
    """Weights in pinned RAM.  (a) The expert layer of run_moe at one token with all experts in RAM
    (hostmem, read over PCIe through the address tables) against the same experts in VRAM, eager calls.
    The VRAM figures read the same 8 experts (2.6 MB) on every call, so they are cache-warm; the RAM
    figure crosses PCIe on every call (host memory is not cached by the GPU).
    (b) A pass over 8 Q4_K 4096x4096 layers (9.4 MB each, the same generator) streamed through a
    Fliessband (4 VRAM slots, whole copies a few layers ahead) against the same layers in VRAM; the
    copy rate is the weight bytes of the pass over its time.  Every result is checked equal to the
    VRAM one bit for bit before timing.  The RAM paths get at least half a second of warm-up: PCIe
    reads and copies of fresh pinned blocks run about a fifth slower during their first ~0.5 s."""
    import numpy as np
    import torch
    from ggufengine_amd import band, encode, experts, hostmem, packed
    dev = torch.device("cuda", 0)
    n_exp, k, E, FF = 128, 8, 2048, 768
    g = np.random.Generator(np.random.PCG64(41))

    def enc(fmt, rows, n_in, n=n_exp):
        w = g.standard_normal(n * rows * n_in, dtype=np.float32) * np.float32(0.02)
        return encode.encode(fmt, w, threads=threads)

    def pinned(raw):
        h = hostmem.empty(raw.size, dev)
        h.numpy()[:] = raw
        return h

    def timed(fn, reps, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps * 1e3

    raw = {"gate": enc("Q4_K", FF, E), "up": enc("Q4_K", FF, E), "down": enc("Q6_K", E, FF)}
    shapes = {"gate": (12, FF, E), "up": (12, FF, E), "down": (14, E, FF)}
    hosts = {n: pinned(r) for n, r in raw.items()}
    names = ("gate", "up", "down")
    ram_parts = [experts.PackedExperts(hostmem.abbilden(hosts[n], dev), shapes[n][0], n_exp, *shapes[n][1:])
                 for n in names]
    in_ram = experts.Experten(*ram_parts)
    in_vram = experts.Experten(*[experts.PackedExperts(torch.from_numpy(raw[n]).to(dev), shapes[n][0], n_exp,
                                                       *shapes[n][1:]) for n in names])
    logits = torch.from_numpy(_x(42, (1, n_exp))).to(dev)
    x = torch.from_numpy(_x(43, (1, E))).to(dev)
    idx, w = experts.auswahl(logits, k)
    assert torch.equal(in_ram(x, idx, w), in_vram(x, idx, w))
    us_ram = timed(lambda: in_ram(x, idx, w), steps, max(warmup, 1000))
    us_vram = timed(lambda: in_vram(x, idx, w), steps, warmup)
    # the routed experts moved into VRAM slots (ExpertenLager, 8 slots per part): kernels read the slots
    lager = experts.ExpertenLager(ram_parts, plaetze=k, device=dev)
    lager.zaehlen(idx)
    lager.umsortieren()
    assert torch.equal(in_ram(x, idx, w), in_vram(x, idx, w))
    us_slots = timed(lambda: in_ram(x, idx, w), steps, warmup)
    moved = k * sum(r.size for r in raw.values()) // n_exp
    _record("offload", "128 experts top-8, 1 token, experts in pinned RAM", "Q4_K+Q6_K", us_ram, moved, None,
            us_experts_in_vram=round(us_vram, 3), us_routed_experts_in_vram_slots=round(us_slots, 3),
            pcie_GBs=round(moved / (us_ram * 1e-6) / 1e9, 1), equal_to_vram=True, timing="eager calls (all three)")
    del in_ram, in_vram, ram_parts, lager, hosts

    n_lay, rows, n_in = 8, 4096, 4096
    raws = [enc("Q4_K", rows, n_in, 1) for _ in range(n_lay)]
    fl = band.Fliessband(dev)
    ram_l, vram_l, keep = [], [], []
    for r in raws:
        h = pinned(r)
        keep.append(h)
        lay = packed.PackedLinear(hostmem.abbilden(h, dev), 12, rows, n_in, dtype=torch.float32)
        lay.band, lay.nr = fl, fl.anmelden(h)
        ram_l.append(lay)
        vram_l.append(packed.PackedLinear(torch.from_numpy(r).to(dev), 12, rows, n_in, dtype=torch.float32))
    xs = torch.from_numpy(_x(62, (1, n_in))).to(dev)
    for a, b in zip(ram_l, vram_l):
        assert torch.equal(a(xs), b(xs))
    us_band = timed(lambda: [lay(xs) for lay in ram_l], max(20, steps // 10), max(warmup, 300))
    us_vram = timed(lambda: [lay(xs) for lay in vram_l], max(20, steps // 10), warmup)
    moved = sum(r.size for r in raws)
    _record("offload", "8 Q4_K 4096x4096 layers through the band (pinned RAM -> 4 VRAM slots)", "Q4_K", us_band,
            moved, None, us_layers_in_vram=round(us_vram, 3), copy_GBs=round(moved / (us_band * 1e-6) / 1e9, 1),
            equal_to_vram=True, timing="eager calls (both)")
    hostmem.flush()


def run_moe(steps, warmup, threads):
    """Qwen3-30B-A3B-style expert layer: 128 experts, gate/up 768x2048 Q4_K, down 2048x768 Q6_K
    (seed 41) in 4 copies, 16 routings (router logits ~N(0,1), seeds 42, 44, ..., 72 -> top-8 softmax
    renormalised), x ~N(0,1) (seed 43), 1 and 4 tokens.  Timed: the whole expert layer after routing
    (2 activation quantisations, 3 gathered mat-vec launches, silu * up, weighted combine), 16 layers
    in a row (routing q on copy (j + q) % 4, as a decode step holds one such layer per block) captured
    in one HIP graph per j and replayed, us per layer: the experts a cycle reads (about 1 GB) exceed
    the last-level cache.  One layer per graph and the eager Python-driven time beside it.  Checked:
    every replayed output equals the eager layer; routing 0 on copy 0 against the oracle chain."""
    import numpy as np
    import torch
    import oracle
    from ggufengine_amd import encode, experts
    n_exp, k, E, FF = 128, 8, 2048, 768
    g = np.random.Generator(np.random.PCG64(41))

    def enc(fmt, rows, n_in):
        w = g.standard_normal(n_exp * rows * n_in, dtype=np.float32) * np.float32(0.02)
        return encode.encode(fmt, w, threads=threads)
    raw = {"gate": enc("Q4_K", FF, E), "up": enc("Q4_K", FF, E), "down": enc("Q6_K", E, FF)}
    dev = torch.device("cuda", 0)
    per_set = sum(r.size for r in raw.values())
    NSETS, PER = 4, 16
    base = {n: torch.from_numpy(r).to(dev) for n, r in raw.items()}
    sets = [base] + [{n: t.clone() for n, t in base.items()} for _ in range(NSETS - 1)]
    layers = [experts.Experten(experts.PackedExperts(s["gate"], 12, n_exp, FF, E),
                               experts.PackedExperts(s["up"], 12, n_exp, FF, E),
                               experts.PackedExperts(s["down"], 14, n_exp, E, FF)) for s in sets]
    per_expert = per_set // n_exp
    for Ltok in (1, 4):
        # one routing per layer of a PER-layer step (logits seeds 42, 44, ...): layer q of a step uses
        # routing q on expert set (j + q) % NSETS, so the experts read by consecutive steps (about 1 GB
        # over all sets and routings) do not stay in the 256 MB last-level cache
        routes = [experts.auswahl(torch.from_numpy(_x(42 + 2 * q, (Ltok, n_exp))).to(dev), k) for q in range(PER)]
        idx, w = routes[0]
        x = torch.from_numpy(_x(43, (Ltok, E))).to(dev)
        touched = {((j + q) % NSETS, e) for j in range(NSETS) for q in range(PER)
                   for e in routes[q][0].cpu().numpy().reshape(-1).tolist()}
        eager = {}
        for j in range(NSETS):
            for q in range(PER):
                if (j, q) not in eager:
                    eager[(j, q)] = layers[j](x, *routes[q]).clone()
        out = {}

        def go(i):
            out["y"] = layers[(i // PER + i) % NSETS](x, *routes[i % PER])
        us_eager = _events_us(go, max(50, steps // 10), max(10, warmup // 10))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for j in range(NSETS):
                layers[j](x, idx, w)
        torch.cuda.current_stream().wait_stream(side)
        # one layer per graph (graph g: routing g, set g % NSETS) ...
        graphs, outs = [], []
        for q in range(PER):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                outs.append(layers[q % NSETS](x, *routes[q]))
            graphs.append(gr)
        us_one = _events_us(lambda i: graphs[i % PER].replay(), steps, warmup)
        torch.cuda.synchronize()
        for q in range(PER):
            graphs[q].replay()
            torch.cuda.synchronize()
            if not torch.equal(outs[q], eager[(q % NSETS, q)]):
                raise SystemExit(f"moe: graph replay of routing {q} differs from the eager layer")
        # ... and a whole decode step's worth, PER layers per graph, so the graph launch's own cost
        # (~8 us on this stack) is spread as in a real step; every replayed output equals the eager one
        mgraphs, mouts = [], []
        for j in range(NSETS):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                mouts.append([layers[(j + q) % NSETS](x, *routes[q]) for q in range(PER)])
            mgraphs.append(gr)
        us = _events_us(lambda i: mgraphs[i % NSETS].replay(), max(20, steps // PER), max(5, warmup // PER)) / PER
        torch.cuda.synchronize()
        for j in range(NSETS):
            mgraphs[j].replay()
            torch.cuda.synchronize()
            if not all(torch.equal(mouts[j][q], eager[((j + q) % NSETS, q)]) for q in range(PER)):
                raise SystemExit(f"moe: {PER}-layer graph replay of set {j} differs from the eager layer")
        out["y"] = eager[(0, 0)]
        distinct = sum(len(set(r[0].cpu().numpy().reshape(-1).tolist())) for r in routes) / PER
        ab = int(distinct * per_expert) + Ltok * 4 * E * 2
        # end to end against the oracle chain on the selected experts (dequantised weights, fp64)
        ids = idx.cpu().numpy()
        wts = w.cpu().numpy().astype(np.float64)
        xb = oracle.round_bf16(x.cpu().numpy())
        ref = np.zeros((Ltok, E))

        def part(name, e):
            r = raw[name]
            return r[e * (r.size // n_exp):(e + 1) * (r.size // n_exp)]
        for t in range(Ltok):
            for j in range(k):
                e = int(ids[t, j])
                gg = oracle.mv_deq("Q4_K", part("gate", e), FF, E, xb[t:t + 1])[0]
                uu = oracle.mv_deq("Q4_K", part("up", e), FF, E, xb[t:t + 1])[0]
                a = oracle.round_bf16((gg / (1.0 + np.exp(-gg)) * uu).astype(np.float32)[None])
                ref[t] += wts[t, j] * oracle.mv_deq("Q6_K", part("down", e), E, FF, a)[0]
        err = float(oracle.rel_err_rows(out["y"].cpu().numpy(), ref).max())
        _record("moe", f"128 experts top-8, {Ltok} token(s)", "Q4_K+Q6_K", us, ab, err,
                distinct_experts_per_layer=distinct, expert_sets=NSETS, routings=PER,
                bytes_touched_per_cycle=len(touched) * per_expert, us_eager_python=round(us_eager, 3),
                us_graph_of_one_layer=round(us_one, 3),
                timing=f"graph replay, {PER} expert layers per graph, us per layer")
        del graphs, outs, mgraphs, mouts, eager


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-layer", action="store_true", help="skip the per-layer timing")
    ap.add_argument("--config", default="headline",
                    choices=("headline", "q8_0", "speculative", "q4_0", "fewtoken", "lowbit", "prefill", "moe", "offload", "ceiling",
                             "all"),
                    help="headline (default): the metric line; the others print one record per case of "
                         "the other workloads (Q8_0 batch 1, speculative verify n=1..8, Q4_0, TQ2_0/IQ2_XXS, "
                         "16..112 tokens on the fp16 matrix cores, MoE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the mat-vec path is single-GPU "
                                   "(sharding by output rows over several GPUs is not built)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.config != "headline":
        run_configs(args.config, min(args.steps, 500), min(args.warmup, 50))
        return

    import numpy as np
    import torch
    from ggufengine_amd import _native, mmvq

    if not _native.available("cuda"):
        raise SystemExit("libnmq.so not loaded or device is not gfx950")
    L = _native.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream().cuda_stream

    # ---- headline: Q4_K 14336 x 4096, batch 1 ----
    fmt, rows, n_in, seed = "Q4_K", 14336, 4096, 25
    raw = make_weights(fmt, rows, n_in, seed)
    wb = raw.size
    copies = max(2, -(-2 * LLC_BYTES // wb))
    base = torch.from_numpy(raw).to(dev)
    ws = [base] + [base.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(np.random.Generator(np.random.PCG64(28)).standard_normal(n_in, dtype=np.float32)).to(dev)
    e = mmvq.Eingang(x)
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    eptr = [e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr()]
    wptr = [w.data_ptr() for w in ws]

    def launch(i):
        rc = L.nmq_mv(TYPE[fmt], wptr[i % copies], *eptr, y.data_ptr(), rows, n_in, 1, stream)
        if rc:
            _native.check(rc)

    timing = _timed(launch, args.steps, args.warmup, pairs=True)
    ms = timing["us_back_to_back"] * 1e-3
    ab = alg_bytes(fmt, rows, n_in)
    gbs = ab / (ms * 1e-3) / 1e9
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    # reference point on the same box: the runtime's device copy of the same weight bytes, one launch
    # per copy, source and destination rotating over copies larger than the last-level cache (it reads
    # and writes every byte: its rate counts both)
    dsts = [torch.empty_like(base) for _ in range(copies)]
    copy_us = _events_us(lambda i: dsts[i % copies].copy_(ws[(i + 1) % copies]), 200, 20)
    del dsts
    # reference point: the pure streaming read of the same weight bytes in one launch (best launch shape
    # of a small sweep; `--config ceiling` sweeps more shapes and sizes)
    ceiling, _ = read_ceiling(wb, 200, 20, [(wpc, wgw, 4) for wpc, wgw in ((8, 8), (16, 8), (16, 16), (32, 16))])

    # parity of the timed kernel's output against the oracle (cheap, full size)
    import oracle
    ref = oracle.mv_deq(fmt, raw, rows, n_in, x.cpu().numpy()[None])
    parity = float(oracle.rel_err_rows(y.cpu().numpy()[None], ref).max())

    cfg = {"workload": "Q4_K 14336x4096 mat-vec, batch 1 (Llama-3-8B ffn gate/up)", "format": fmt, "rows": rows,
           "n_in": n_in, "batch": 1, "weight_copies": copies, "algorithmic_bytes": ab,
           "us_per_matvec": round(ms * 1e3, 3), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
           "timing": "HIP events around the K launches, queued while a spin kernel holds the GPU so that "
                     "they run back to back (launch gaps included, the host's launch rate not)",
           "us_per_matvec_event_pairs": round(timing["us_event_pairs"], 3),
           "host_us_per_launch": round(timing["host_us_per_step"], 3),
           "max_rel_err_vs_oracle": parity,
           "pure_read_same_bytes": ceiling,
           "device_copy_same_bytes": {"us": round(copy_us, 3), "bytes_read_and_written": 2 * wb,
                                      "GB/s": round(2 * wb / (copy_us * 1e-6) / 1e9, 1)}}

    # ---- one Llama-3-8B layer: 4 activation quantisations + 7 mat-vecs ----
    if not args.no_layer:
        mats, raws_np = {}, {}
        for name, f, r, k, s, _ in LAYER:
            raws_np[name] = make_weights(f, r, k, s) if name != "gate" else raw
            mats[name] = torch.from_numpy(raws_np[name]).to(dev)
        layer_bytes = sum(weight_bytes(f, r, k) for _, f, r, k, _, _ in LAYER)
        nl = max(2, -(-2 * LLC_BYTES // layer_bytes))
        layers = [mats] + [{k: v.clone() for k, v in mats.items()} for _ in range(nl - 1)]
        xin = {n: torch.from_numpy(np.random.Generator(np.random.PCG64(sd)).standard_normal(k, dtype=np.float32)).to(dev)
               for n, (k, sd) in INPUTS.items()}
        eg = {n: mmvq.Eingang(n=k, device=dev) for n, (k, _) in INPUTS.items()}
        ys = {name: torch.empty(r, dtype=torch.float32, device=dev) for name, _, r, _, _, _ in LAYER}

        order = [("x_attn", ("q", "k", "v")), ("attn_out", ("o",)), ("x_ffn", ("gate", "up")), ("act", ("down",))]
        spec = {t[0]: t for t in LAYER}

        def mats_of(lw, names):
            """(format, n_in, weight pointers, rows, output pointers) of matrices sharing one input."""
            f, k = spec[names[0]][1], spec[names[0]][3]
            return (f, k, [lw[n].data_ptr() for n in names], [spec[n][2] for n in names],
                    [ys[n].data_ptr() for n in names])

        def one_layer(li, how, st=stream):
            """The 7 mat-vecs and their 4 inputs.  how = "separate": each input quantised by nmq_quant_q8,
            one nmq_mv launch per matrix; "multi": the matrices of one input (q, k, v and gate, up) in
            one nmq_mv_multi launch; "values": the launches on 4096-value inputs take the fp32 input
            directly (nmq_mv_x: each launch quantises it itself), the down projection (14336 values,
            where staging fp32 values costs more than a quantisation launch) as in "multi"; "act": as
            "values", but the down input is the layer's own activation silu(gate) * up, formed and
            quantised by the gate|up launch (nmq_mv_gate_up_act) -- 4 launches."""
            lw = layers[li % nl]
            for inp, names in order:
                f, k, wp, rows_, yp = mats_of(lw, names)
                m = len(names)
                if how == "act" and inp == "x_ffn":
                    ea = eg["act"]
                    _native.check(L.nmq_mv_gate_up_act(TYPE[f], wp[0], wp[1], xin[inp].data_ptr(), _native.X_F32,
                                                       _native.ACT_SILU, ea.xq.data_ptr(), ea.xq2.data_ptr(),
                                                       ea.xd.data_ptr(), ea.xs.data_ptr(), rows_[0], k, st))
                    continue
                if how == "act" and inp == "act":
                    ea = eg["act"]
                    _native.check(L.nmq_mv(TYPE[f], wp[0], ea.xq.data_ptr(), ea.xq2.data_ptr(), ea.xd.data_ptr(),
                                           ea.xs.data_ptr(), yp[0], rows_[0], k, 1, st))
                    continue
                if how in ("values", "act") and k <= VALUES_MAX_N_IN:
                    _native.check(L.nmq_mv_x(TYPE[f], m, (ctypes.c_void_p * m)(*wp), (ctypes.c_int * m)(*rows_),
                                             (ctypes.c_void_p * m)(*yp), xin[inp].data_ptr(), _native.X_F32, None,
                                             k, st))
                    continue
                ei = eg[inp]
                ep = (ei.xq.data_ptr(), ei.xq2.data_ptr(), ei.xd.data_ptr(), ei.xs.data_ptr())
                _native.check(L.nmq_quant_q8(xin[inp].data_ptr(), 1, *ep, ei.n, st))
                if how != "separate" and m > 1:
                    _native.check(L.nmq_mv_multi(TYPE[f], m, (ctypes.c_void_p * m)(*wp), (ctypes.c_int * m)(*rows_),
                                                 (ctypes.c_void_p * m)(*yp), *ep, k, st))
                else:
                    for w_, r_, y_ in zip(wp, rows_, yp):
                        _native.check(L.nmq_mv(TYPE[f], w_, *ep, y_, r_, k, 1, st))

        reps = max(20, args.steps // 10)
        for how in ("separate", "multi", "values", "act"):
            us_layer = _events_us(lambda i: one_layer(i, how), reps, max(5, args.warmup // 10))
            if how != "act":
                cfg[f"us_per_layer_{how}"] = round(us_layer, 3)
        cfg["us_per_layer"] = round(us_layer, 3)

        def graph_us(fn, per=1):
            """fn(li, stream) for `per` consecutive layers captured as one HIP graph, one graph per weight
            copy, the graphs replayed in turn: the one-token step as the reference runs it (captured,
            replayed).  The first replay is checked against the eager outputs.  us per layer."""
            graphs = []
            for j in range(nl):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for q in range(per):
                        fn(j + q, torch.cuda.current_stream().cuda_stream)
                graphs.append(gr)
            fn(per - 1, stream)
            torch.cuda.synchronize()
            eager = {n: y.clone() for n, y in ys.items()}
            graphs[0].replay()
            torch.cuda.synchronize()
            assert all(torch.equal(eager[n], ys[n]) for n in ys), "graph replay differs from the eager layer"
            n_rep = max(5, reps // per)
            us = _events_us(lambda i: graphs[i % nl].replay(), n_rep, max(5, args.warmup // 10))
            return round(us / per, 3)

        cfg["us_per_layer_graph"] = graph_us(lambda j, st: one_layer(j, "act", st))
        cfg["us_per_layer_graph_32_layers"] = graph_us(lambda j, st: one_layer(j, "act", st), 32)
        cfg["layer_weight_bytes"] = layer_bytes
        cfg["layer_pct_hbm_peak"] = round(100 * layer_bytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)
        # the layer's outputs against the oracle (the weight copies are identical), max relative error per
        # output row-vector: every matrix of the "values" form on its given input, then the down
        # projection of the "act" form on the oracle's silu(gate) * up
        one_layer(0, "values")
        torch.cuda.synchronize()
        errs, ref = [], {}
        for inp, names in order:
            xv = xin[inp].cpu().numpy()[None]
            for n in names:
                f, r, k = spec[n][1], spec[n][2], spec[n][3]
                ref[n] = oracle.mv_deq(f, raws_np[n], r, k, xv)
                errs.append(float(oracle.rel_err_rows(ys[n].cpu().numpy()[None], ref[n]).max()))
        one_layer(0, "act")
        torch.cuda.synchronize()
        act_o = oracle.akt(ref["gate"][0], ref["up"][0]).astype(np.float32)[None]
        f, r, k = spec["down"][1], spec["down"][2], spec["down"][3]
        errs.append(float(oracle.rel_err_rows(ys["down"].cpu().numpy()[None],
                                              oracle.mv_deq(f, raws_np["down"], r, k, act_o)).max()))
        cfg["layer_max_rel_err_vs_oracle"] = max(errs)

        # The same layer with its inputs formed as the reference's one-token step forms them
        # (models/baukasten.py:217-241 without rope and attention): RMS norm fused with the q/k/v input,
        # the attention output quantised, residual add + RMS norm fused with the gate/up input, the gate|up
        # launch forming silu(gate) * up and the down input (nmq_mv_gate_up_act, akt_q8's arithmetic).
        E, FF = 4096, 14336
        rng_s = np.random.Generator(np.random.PCG64(34))
        h_s = torch.from_numpy(rng_s.standard_normal(E, dtype=np.float32)).to(dev)
        nw_s = torch.from_numpy((1 + 0.1 * rng_s.standard_normal(E)).astype(np.float32)).to(dev)
        xn_s = torch.empty(E, dtype=torch.float32, device=dev)
        hn_s = torch.empty(E, dtype=torch.float32, device=dev)
        a_s = torch.empty(FF, dtype=torch.float32, device=dev)

        def ptrs(e):
            return e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr()

        def mv_named(lw, name, ei, st):
            _, f, r, k, _, _ = next(t for t in LAYER if t[0] == name)
            _native.check(L.nmq_mv(TYPE[f], lw[name].data_ptr(), *ptrs(ei), ys[name].data_ptr(), r, k, 1, st))

        def mv_shared(lw, names, ei, st):
            f, k, wp, rows_, yp = mats_of(lw, names)
            m = len(names)
            _native.check(L.nmq_mv_multi(TYPE[f], m, (ctypes.c_void_p * m)(*wp), (ctypes.c_int * m)(*rows_),
                                         (ctypes.c_void_p * m)(*yp), *ptrs(ei), k, st))

        def step_layer(li, st=stream):
            lw = layers[li % nl]
            _native.check(L.nmq_norm_q8(h_s.data_ptr(), None, 1.0, None, nw_s.data_ptr(), 1e-5, xn_s.data_ptr(),
                                        *ptrs(eg["x_attn"]), E, st))
            mv_shared(lw, ("q", "k", "v"), eg["x_attn"], st)
            _native.check(L.nmq_quant_q8(xin["attn_out"].data_ptr(), 1, *ptrs(eg["attn_out"]), E, st))
            mv_named(lw, "o", eg["attn_out"], st)
            _native.check(L.nmq_norm_q8(h_s.data_ptr(), ys["o"].data_ptr(), 1.0, hn_s.data_ptr(), nw_s.data_ptr(),
                                        1e-5, xn_s.data_ptr(), *ptrs(eg["x_ffn"]), E, st))
            _native.check(L.nmq_mv_gate_up_act(TYPE["Q4_K"], lw["gate"].data_ptr(), lw["up"].data_ptr(),
                                               xn_s.data_ptr(), _native.X_F32, _native.ACT_SILU,
                                               *ptrs(eg["act"]), FF, E, st))
            mv_named(lw, "down", eg["act"], st)

        cfg["us_per_layer_fused_inputs"] = round(_events_us(step_layer, reps, max(5, args.warmup // 10)), 3)
        cfg["us_per_layer_fused_inputs_graph"] = graph_us(step_layer)
        cfg["us_per_layer_fused_inputs_graph_32_layers"] = graph_us(step_layer, 32)
        del layers
        # per-matrix breakdown: each mat-vec timed alone, rotating over its own copies (> 2x the LLC)
        parts = {}
        for name, f, r, k, _, inp in LAYER:
            ei = eg[inp]
            nc_ = max(2, -(-2 * LLC_BYTES // mats[name].numel()))
            cps = [mats[name]] + [mats[name].clone() for _ in range(nc_ - 1)]

            def one(i, f=f, r=r, k=k, ei=ei, cps=cps, name=name):
                rc = L.nmq_mv(TYPE[f], cps[i % len(cps)].data_ptr(), ei.xq.data_ptr(), ei.xq2.data_ptr(),
                              ei.xd.data_ptr(), ei.xs.data_ptr(), ys[name].data_ptr(), r, k, 1, stream)
                if rc:
                    _native.check(rc)
            us = _events_us(one, reps, 20)
            parts[name] = {"format": f, "shape": [r, k], "us": round(us, 3),
                           "pct_hbm_peak": round(100 * alg_bytes(f, r, k) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)}
            del cps
        xq_in = xin["x_attn"]
        small = {"quant_q8_4096": lambda: L.nmq_quant_q8(xq_in.data_ptr(), 1, *ptrs(eg["x_attn"]), 4096, stream)}
        small.update({
            "norm_q8_4096": lambda: L.nmq_norm_q8(h_s.data_ptr(), ys["o"].data_ptr(), 1.0, hn_s.data_ptr(),
                                                  nw_s.data_ptr(), 1e-5, xn_s.data_ptr(), *ptrs(eg["x_ffn"]), E,
                                                  stream),
            "akt_q8_14336": lambda: L.nmq_akt_q8(ys["gate"].data_ptr(), ys["up"].data_ptr(), 0, a_s.data_ptr(),
                                                 *ptrs(eg["act"]), FF, stream)})
        for pname, fn in small.items():
            _native.check(fn())
            parts[pname] = {"us": round(_events_us(lambda i, fn=fn: fn(), reps, 20), 3)}
        cfg["layer_parts"] = parts
        del mats

    out = {"metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8", "data": "synthetic", "config": cfg,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_bytes()}}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(raw, fmt, rows, n_in, x.cpu().numpy(), args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
