#!/usr/bin/env python3
"""Benchmark of the GGUF quantized mat-vec path on one MI355X.

Headline (one JSON line on stdout): Q4_K 14336x4096 mat-vec at batch 1 (the gate/up projection of a
Llama-3-8B decoder layer) -- GB/s of algorithmic bytes, % of the 8 TB/s HBM peak, us per mat-vec --
plus us per Llama-3-8B layer (7 mat-vecs + 4 activation quantisations).

A "step" is one launch of the mat-vec kernel over one token whose two-stage int8 input (Eingang) is
already resident in HBM.  The weight matrix of each step is one of several identical copies whose
total exceeds twice the 256 MB last-level cache, so every step streams its weights from HBM.
Timing: HIP events on the launch stream around K back-to-back launches (after W warm-up launches).

Weights: ~N(0, 0.02) fp32 (numpy PCG64, fixed seeds) quantised by this library's encoders;
x ~N(0, 1).  The CPU baseline (reported, not the target) times the oracle's restatement of the
reference's CPU path on this host: the matrix dequantised once, then an fp32 GEMV per call.
"""
import argparse
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
BLOCK = {"Q8_0": (32, 34), "Q4_K": (256, 144), "Q6_K": (256, 210), "TQ2_0": (256, 66), "IQ2_XXS": (256, 66)}
TYPE = {"Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ2_XXS": 16, "TQ2_0": 35}
# Llama-3-8B decoder layer (Q4_K_M mix): name, format, rows, n_in, weight seed, input
LAYER = [("q", "Q4_K", 4096, 4096, 21, "x_attn"), ("k", "Q4_K", 1024, 4096, 22, "x_attn"),
         ("v", "Q4_K", 1024, 4096, 23, "x_attn"), ("o", "Q4_K", 4096, 4096, 24, "attn_out"),
         ("gate", "Q4_K", 14336, 4096, 25, "x_ffn"), ("up", "Q4_K", 14336, 4096, 26, "x_ffn"),
         ("down", "Q6_K", 4096, 14336, 27, "act")]
INPUTS = {"x_attn": (4096, 28), "attn_out": (4096, 30), "x_ffn": (4096, 31), "act": (14336, 29)}


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


def cpu_baseline(raw, fmt, rows, n_in, x, budget_s):
    """The oracle's restatement of the reference CPU path (models/common.py:190, 526-527): dequantise
    once, then fp32 GEMV per call, timed for about budget_s seconds."""
    import oracle
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
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
                      f"{calls} calls ({el:.1f} s, {per * 1e6:.0f} us/call) on {threads} threads of {cpu}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-layer", action="store_true", help="skip the per-layer timing")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the mat-vec path is single-GPU "
                                   "(multi-GPU sharding by output rows is described in DESIGN.md, not built)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

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

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        launch(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    ab = alg_bytes(fmt, rows, n_in)
    gbs = ab / (ms * 1e-3) / 1e9

    # parity of the timed kernel's output against the oracle (cheap, full size)
    import oracle
    ref = oracle.mv_deq(fmt, raw, rows, n_in, x.cpu().numpy()[None])
    parity = float(oracle.rel_err_rows(y.cpu().numpy()[None], ref).max())

    cfg = {"workload": "Q4_K 14336x4096 mat-vec, batch 1 (Llama-3-8B ffn gate/up)", "format": fmt, "rows": rows,
           "n_in": n_in, "batch": 1, "weight_copies": copies, "algorithmic_bytes": ab,
           "us_per_matvec": round(ms * 1e3, 3), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
           "max_rel_err_vs_oracle": parity}

    # ---- one Llama-3-8B layer: 4 activation quantisations + 7 mat-vecs ----
    if not args.no_layer:
        mats = {}
        for name, f, r, k, s, _ in LAYER:
            mats[name] = torch.from_numpy(make_weights(f, r, k, s) if name != "gate" else raw).to(dev)
        layer_bytes = sum(weight_bytes(f, r, k) for _, f, r, k, _, _ in LAYER)
        nl = max(2, -(-2 * LLC_BYTES // layer_bytes))
        layers = [mats] + [{k: v.clone() for k, v in mats.items()} for _ in range(nl - 1)]
        xin = {n: torch.from_numpy(np.random.Generator(np.random.PCG64(sd)).standard_normal(k, dtype=np.float32)).to(dev)
               for n, (k, sd) in INPUTS.items()}
        eg = {n: mmvq.Eingang(n=k, device=dev) for n, (k, _) in INPUTS.items()}
        ys = {name: torch.empty(r, dtype=torch.float32, device=dev) for name, _, r, _, _, _ in LAYER}

        def one_layer(li):
            lw = layers[li % nl]
            order = [("x_attn", ("q", "k", "v")), ("attn_out", ("o",)), ("x_ffn", ("gate", "up")), ("act", ("down",))]
            for inp, names in order:
                ei = eg[inp]
                rc = L.nmq_quant_q8(xin[inp].data_ptr(), 1, ei.xq.data_ptr(), ei.xq2.data_ptr(), ei.xd.data_ptr(),
                                    ei.xs.data_ptr(), ei.n, stream)
                if rc:
                    _native.check(rc)
                for name in names:
                    _, f, r, k, _, _ = next(t for t in LAYER if t[0] == name)
                    rc = L.nmq_mv(TYPE[f], lw[name].data_ptr(), ei.xq.data_ptr(), ei.xq2.data_ptr(), ei.xd.data_ptr(),
                                  ei.xs.data_ptr(), ys[name].data_ptr(), r, k, 1, stream)
                    if rc:
                        _native.check(rc)

        reps = max(20, args.steps // 10)
        for i in range(max(5, args.warmup // 10)):
            one_layer(i)
        torch.cuda.synchronize()
        t0.record()
        for i in range(reps):
            one_layer(i)
        t1.record()
        torch.cuda.synchronize()
        us_layer = t0.elapsed_time(t1) / reps * 1e3
        cfg["us_per_layer"] = round(us_layer, 3)
        cfg["layer_weight_bytes"] = layer_bytes
        cfg["layer_pct_hbm_peak"] = round(100 * layer_bytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)
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
            for i in range(20):
                one(i)
            torch.cuda.synchronize()
            t0.record()
            for i in range(reps):
                one(i)
            t1.record()
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) / reps * 1e3
            parts[name] = {"format": f, "shape": [r, k], "us": round(us, 3),
                           "pct_hbm_peak": round(100 * alg_bytes(f, r, k) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)}
            del cps
        xq_in = xin["x_attn"]
        for i in range(20):
            L.nmq_quant_q8(xq_in.data_ptr(), 1, eg["x_attn"].xq.data_ptr(), eg["x_attn"].xq2.data_ptr(),
                           eg["x_attn"].xd.data_ptr(), eg["x_attn"].xs.data_ptr(), 4096, stream)
        torch.cuda.synchronize()
        t0.record()
        for i in range(reps):
            L.nmq_quant_q8(xq_in.data_ptr(), 1, eg["x_attn"].xq.data_ptr(), eg["x_attn"].xq2.data_ptr(),
                           eg["x_attn"].xd.data_ptr(), eg["x_attn"].xs.data_ptr(), 4096, stream)
        t1.record()
        torch.cuda.synchronize()
        parts["quant_q8_4096"] = {"us": round(t0.elapsed_time(t1) / reps * 1e3, 3)}
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
