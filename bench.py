#!/usr/bin/env python3
"""Decode-attention bench on one MI355X (gfx950).

Workload (default, BASELINE config 4 -- the north-star case): Gemma-4-31B global-layer
decode step, B=1, Hq=32, Hkv=4 (GQA 8), head_dim 512, attention_k_eq_v (one K=V
buffer), 131072 visible rows (rows 0..131070 cached + the new token appended at
131071), scale 1/sqrt(512).  One step = esda_decode: fused append + split-K attention
+ merge, with every input already resident in HBM.

Printed: ONE JSON line.  value = algorithmic HBM bytes per step / step time (GB/s);
algorithmic bytes = visible rows x row bytes (K only under k_eq_v) + q read + out
write + new-row read and write.  `roofline` prices the dominant kernel (the split-K
attend kernel, timed alone with HIP events on the launch stream); `cpu_baseline` times
the CPU oracle's reference-rounding restatement on the same inputs.

  python bench.py [--steps K] [--warmup W] [--workload c4|c2|c1|c3|c4raw|c4q8|c5|p512g|p4kg|p512gs|p4kgs|p512l|p4kl] [--no-cpu]

Workload c5 is the full Gemma-4-31B-shaped attention step: 60 layers (every 6th
global: D=512, Hkv=4, k_eq_v, linear caches; the rest local: D=256, Hkv=16, window
1024 over a 1024-row ring), B=32, lengths ~ U[1024, 32768]; each layer appends and
attends in order (one esda_decode per layer, 120 kernels per step, replayed from a HIP
graph).  It reports total attention us per token step.

Workloads p512g / p4kg / p512l / p4kl are the prefill side (esda_prefill): a 512-token
chunk over a 16384-token global cache (the reference's own prefill decomposition shape:
d512, nKV 4, groups 8, seqQ 512 at 16K, WIDE_HEAD_ATTENTION.md), a fresh 4096-token
global prefill, a 512-token chunk of a local layer (D=256, Hkv=16, window 1024 over
window + chunk keys) and a fresh 4096-token local prefill (window 1024); p512gs / p4kgs are
the two global shapes over one K = V buffer (attention_k_eq_v).  They report TFLOP/s of
algorithmic attention FLOPs (4 * D per visible (query head, key) pair) against the bf16 MFMA
peak.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def _die_multi_gpu(n: int) -> None:
    print(json.dumps({"error": f"--gpus {n}: this build measures one GPU only; the decode "
                      "path shards by sequence / kv head with no exchange"}))
    sys.exit(2)


WORKLOADS = {
    # name: (B, Hq, Hkv, D, cap, window, ring, shared, pos_fn, scale)
    "c1": dict(B=1, Hq=16, Hkv=8, D=256, cap=1024, window=1024, ring=False, shared=False,
               pos=lambda rng, B: [1023], scale=1 / 16),
    "c2": dict(B=1, Hq=32, Hkv=4, D=512, cap=8448, window=0, ring=False, shared=True,
               pos=lambda rng, B: [8192], scale=512 ** -0.5),
    "c3": dict(B=8, Hq=32, Hkv=16, D=256, cap=1024, window=1024, ring=True, shared=False,
               pos=lambda rng, B: [int(x) for x in rng.integers(2048, 32769, size=B)], scale=1 / 16),
    # C4 plants 64 keys per kv head whose logit rises by +4.0 (plant_peaked_keys)
    "c4": dict(B=1, Hq=32, Hkv=4, D=512, cap=131072, window=0, ring=False, shared=True,
               pos=lambda rng, B: [131071], scale=512 ** -0.5, peaks=64, bump=4.0),
    # C4's shape in raw-K mode (the reference's esDecodeAttnGlobal path): the cache holds
    # pre-norm k_proj rows; K and V are rebuilt in the kernel; in-model scale 1.0.
    # The same over a q8 raw stream (rawKVQ8: u8 rows + per-row scale / bias, 520 B a row).
    "c4q8": dict(B=1, Hq=32, Hkv=4, D=512, cap=131072, window=0, ring=False, shared=True, raw=True, q8=True,
                 pos=lambda rng, B: [131071], scale=1.0),
    "c4raw": dict(B=1, Hq=32, Hkv=4, D=512, cap=131072, window=0, ring=False, shared=True, raw=True,
                  pos=lambda rng, B: [131071], scale=1.0),
}

PREFILL_WORKLOADS = {
    "p512g": dict(Hq=32, Hkv=4, D=512, Sq=512, Sk=16384, q_pos0=15872, k_pos0=0, window=0, scale=512 ** -0.5,
                  name="global-layer prefill chunk: 512 queries over 16384 keys (causal), D=512, GQA 32/4"),
    "p4kg": dict(Hq=32, Hkv=4, D=512, Sq=4096, Sk=4096, q_pos0=0, k_pos0=0, window=0, scale=512 ** -0.5,
                 name="global-layer fresh prefill: 4096 tokens (causal), D=512, GQA 32/4"),
    # the same two over one K = V buffer (attention_k_eq_v, the global layers' layout): the
    # kernel streams the buffer once and reads V^T from the K stage
    "p512gs": dict(Hq=32, Hkv=4, D=512, Sq=512, Sk=16384, q_pos0=15872, k_pos0=0, window=0, scale=512 ** -0.5,
                   shared=True, name="global-layer prefill chunk, k_eq_v (V = K): 512 queries over 16384 keys "
                                     "(causal), D=512, GQA 32/4"),
    "p4kgs": dict(Hq=32, Hkv=4, D=512, Sq=4096, Sk=4096, q_pos0=0, k_pos0=0, window=0, scale=512 ** -0.5,
                  shared=True, name="global-layer fresh prefill, k_eq_v (V = K): 4096 tokens (causal), D=512, "
                                    "GQA 32/4"),
    "p4kl": dict(Hq=32, Hkv=16, D=256, Sq=4096, Sk=4096, q_pos0=0, k_pos0=0, window=1024, scale=1 / 16,
                 name="local-layer fresh prefill: 4096 tokens, window 1024, D=256, GQA 32/16"),
    "p512l": dict(Hq=32, Hkv=16, D=256, Sq=512, Sk=1536, q_pos0=15872, k_pos0=15872 + 512 - 1536, window=1024,
                  scale=1 / 16, name="local-layer prefill chunk: 512 queries over window + chunk = 1536 keys, "
                                     "window 1024, D=256, GQA 32/16"),
}

# C5 layer types (ESModelConfig.mm:82-86: every 6th layer is global, the last one too).
C5_LAYERS = 60
C5_B = 32
C5_LOCAL = dict(Hq=32, Hkv=16, D=256, cap=1024, window=1024, ring=True, shared=False, scale=1 / 16)
C5_GLOBAL = dict(Hq=32, Hkv=4, D=512, window=0, ring=False, shared=True, scale=512 ** -0.5)


WARM_SECONDS = 1.0


def warm_up(fn, steps: int, seconds: float = WARM_SECONDS) -> int:
    """Runs the W untimed warm-up steps, continued until the GPU has been stepping for
    `seconds`.  Under sustained load the MI355X settles its clocks over a few hundred
    milliseconds; C4 steps timed right after 20 warm-up steps read ~10% slower than the
    same steps a second later.  A freshly captured HIP graph likewise replays ~6% slower
    over its first ~50 ms.  Returns the number of warm-up calls run."""
    import torch

    t0, n = time.perf_counter(), 0
    while n < steps or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()  # keeps wall time in step with GPU time
    torch.cuda.synchronize()
    return n


def plant_peaked_keys(w, q, k_cache, pos, rng) -> None:
    """BASELINE config 4's peaked softmax mass: at w["peaks"] cached positions per sequence,
    add bump * q_hat to every kv head's key, q_hat the unit direction of that kv head's
    first query head, in fp32 before rounding to bf16 -- with scale * |q| = 1 that head's
    logit rises by exactly `bump` (the rule the parity tests use)."""
    import torch

    G = w["Hq"] // w["Hkv"]
    for b in range(w["B"]):
        picks = torch.tensor(sorted(int(x) for x in rng.choice(pos[b], size=w["peaks"], replace=False)),
                             device=k_cache.device)
        for h in range(w["Hkv"]):
            qh = q[b, h * G].float()
            alpha = w["bump"] / (w["scale"] * qh.norm())
            rows = k_cache[b, h, picks].float() + alpha * qh / qh.norm()
            k_cache[b, h, picks] = rows.to(torch.bfloat16)


def c5_is_global(layer: int) -> bool:
    return layer % 6 == 5 or layer == C5_LAYERS - 1


def visible_rows(w, pos):
    out = []
    for p in pos:
        lo = max(0, p - w["window"] + 1) if w["window"] else 0
        out.append(p - lo + 1)
    return out


Q8_ROW_BYTES = 512 + 8  # u8 row + f32 scale and bias


def algorithmic_bytes(w, pos) -> int:
    row = Q8_ROW_BYTES if w.get("q8") else w["D"] * 2 * (1 if w["shared"] else 2)
    kv = sum(visible_rows(w, pos)) * w["Hkv"] * row
    q_o = 2 * w["B"] * w["Hq"] * w["D"] * 2
    # new-row read + cache write (q8: the bf16 row read, its quantized row written)
    append = w["B"] * w["Hkv"] * ((w["D"] * 2 + row) if w.get("q8") else 2 * row)
    return kv + q_o + append


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c4", choices=sorted(WORKLOADS) + ["c5"] + sorted(PREFILL_WORKLOADS))
    ap.add_argument("--split-rows", type=int, default=0)
    ap.add_argument("--local-split-rows", type=int, default=0, help="c5: split rows of local layers")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache timing (small configs)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU baseline threads (0: OMP_NUM_THREADS, the host's CPU share, else every cpu)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="time a plain device copy of MIB MiB instead (HBM counter calibration)")
    ap.add_argument("--calibrate-read", type=int, default=0, metavar="MIB",
                    help="read MIB MiB through the attend kernel's load path instead (esda_stream_read): "
                         "the measured read ceiling and the counter calibration for that path")
    ap.add_argument("--read-workgroups", type=int, default=0,
                    help="calibrate-read: workgroups per launch (0: sweep 256 .. 2048)")
    ap.add_argument("--calibrate-lds", action="store_true",
                    help="measure the LDS read rate of the prefill kernel's operand reads instead "
                         "(esda_lds_read: 128-bit row reads and 64-bit transpose reads, 4 / 8 / 16 waves per CU)")
    args = ap.parse_args()
    if args.cpu_threads <= 0:
        args.cpu_threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or os.cpu_count() or 1
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        _die_multi_gpu(max(args.gpus, int(os.environ.get("WORLD_SIZE", "1"))))

    import numpy as np
    import torch

    from apertura_amd.decode import (DecodeCall, DecodeStep, RawCall, RawQ8Call, RawStep, STAGE_ATTEND,
                                     new_raw_workspace, new_workspace, q8_step_for, quantize_raw_rows,
                                     rope_table)

    if args.calibrate_copy:
        return calibrate_copy(args)
    if args.calibrate_read:
        return calibrate_read(args)
    if args.calibrate_lds:
        return calibrate_lds(args)
    if args.workload == "c5":
        return bench_c5(args)
    if args.workload in PREFILL_WORKLOADS:
        return bench_prefill(args)
    w = WORKLOADS[args.workload]
    rng = np.random.default_rng(1234)
    pos = w["pos"](rng, w["B"])
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def rms_bf16(shape):
        x = torch.randn(shape, device=dev, dtype=torch.float32, generator=gen)
        x = x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6)
        return x.to(torch.bfloat16)

    B, Hq, Hkv, D, cap = w["B"], w["Hq"], w["Hkv"], w["D"], w["cap"]
    q = rms_bf16((B, Hq, D))
    k_cache = rms_bf16((B, Hkv, cap, D))
    v_cache = k_cache if w["shared"] else rms_bf16((B, Hkv, cap, D))
    k_new = rms_bf16((B, Hkv, D))
    v_new = None if w["shared"] else rms_bf16((B, Hkv, D))
    pos_d = torch.tensor(pos, dtype=torch.int32, device=dev)
    if w.get("peaks"):
        plant_peaked_keys(w, q, k_cache, pos, np.random.default_rng(4321))
    out = torch.empty_like(q)
    stream = torch.cuda.Stream()  # default priority (side stream for graph capture)
    raw = None
    if w.get("raw"):
        # raw k_proj rows (not normalised), a k-norm weight and Gemma-4's global rotary table
        k_cache.mul_(2.0)
        k_new.mul_(2.0)
        kw = (1.0 + 0.25 * torch.randn(D, device=dev, generator=gen)).to(torch.bfloat16)
        inv_freq = torch.zeros(D // 2, dtype=torch.float32, device=dev)
        inv_freq[:64] = 1.0 / (1.0e6 ** (torch.arange(64, dtype=torch.float64, device=dev) * 2 / D)).float()
        # the per-model rotary table (esda_rope_table), built once like the weights
        tab = rope_table(inv_freq, cap)
        if w.get("q8"):
            # the same raw rows quantized into a q8 stream on the GPU (esda_quantize_raw_rows)
            q8 = torch.empty((B, Hkv, cap, D), dtype=torch.uint8, device=dev)
            sc = torch.empty((B, Hkv, cap), dtype=torch.float32, device=dev)
            bs = torch.empty_like(sc)
            for b in range(B):
                quantize_raw_rows(k_cache[b], q8[b], sc[b], bs[b])
            step = q8_step_for(q8, Hq, eps=1e-6, scale=w["scale"], split_rows=args.split_rows)
            ws = new_raw_workspace(step, dev)
            call = RawQ8Call(step, q, k_new, q8, sc, bs, pos_d, kw, inv_freq, out=out, workspace=ws, rope_table=tab)
            raw = (kw, inv_freq, q8, sc, bs)
        else:
            step = RawStep.for_cache(k_cache, Hq, eps=1e-6, scale=w["scale"], split_rows=args.split_rows)
            ws = new_raw_workspace(step, dev)
            call = RawCall(step, q, k_new, k_cache, pos_d, kw, inv_freq, out=out, workspace=ws, rope_table=tab)
            raw = (kw, inv_freq)
    else:
        step = DecodeStep.for_cache(k_cache, Hq, window=w["window"], ring=w["ring"],
                                    kv_shared=w["shared"], scale=w["scale"], split_rows=args.split_rows)
        ws = new_workspace(step, dev)
        call = DecodeCall(step, q, k_new, v_new, k_cache, v_cache, pos_d, out=out, workspace=ws)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    with torch.cuda.stream(stream):
        warm_steps = warm_up(lambda: call(stream), args.warmup)
        # Eager: K steps (append + attend + merge) issued one by one.
        ms_eager = timed(lambda: call(stream), args.steps)
        # Graph: the decode loop's production form -- steps replayed from a HIP graph, so
        # no host launch cost sits between them.  Each replay is checked against eager.
        per_graph = 10
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(per_graph):
                call(stream)
        warm_up(graph.replay, 1, 0.5)
        reps = max(1, args.steps // per_graph)
        ms_graph = timed(graph.replay, reps) / per_graph
        # Dominant kernel alone (split-K attend with the fused append), same stream, also
        # replayed from a graph: eager launches of a few-microsecond kernel would time the
        # host's launch rate instead (C1: ~5 us between back-to-back eager launches).
        g_att = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_att, stream=stream):
            for _ in range(per_graph):
                call(stream, STAGE_ATTEND)
        warm_up(g_att.replay, 1, 0.5)
        ms_attend = timed(g_att.replay, reps) / per_graph
        ref = out.clone()
        call(stream)
        torch.cuda.synchronize()
        graph_ok = bool(torch.equal(out, ref))
    ms_step = ms_graph if graph_ok else ms_eager

    # Cold-cache timing: a working set below 1 GiB stays in the 256 MB MALL between steps,
    # so the same step is also timed rotating over ceil(1 GiB / working set) distinct caches
    # (one graph replay visits each once).
    ms_cold = None
    ws_bytes = k_cache.numel() * 2 * (1 if (w["shared"] or raw is not None) else 2)
    if ws_bytes < (1 << 30) and raw is None and not args.no_cold:
        sets = -(-(1 << 30) // ws_bytes)
        calls = []
        for _ in range(sets):
            kc = torch.empty_like(k_cache).copy_(k_cache)
            vc = kc if w["shared"] else torch.empty_like(v_cache).copy_(v_cache)
            calls.append(DecodeCall(step, q, k_new, v_new, kc, vc, pos_d, out=out, workspace=ws))
        with torch.cuda.stream(stream):
            for c in calls:
                c(stream)
            gcold = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gcold, stream=stream):
                for c in calls:
                    c(stream)
            warm_up(gcold.replay, 1, 0.5)
            ms_cold = timed(gcold.replay, max(2, args.steps // sets)) / sets
        del calls, gcold

    nbytes = algorithmic_bytes(w, pos)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    gbs_attend = nbytes / (ms_attend * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        if raw is not None and w.get("q8"):
            cpu = cpu_baseline_q8(w, pos, q, raw, args.cpu_threads)
        elif raw is not None:
            cpu = cpu_baseline_raw(w, pos, q, k_cache, raw[0], raw[1], args.cpu_threads)
        else:
            cpu = cpu_baseline(w, pos, q, k_cache, v_cache, k_new, v_new, args.cpu_threads)

    line = {
        "metric": "decode-attn HBM GB/s (and us/step) at Gemma-4-31B shapes, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_step, 6),
        "us_per_step": round(ms_step * 1e3, 3),
        "us_per_step_eager": round(ms_eager * 1e3, 3),
        "us_per_step_graph": round(ms_graph * 1e3, 3),
        "us_per_step_cold": None if ms_cold is None else round(ms_cold * 1e3, 3),
        "timing": "HIP graph replay of the step (eager launches alongside)" if graph_ok else "eager",
        "pct_of_hbm_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, unit-RMS, bf16" +
                ("; 64 keys per kv head +4.0 along the query direction)" if w.get("peaks") else ")"),
        "config": {
            "workload": {"c4": "C4 global k_eq_v decode, L=131072", "c2": "C2 global k_eq_v decode, L=8193",
                         "c1": "C1 local decode, L=1024", "c3": "C3 local ring decode, B=8",
                         "c4raw": "C4 shape, raw-K mode (K/V rebuilt in-kernel), L=131072",
                         "c4q8": "C4 shape, q8 raw-K stream (u8 rows + scale/bias, K/V rebuilt in-kernel), "
                                 "L=131072"}[args.workload],
            "batch": B, "num_q_heads": Hq, "num_kv_heads": Hkv, "head_dim": D,
            "visible_rows": visible_rows(w, pos), "kv_shared": w["shared"],
            "window": w["window"], "ring": w["ring"], "split_rows": step.split_rows or "auto",
            "algorithmic_bytes_per_step": nbytes,
            **({"rope_table": "precomputed per model (esda_rope_table): 256 B per cache row read per "
                              "pair of kv heads, beside the algorithmic bytes"} if w.get("raw") else {}),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("attend_kernel<512,shared,raw,q8> (u8 widening + raw-K rebuild + split-K + fused quantize-append)"
                       if w.get("q8") else
                       "attend_kernel<512,shared,raw> (raw-K rebuild + split-K + fused append)" if raw is not None
                       else "attend_kernel<D,kv_shared> (split-K + fused append)"),
            "achieved": round(gbs_attend, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs_attend / PEAK_HBM_GBS, 4), "traffic": profiled_traffic(args.workload),
            "traffic_source": f"profiles/attend_{args.workload}.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "kernel_us": round(ms_attend * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "device": device_facts(),
    }
    print(json.dumps(line), flush=True)
    return 0


def device_facts() -> dict:
    """What the runtime reports for cuda:0, beside the figures the roofline assumes (256 CUs,
    wave64, 288 GB of HBM3E, 160 KB of LDS per CU)."""
    import torch

    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", None), "compute_units": p.multi_processor_count,
            "wave_size": getattr(p, "warp_size", None), "hbm_bytes": p.total_memory,
            "l2_bytes": getattr(p, "L2_cache_size", None),
            "lds_bytes_per_workgroup": getattr(p, "shared_memory_per_block", None)}


def profiled_traffic(workload: str, kind: str = "attend"):
    """HBM bytes per launch of the dominant kernel measured by rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (calibrated against a plain copy), as recorded in
    profiles/<kind>_<workload>.md; None when that workload has no profile."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{kind}_{workload}.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def calibrate_copy(args) -> int:
    """A plain device-to-device copy of known size: the rocprofv3 FETCH_SIZE / WRITE_SIZE
    readings of this kernel give the factor between those counters and true HBM bytes."""
    import torch

    n = args.calibrate_copy << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(max(1, args.warmup)):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n,
                      "us": round(ms * 1e3, 3), "GB/s": round(2 * n / (ms * 1e-3) / 1e9, 2)}), flush=True)
    return 0


def calibrate_read(args) -> int:
    """One pass over a buffer of known size through the attend kernel's load path
    (esda_stream_read: LDS DMA, non-temporal, 1 KiB per wave instruction), timed with HIP
    events on the launch stream: the stream-read ceiling the attend kernel is measured
    against, and (under rocprofv3 --pmc FETCH_SIZE) the counter's factor on that path."""
    import torch

    from apertura_amd._lib import check, lib

    n = args.calibrate_read << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    stream = torch.cuda.current_stream()
    results = []
    for wgs in ((args.read_workgroups,) if args.read_workgroups else (256, 512, 1024, 2048)):
        sink = torch.zeros(4 * wgs, dtype=torch.int32, device="cuda:0")

        def launch():
            check(lib().esda_stream_read(src.data_ptr(), n, wgs, sink.data_ptr(), stream.cuda_stream))

        warm_up(launch, max(1, args.warmup), 0.5)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        results.append({"workgroups": wgs, "us": round(ms * 1e3, 3), "GB/s": round(n / (ms * 1e-3) / 1e9, 2)})
    best = max(results, key=lambda r: r["GB/s"])
    print(json.dumps({"calibration": "stream read (global_load_lds_dwordx4 nt, esda_stream_read)",
                      "bytes_read": n, "best": best, "sweep": results,
                      "frac_of_8TBs": round(best["GB/s"] / PEAK_HBM_GBS, 4)}), flush=True)
    return 0


def calibrate_lds(args) -> int:
    """LDS read rate of the prefill kernel's two operand read forms (esda_lds_read), one
    workgroup per CU of 4, 8 or 16 waves, timed with HIP events on the launch stream: the
    ceiling its per-stage LDS bytes are priced against."""
    import torch

    from apertura_amd._lib import check, lib

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 4000
    stream = torch.cuda.current_stream()
    results = []
    for tr in (0, 1):
        for waves in (4, 8, 16):
            sink = torch.zeros(cus * waves * 64, dtype=torch.int32, device="cuda:0")

            def launch():
                check(lib().esda_lds_read(waves, tr, iters, cus, sink.data_ptr(), stream.cuda_stream))

            warm_up(launch, max(1, args.warmup), 0.5)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                launch()
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / args.steps
            n = cus * waves * 64 * iters * 8 * (8 if tr else 16)
            results.append({"read": "ds_read_b64_tr_b16" if tr else "ds_read_b128", "waves_per_cu": waves,
                            "us": round(ms * 1e3, 3), "TB/s": round(n / (ms * 1e-3) / 1e12, 2),
                            "GB/s_per_cu": round(n / (ms * 1e-3) / 1e9 / cus, 1)})
    print(json.dumps({"calibration": "LDS read rate (esda_lds_read)", "cus": cus, "workgroups": cus,
                      "results": results}), flush=True)
    return 0


def prefill_visible_pairs(w) -> int:
    """Sum over query rows of the keys each sees (per query head)."""
    import numpy as np
    qa = w["q_pos0"] + np.arange(w["Sq"], dtype=np.int64)
    lo = np.full_like(qa, w["k_pos0"]) if not w["window"] else np.maximum(w["k_pos0"], qa - w["window"] + 1)
    hi = np.minimum(qa, w["k_pos0"] + w["Sk"] - 1)
    return int(np.maximum(hi - lo + 1, 0).sum())


def bench_prefill(args) -> int:
    """One prefill attention call per step (esda_prefill: attention kernel + split merge)."""
    import numpy as np
    import torch

    from apertura_amd.prefill import STAGE_ATTEND, PrefillStep, prefill, prefill_workspace_bytes

    w = PREFILL_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def rms_bf16(shape):
        x = torch.randn(shape, device=dev, dtype=torch.float32, generator=gen)
        x = x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6)
        return x.to(torch.bfloat16)

    Hq, Hkv, D, Sq, Sk = w["Hq"], w["Hkv"], w["D"], w["Sq"], w["Sk"]
    q, k = rms_bf16((Hq, Sq, D)), rms_bf16((Hkv, Sk, D))
    v = k if w.get("shared") else rms_bf16((Hkv, Sk, D))
    out = torch.empty((Sq, Hq, D), dtype=torch.bfloat16, device=dev)
    step = PrefillStep(num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, seq_q=Sq, seq_k=Sk, q_pos0=w["q_pos0"],
                       k_pos0=w["k_pos0"], window=w["window"], scale=w["scale"])
    ws = torch.empty(max(1, prefill_workspace_bytes(step)), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream()

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    with torch.cuda.stream(stream):
        call = lambda: prefill(step, q, k, v, out, ws, stream)
        attend = lambda: prefill(step, q, k, v, out, ws, stream, stages=STAGE_ATTEND)
        warm_steps = warm_up(call, args.warmup)
        ms_step = timed(call, args.steps)
        ms_attend = timed(attend, args.steps)
        call()
    torch.cuda.synchronize()

    pairs = prefill_visible_pairs(w)
    flops = 4 * D * Hq * pairs
    tf = flops / (ms_step * 1e-3) / 1e12
    tf_attend = flops / (ms_attend * 1e-3) / 1e12
    cpu = None if args.no_cpu else cpu_baseline_prefill(w, q, k, v, args.cpu_threads)
    line = {
        "metric": "prefill-attn TFLOP/s at Gemma-4-31B shapes, 1 GPU",
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_step, 6),
        "us_per_step": round(ms_step * 1e3, 3),
        "timing": "eager (one esda_prefill per step)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, unit-RMS, bf16)",
        "config": {"workload": w["name"], "num_q_heads": Hq, "num_kv_heads": Hkv, "head_dim": D, "seq_q": Sq,
                   "seq_k": Sk, "q_pos0": w["q_pos0"], "k_pos0": w["k_pos0"], "window": w["window"],
                   "visible_pairs_per_head": pairs, "algorithmic_flops_per_step": flops,
                   "key_splits": (prefill_workspace_bytes(step) > 0)},
        "roofline": {
            "bound": "mfma",
            "kernel": f"prefill_kernel<{D}> (QK and PV on v_mfma_f32_16x16x32_bf16, online softmax)",
            "achieved": round(tf_attend, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf_attend / PEAK_BF16_TFLOPS, 4), "traffic": profiled_traffic(args.workload, "prefill"),
            "traffic_source": f"profiles/prefill_{args.workload}.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "kernel_us": round(ms_attend * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "device": device_facts(),
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_prefill(w, q, k, v, threads: int):
    """The fp64 prefill oracle on the host over a sample of query rows (rows are
    independent; every row sees its full visible key range), doubled until >= 10 s."""
    import numpy as np
    import torch

    from oracle import oracle as orc

    qh = q.cpu().view(torch.int16).numpy().view(np.uint16)
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16)
    vh = v.cpu().view(torch.int16).numpy().view(np.uint16)
    Sq = w["Sq"]
    n, secs, pairs = 1, 0.0, 0
    while True:
        rows = np.linspace(0, Sq - 1, num=min(n, Sq)).astype(int)
        t0 = time.perf_counter()
        for r in rows:
            orc.prefill_f64(qh[:, r:r + 1], kh, vh, w["q_pos0"] + int(r), w["k_pos0"], w["window"], w["scale"],
                            threads=threads)
        secs = time.perf_counter() - t0
        sub = dict(w, Sq=1)
        pairs = sum(prefill_visible_pairs(dict(sub, q_pos0=w["q_pos0"] + int(r))) for r in rows)
        if secs >= 10.0 or len(rows) >= Sq:
            break
        n *= 2
    flops = 4 * w["D"] * w["Hq"] * pairs
    return {"value": round(flops / secs / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{len(rows)} of {Sq} query rows (all heads, full visible key ranges), fp64 prefill oracle, "
                      f"{secs:.1f} s"}


def bench_c5(args) -> int:
    """60-layer attention step at B=32 (see the module docstring)."""
    import numpy as np
    import torch

    from apertura_amd.decode import DecodeCall, DecodeStep, STAGE_ATTEND

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(55)
    lens = [int(x) for x in rng.integers(1024, 32769, size=C5_B)]
    pos = [n - 1 for n in lens]
    gcap = max(lens)
    gen = torch.Generator(device=dev)
    gen.manual_seed(55)

    def rms_bf16(shape):
        out = torch.empty(shape, device=dev, dtype=torch.bfloat16)
        flat = out.view(-1, shape[-1])
        for r0 in range(0, flat.shape[0], 1 << 20):
            x = torch.randn((min(1 << 20, flat.shape[0] - r0), shape[-1]), device=dev, generator=gen)
            flat[r0:r0 + x.shape[0]] = (x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6)).bfloat16()
        return out

    pos_d = torch.tensor(pos, dtype=torch.int32, device=dev)
    g_split = args.split_rows  # 0: the library's automatic split (balanced over the batch)
    l_split = args.local_split_rows
    calls, kinds, nbytes = [], [], 0
    shared_q = {}
    for layer in range(C5_LAYERS):
        t = C5_GLOBAL if c5_is_global(layer) else C5_LOCAL
        cap = gcap if c5_is_global(layer) else t["cap"]
        key = "g" if c5_is_global(layer) else "l"
        if key not in shared_q:
            shared_q[key] = (rms_bf16((C5_B, t["Hq"], t["D"])), rms_bf16((C5_B, t["Hkv"], t["D"])),
                             None if t["shared"] else rms_bf16((C5_B, t["Hkv"], t["D"])))
        q, kn, vn = shared_q[key]
        kc = rms_bf16((C5_B, t["Hkv"], cap, t["D"]))
        vc = kc if t["shared"] else rms_bf16((C5_B, t["Hkv"], cap, t["D"]))
        step = DecodeStep.for_cache(kc, t["Hq"], window=t["window"], ring=t["ring"], kv_shared=t["shared"],
                                    scale=t["scale"], split_rows=g_split if c5_is_global(layer) else l_split)
        calls.append(DecodeCall(step, q, kn, vn, kc, vc, pos_d))
        kinds.append(key)
        vis = [min(n, t["window"]) if t["window"] else n for n in lens]
        row = t["D"] * 2 * (1 if t["shared"] else 2)
        nbytes += sum(vis) * t["Hkv"] * row + 2 * C5_B * t["Hq"] * t["D"] * 2 + 2 * C5_B * t["Hkv"] * row
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()

    def step_all(stages=3, only=None):
        for c, k in zip(calls, kinds):
            if only is None or k == only:
                c(stream, stages)

    def graph_of(stages, only=None):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            step_all(stages, only)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=stream):
                step_all(stages, only)
        warm_up(g.replay, 1, 0.5)  # a fresh graph's first replays run slow
        return g

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    with torch.cuda.stream(stream):
        warm_steps = warm_up(step_all, max(1, args.warmup // 10))
        ms_eager = timed(step_all, max(2, args.steps // 10))
        g_full, g_att = graph_of(3), graph_of(STAGE_ATTEND)
        ms_graph = timed(g_full.replay, max(2, args.steps // 10))
        ms_att = timed(g_att.replay, max(2, args.steps // 10))
        ms_local = timed(graph_of(3, "l").replay, max(2, args.steps // 10))
        ms_global = timed(graph_of(3, "g").replay, max(2, args.steps // 10))
        # Every layer's output of one eager step against one replay of the step's graph, bit
        # for bit (each step appends the same rows at the same positions, so the steps are
        # idempotent); a mismatch reports the eager time instead.
        step_all()
        torch.cuda.synchronize()
        eager_out = [c.out.clone() for c in calls]
        for c in calls:
            c.out.zero_()
        g_full.replay()
        torch.cuda.synchronize()
        graph_ok = all(bool(torch.equal(c.out, e)) for c, e in zip(calls, eager_out))
    ms_step = ms_graph if graph_ok else ms_eager
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    traffic = profiled_traffic_c5()
    cpu = None if args.no_cpu else cpu_baseline_c5(calls, kinds, lens, pos, args.cpu_threads)
    line = {
        "metric": "decode-attn HBM GB/s (and us/step) at Gemma-4-31B shapes, 1 GPU",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": max(2, args.steps // 10), "warmup": args.warmup, "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_step, 6), "us_per_step": round(ms_step * 1e3, 3),
        "us_per_step_eager": round(ms_eager * 1e3, 3), "us_per_step_graph": round(ms_graph * 1e3, 3),
        "graph_matches_eager": graph_ok,
        "timing": ("HIP graph replay of the 60-layer step (120 kernels)" if graph_ok
                   else "eager (the graph replay differed from eager)"),
        "pct_of_hbm_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, unit-RMS, bf16)",
        "config": {"workload": "C5 Gemma-4-31B attention step: 60 layers (50 local D256 ring 1024, "
                               "10 global D512 k_eq_v), B=32, len~U[1024,32768]",
                   "batch": C5_B, "lengths_min_mean_max": [min(lens), sum(lens) // len(lens), max(lens)],
                   "global_split_rows": g_split, "local_split_rows": l_split or "auto",
                   "algorithmic_bytes_per_step": nbytes,
                   "us_50_local_layers": round(ms_local * 1e3, 1), "us_10_global_layers": round(ms_global * 1e3, 1)},
        "roofline": {"bound": "hbm", "kernel": "attend_kernel (all 60 layers, merges excluded)",
                     "achieved": round(nbytes / (ms_att * 1e-3) / 1e9, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(nbytes / (ms_att * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": traffic["step"] if traffic else None,
                     "traffic_per_launch": traffic,
                     "traffic_source": "profiles/attend_c5.md (rocprofv3 FETCH_SIZE + WRITE_SIZE per attend "
                                       "dispatch, copy-calibrated): 50 local + 10 global launches per step",
                     "kernel_us": round(ms_att * 1e3, 3)},
        "cpu_baseline": cpu,
        "device": device_facts(),
    }
    print(json.dumps(line), flush=True)
    return 0


def profiled_traffic_c5():
    """HBM bytes per attend launch of C5's local and global layers (profiles/attend_c5.md,
    rocprofv3 FETCH_SIZE / WRITE_SIZE, copy-calibrated) and per step (50 local + 10 global
    launches); None when the profile is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "attend_c5.md")
    got = {}
    try:
        for line in open(path):
            for kind in ("local", "global"):
                tag = f"traffic_bytes_per_launch_{kind}:"
                if line.startswith(tag):
                    got[kind] = int(float(line.split(":", 1)[1].split()[0]))
    except OSError:
        return None
    if len(got) != 2:
        return None
    n_global = sum(1 for layer in range(C5_LAYERS) if c5_is_global(layer))
    got["step"] = (C5_LAYERS - n_global) * got["local"] + n_global * got["global"]
    return got


def cpu_baseline_c5(calls, kinds, lens, pos, threads: int):
    """The reference-rounding restatement (orc_decode_refround_grouped) over one local and
    one global layer of the C5 step at full shape (B=32, the same caches and positions, after
    the same append), each repeated for >= 5 s; the 60-layer step is estimated as 50 x the
    local time + 10 x the global time (every layer of a kind has the same shape and work)."""
    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    from oracle import oracle as orc

    def host(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    secs, nbytes, reps_of = {}, {}, {}
    for kind, t in (("l", C5_LOCAL), ("g", C5_GLOBAL)):
        c = calls[kinds.index(kind)]
        q, kn, vn, kc, vc = c._keep[:5]
        cap = kc.shape[2]
        step = orc.Step(B=C5_B, Hq=t["Hq"], Hkv=t["Hkv"], D=t["D"], cap=cap, window=t["window"], ring=t["ring"],
                        scale=t["scale"])
        kch = host(kc)
        vch = kch if t["shared"] else host(vc)
        knh = host(kn).reshape(C5_B, t["Hkv"], t["D"])
        vnh = knh if t["shared"] else host(vn).reshape(C5_B, t["Hkv"], t["D"])
        orc.append(step, kch, None if t["shared"] else vch, knh, None if t["shared"] else vnh, pos)
        qh = host(q).reshape(C5_B, t["Hq"], t["D"])
        reps, total = 0, 0.0
        while total < 5.0 and reps < 200:
            t0 = time.perf_counter()
            orc.decode_refround_grouped(step, qh, kch, vch, pos, threads=threads)
            total += time.perf_counter() - t0
            reps += 1
        secs[kind], reps_of[kind] = total / reps, reps
        vis = [min(n, t["window"]) if t["window"] else n for n in lens]
        row = t["D"] * 2 * (1 if t["shared"] else 2)
        nbytes[kind] = sum(vis) * t["Hkv"] * row + 2 * C5_B * t["Hq"] * t["D"] * 2 + 2 * C5_B * t["Hkv"] * row
    n_global = sum(1 for layer in range(C5_LAYERS) if c5_is_global(layer))
    n_local = C5_LAYERS - n_global
    sec = n_local * secs["l"] + n_global * secs["g"]
    step_bytes = n_local * nbytes["l"] + n_global * nbytes["g"]
    return {"value": round(step_bytes / sec / 1e9, 3), "unit": "GB/s", "us_per_step": round(sec * 1e6, 1),
            "cores": threads, "kind": "port",
            "sample": f"one local layer x{reps_of['l']} ({secs['l'] * 1e3:.1f} ms each) and one global layer "
                      f"x{reps_of['g']} ({secs['g'] * 1e3:.1f} ms each) at full C5 shape, reference-rounding "
                      f"restatement grouped by kv head over {threads} threads; step = {n_local} x local + "
                      f"{n_global} x global (MLX CPU path unavailable offline); host {os.cpu_count()} cpus visible"}


def cpu_baseline(w, pos, q, k_cache, v_cache, k_new, v_new, threads: int):
    """CPU port of the reference-rounding restatement of ESAttention.mm:136-165 on the same
    inputs, after the same append: orc_decode_refround_grouped (each K / V row read once for
    the query heads of its kv head, the rows of a (sequence, kv head) split over the threads;
    bit-identical to orc_decode_refround with one split).  Timed for ~10 s of CPU work over
    repeats."""
    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    from oracle import oracle as orc

    def host(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    B, Hq, Hkv, D, cap = w["B"], w["Hq"], w["Hkv"], w["D"], w["cap"]
    step = orc.Step(B=B, Hq=Hq, Hkv=Hkv, D=D, cap=cap, window=w["window"], ring=w["ring"],
                    scale=w["scale"])
    qh = host(q).reshape(B, Hq, D)
    kc = host(k_cache)
    vc = kc if w["shared"] else host(v_cache)
    kn = host(k_new).reshape(B, Hkv, D)
    vn = kn if w["shared"] else host(v_new).reshape(B, Hkv, D)
    orc.append(step, kc, None if w["shared"] else vc, kn, None if w["shared"] else vn, pos)
    reps, t_total = 0, 0.0
    while t_total < 10.0 and reps < 1000:
        t0 = time.perf_counter()
        orc.decode_refround_grouped(step, qh, kc, vc, pos, threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    sec = t_total / reps
    nbytes = algorithmic_bytes(w, pos)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "us_per_step": round(sec * 1e6, 1),
            "cores": threads, "kind": "port",
            "sample": f"full workload step x{reps} repeats ({t_total:.1f} s), reference-rounding "
                      f"restatement grouped by kv head over {threads} threads (MLX CPU path unavailable "
                      f"offline); host {os.cpu_count()} cpus visible"}


def cpu_baseline_raw(w, pos, q, k_cache, kw, inv_freq, threads: int):
    """CPU oracle of the raw-K step (orc_decode_raw_f64: the reconstruction of
    ESDecodeAttn.mm:17-117 in fp64, query heads over the threads) over the full step's rows,
    repeated for >= 10 s; throughput in the step's algorithmic bytes."""
    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    from oracle import oracle as orc

    def host(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    B, Hq, Hkv, D = w["B"], w["Hq"], w["Hkv"], w["D"]
    rows = visible_rows(w, pos)[0]
    qh = host(q).reshape(B, Hq, D)[0]
    raw = np.ascontiguousarray(host(k_cache).reshape(B, Hkv, -1, D)[0])  # the appended row is in place
    kwh = host(kw).reshape(-1)
    inv = inv_freq.detach().cpu().numpy()
    reps, t_total = 0, 0.0
    while t_total < 10.0 and reps < 50:
        t0 = time.perf_counter()
        orc.decode_raw_f64(qh, raw, rows, kwh, 1e-6, inv, w["scale"], threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    sec = t_total / reps
    nbytes = algorithmic_bytes(w, pos)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "us_per_step": round(sec * 1e6, 1),
            "cores": threads, "kind": "port",
            "sample": f"full step ({rows} rows per kv head) x{reps} repeats ({t_total:.1f} s), fp64 raw-K "
                      f"oracle, query heads over {threads} threads (MLX CPU path unavailable offline); "
                      f"host {os.cpu_count()} cpus visible"}


def cpu_baseline_q8(w, pos, q, raw, threads: int):
    """CPU oracle of the q8 raw-K step (orc_decode_raw_q8_f64) over the full step's rows, as
    cpu_baseline_raw; throughput in the step's algorithmic bytes (520 per row)."""
    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    from oracle import oracle as orc

    kw, inv_freq, q8, sc, bs = raw
    B, Hq, Hkv, D = w["B"], w["Hq"], w["Hkv"], w["D"]
    rows = visible_rows(w, pos)[0]
    qh = q.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(B, Hq, D)[0]
    q8h = np.ascontiguousarray(q8[0].cpu().numpy())  # the appended row is quantized in place
    sch = np.ascontiguousarray(sc[0].cpu().numpy())
    bsh = np.ascontiguousarray(bs[0].cpu().numpy())
    kwh = kw.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
    inv = inv_freq.detach().cpu().numpy()
    reps, t_total = 0, 0.0
    while t_total < 10.0 and reps < 50:
        t0 = time.perf_counter()
        orc.decode_raw_q8_f64(qh, q8h, sch, bsh, rows, kwh, 1e-6, inv, w["scale"], threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    sec = t_total / reps
    nbytes = algorithmic_bytes(w, pos)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "us_per_step": round(sec * 1e6, 1),
            "cores": threads, "kind": "port",
            "sample": f"full step ({rows} rows per kv head) x{reps} repeats ({t_total:.1f} s), fp64 q8 "
                      f"raw-K oracle, query heads over {threads} threads (MLX CPU path unavailable offline); "
                      f"host {os.cpu_count()} cpus visible"}


if __name__ == "__main__":
    sys.exit(main())
