"""Benchmark of the flash-attention backward on one MI355X.

Workload (BASELINE.json metric): B=4, H=12, N=4096, d=64, causal, bf16 inputs
with fp32 accumulation. Synthetic seeded N(0,1) Q, K, V, dO generated on the
GPU. The forward (O, LSE) runs once before the timed region, as in the
reference (02-flash-attention/src/main.rs:599-611). One timed step = one full
backward pass from O (mxfa_run_bwd): the dQ pass with Delta = rowsum(dO * O)
folded in, then the dK/dV pass, inputs resident in HBM (--separate-delta: the
reference-shaped preprocess launch + dQ pass + dK/dV pass instead).

Prints one JSON line. ``value`` is the algorithmic backward throughput
(10 N^2 d per (batch, head), halved for causal) in TFLOP/s. ``roofline`` is the
dominant kernel's achieved MFMA rate against MI355X's dense bf16 peak, with the
probe kernels' ceilings measured in the same run beside it (``measured_peak``,
``hbm_measured_gbps``). ``cpu_baseline`` times the CPU oracle (a C restatement
of the reference's CPU backward, main.rs:246-300) on a bounded sample of the
same workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-probe]
       [--B 4 --H 12 --Hkv 12 --N 4096 --d 64 --causal 1 --dtype bf16]
       python bench.py --naive-table   (the reference's naive-vs-flash tables, one JSON line)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}  # MI355X dense MFMA (AMD public spec)
METRIC = "FA bwd TFLOP/s + % MFMA peak at B=4,H=12,N=4096,d=64 causal, 1 MI355X"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # the MI355X raises its clocks over the first ~30 ms of sustained load (and
    # drops them again within 0.5 s idle): 200 steps (~65 ms) put the timed
    # steps past that ramp
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--B", type=int, default=4)
    ap.add_argument("--H", type=int, default=12)
    ap.add_argument("--Hkv", type=int, default=0, help="0 = same as H")
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--d", type=int, default=64)
    ap.add_argument("--causal", type=int, default=1)
    ap.add_argument("--dtype", choices=["bf16", "f32"], default="bf16")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--two-launch", action="store_true",
                    help="time the two-launch backward (dQ pass with Delta, then dK/dV) even where one "
                         "launch is available (set_bwd_options(one_launch=False))")
    # the MI355X raises its clocks over the first ~30 ms of sustained load and
    # drops them again within 0.5 s idle: before the --warmup steps, forward
    # launches run for at least this long (reported as clock_warmup_ms /
    # clock_warmup_fwd_launches, apart from "warmup")
    ap.add_argument("--clock-warmup-ms", type=float, default=150.0)
    ap.add_argument("--separate-delta", action="store_true",
                    help="run the reference-shaped sequence (preprocess launch, then the dQ pass reading Delta)")
    ap.add_argument("--no-probe", action="store_true",
                    help="skip the roofline probes (measured MFMA / HBM ceilings, after the timed region)")
    ap.add_argument("--naive-table", action="store_true",
                    help="instead of the benchmark, time the naive and flash paths on the reference's own "
                         "tables (one fp32 head, d = 64) and print them as one JSON line")
    ap.add_argument("--atomic-probe", action="store_true",
                    help="time the writes a dQ pass fused into the dK/dV pass would make (fp32 atomics "
                         "vs plain stores) at the bench shape, next to the separate dQ pass")
    ap.add_argument("--mix-probe", action="store_true",
                    help="instruction-mix ceilings (mxfa_probe_mix) beside the bf16 kernels' executed MFMA rates "
                         "at the bench shape")
    ap.add_argument("--timeline", action="store_true",
                    help="per-work-group timeline of one one-launch backward at the bench shape (timeline build "
                         "of the code object, mxfa_gfx950_timeline.hsaco)")
    ap.add_argument("--config-table", action="store_true",
                    help="forward and backward timings at every BASELINE config (one JSON line); with the CPU path "
                         "timed per config unless --no-cpu")
    ap.add_argument("--prefill-table", action="store_true",
                    help="the prefill (mxfa_run_prefill), the paged prefill (mxfa_run_prefill_paged, "
                         "16-row blocks) and both with their keys split (mxfa_run_prefill_ws, "
                         "mxfa_run_prefill_paged_ws) at engine shapes (one JSON line)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run a plain device-to-device copy of MIB "
                         "MiB three times (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def copy_probe(mib):
    """A plain copy kernel of known size: reads and writes exactly mib MiB per
    launch, so FETCH_SIZE / WRITE_SIZE read for it give the counters' scale."""
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_per_launch": n * 4, "launches": 3}), flush=True)


# The reference's published MX230 timings for the same rows (ms), for the table
# mode: 02-flash-attention/README.md:16-21 (forward, non-causal) and :85-87
# (backward, causal; flash = dQ pass + dK/dV pass, preprocess excluded).
REF_FWD_MS = {1024: (17.0, 1.4), 2048: (64.7, 4.1), 4096: (275.9, 16.3), 8192: (1152.2, 60.8),
              16384: (4762.1, 250.4), 32768: (None, 992.9)}
REF_BWD_MS = {1024: (43.53, 3.90), 2048: (165.12, 14.43), 4096: (641.55, 54.50)}


def naive_table():
    """The reference's naive-vs-flash tables on one MI355X: one head, d = 64,
    fp32, seeded N(0,1) inputs; each entry the median of 5 timed runs after
    one warm-up (the reference's time_median_ms, common/src/lib.rs:22-43).
    Forward: non-causal, naive = scores + softmax + S.V through the N x N
    scratch (attention_naive.cu), flash = mxfa_run_flash. Backward: causal,
    naive = the atomic kernel into zeroed outputs (zeroing inside the timed
    launch sequence, as its caller must), flash = mxfa_run_bwd_flash (dQ pass +
    dK/dV pass; the preprocess excluded, main.rs:603-611)."""
    import torch
    import mx230_amd as mx
    dev = torch.device("cuda", 0)
    mx.init(0)

    def median_ms(fn):
        # the reference's WARMUP = 1, ITERS = 5 (main.rs:15-16)
        return mx.time_median_ms(fn, warmup=mx.WARMUP, iters=mx.ITERS)

    gen = torch.Generator(device=dev)
    rows = []
    for n in sorted(REF_FWD_MS):
        gen.manual_seed(n)
        q, k, v, do = (torch.randn((1, 1, n, 64), generator=gen, device=dev) for _ in range(4))
        o = torch.empty_like(q)
        flash = median_ms(mx.prepare(mx.run_flash, q, k, v, o, False))
        naive = None
        if n <= 16384:
            s = torch.empty(mx.naive_scratch_bytes(q, k, False) // 4, device=dev)
            naive = median_ms(lambda: mx.naive_run(q, k, v, s, o, False))
            del s
        ref_naive, ref_flash = REF_FWD_MS[n]
        rows.append({"pass": "fwd", "causal": False, "N": n, "naive_ms": naive and round(naive, 4),
                     "flash_ms": round(flash, 4), "speedup": naive and round(naive / flash, 1),
                     "flash_tflops": round(mx.fwd_flops(1, 1, n, 64, False) / (flash * 1e-3) / 1e12, 2),
                     "mx230_naive_ms": ref_naive, "mx230_flash_ms": ref_flash})
        if n in REF_BWD_MS:
            lse = torch.empty((1, 1, n), device=dev)
            delta = torch.empty_like(lse)
            mx.run_flash_lse(q, k, v, o, lse, True)
            mx.run_preprocess(do, o, delta)
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            flash = median_ms(mx.prepare(mx.run_bwd_flash, q, k, v, do, lse, delta, dq, dk, dv, True))

            def naive_bwd():
                dq.zero_()
                dk.zero_()
                dv.zero_()
                mx.run_bwd_naive(q, k, v, do, lse, delta, dq, dk, dv, True)
            naive = median_ms(naive_bwd)
            ref_naive, ref_flash = REF_BWD_MS[n]
            rows.append({"pass": "bwd", "causal": True, "N": n, "naive_ms": round(naive, 4),
                         "flash_ms": round(flash, 4), "speedup": round(naive / flash, 1),
                         "flash_tflops": round(mx.bwd_flops(1, 1, n, 64, True) / (flash * 1e-3) / 1e12, 2),
                         "mx230_naive_ms": ref_naive, "mx230_flash_ms": ref_flash})
    print(json.dumps({"naive_table": rows, "dtype": "f32", "B": 1, "H": 1, "d": 64,
                      "data": "synthetic (seeded N(0,1) on the GPU)",
                      "timing": "median of 5 after 1 warm-up, HIP events on the launch stream"}), flush=True)


# (name, B, Hq, Hkv, N, d, causal, dtype, Q/K/V scale)
CONFIGS = [
    ("cfg1 reference CPU case", 1, 1, 1, 256, 64, False, "f32", 1.0),
    ("cfg2 GPT-2", 4, 12, 12, 1024, 64, True, "f32", 0.5),
    ("cfg3 long sequence", 1, 12, 12, 32768, 64, False, "f32", 1.0),
    ("cfg3 long sequence", 1, 12, 12, 32768, 64, False, "bf16", 1.0),
    ("cfg4 Qwen2.5 GQA 7:1", 2, 14, 2, 4096, 64, True, "bf16", 1.0),
    ("cfg5 TinyLlama GQA 8:1", 1, 32, 4, 2048, 64, True, "bf16", 0.5),
    ("cfg5 TinyLlama GQA 8:1", 1, 32, 4, 2048, 128, True, "bf16", 0.5),
    ("north star", 4, 12, 12, 4096, 64, True, "bf16", 1.0),
]


def prefill_table():
    """The inference-side forward at the reference engine's shapes (Qwen2.5-0.5B:
    14 query heads over 2 KV heads; TinyLlama-1.1B: 32 over 4; head_dim 64): a
    first chunk, a chunk after history and a single row after history, over a
    contiguous cache (mxfa_run_prefill; mxfa_run_prefill_ws, its keys split
    over work-groups where the query blocks alone would not fill the GPU) and
    a paged one (mxfa_run_prefill_paged, 16-row blocks in shuffled order, the
    engine's KV_BLOCK; mxfa_run_prefill_paged_ws split), fp32 (the engine's
    cache) and bf16. Token-major rows, a fused QKV buffer as the engine has; median of
    per-call event pairs after warm-up (mx.time_median_ms), which for the
    short launches holds the host's time to issue the call (the kernels'
    own durations: rocprofv3 --kernel-trace of this mode). TFLOP/s: the
    causal work 4 d sum_i (pos0 + i + 1) per query head, over the call time."""
    import torch
    import mx230_amd as mx
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    rows = []
    for model, nh, nkv in (("Qwen2.5-0.5B", 14, 2), ("TinyLlama-1.1B", 32, 4)):
        for n_tok, pos0 in ((512, 0), (512, 3584), (4096, 0), (1, 4095)):
            for dt in (torch.float32, torch.bfloat16):
                hd, bs = 64, 16
                nk = pos0 + n_tok
                nblk = -(-nk // bs)
                qkv = torch.randn((n_tok, (nh + 2 * nkv) * hd), generator=gen, device=dev).to(dt)
                kc = torch.randn((nblk * bs, nkv * hd), generator=gen, device=dev).to(dt)
                vc = torch.randn_like(kc)
                perm = torch.randperm(nblk, device=dev, generator=gen).to(torch.int32)
                kp, vp = torch.empty_like(kc), torch.empty_like(vc)
                kp.view(nblk, bs, -1)[perm.long()] = kc.view(nblk, bs, -1)
                vp.view(nblk, bs, -1)[perm.long()] = vc.view(nblk, bs, -1)
                out = torch.empty((n_tok, nh * hd), device=dev, dtype=dt)
                q = qkv[:, :nh * hd]
                flops = 4.0 * hd * nh * (n_tok * (pos0 + 1) + n_tok * (n_tok - 1) / 2)
                contig = mx.time_median_ms(lambda: mx.run_prefill(q, kc, vc, out, pos0, nh, nkv, hd),
                                           warmup=20, iters=21)
                paged = mx.time_median_ms(lambda: mx.run_prefill_paged(q, kp, vp, out, perm, bs, pos0, nh, nkv, hd),
                                          warmup=20, iters=21)
                ws = mx.run_prefill_split(q, kc, vc, out, pos0, nh, nkv, hd)
                split = mx.time_median_ms(lambda: mx.run_prefill_split(q, kc, vc, out, pos0, nh, nkv, hd,
                                                                       workspace=ws), warmup=20, iters=21)
                mx.run_prefill_paged(q, kp, vp, out, perm, bs, pos0, nh, nkv, hd, split=True, workspace=ws)
                psplit = mx.time_median_ms(lambda: mx.run_prefill_paged(q, kp, vp, out, perm, bs, pos0, nh, nkv, hd,
                                                                        split=True, workspace=ws),
                                           warmup=20, iters=21)
                nsplit = mx.prefill_workspace_bytes(n_tok, pos0, nh, nkv, hd, dt == torch.bfloat16) // \
                    (nh * n_tok * (hd + 2) * 4)
                rows.append({"model": model, "n_head": nh, "n_kv_head": nkv, "head_dim": hd, "n_tok": n_tok,
                             "pos0": pos0, "dtype": "bf16" if dt == torch.bfloat16 else "f32",
                             "contiguous_call_us": round(contig * 1e3, 1), "paged_call_us": round(paged * 1e3, 1),
                             "key_splits": max(nsplit, 1), "split_call_us": round(split * 1e3, 1),
                             "paged_split_call_us": round(psplit * 1e3, 1),
                             "contiguous_tflops": round(flops / (contig * 1e-3) / 1e12, 1),
                             "paged_tflops": round(flops / (paged * 1e-3) / 1e12, 1),
                             "split_tflops": round(flops / (split * 1e-3) / 1e12, 1),
                             "paged_split_tflops": round(flops / (psplit * 1e-3) / 1e12, 1)})
                print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    print(json.dumps({"prefill_table": rows, "block_size": 16}), flush=True)


def cpu_config(B, H, Hkv, N, d, causal, dtype, sc, threads):
    """The reference's CPU path (cpu_attention, then cpu_attention_bwd,
    02-flash-attention/src/main.rs:213-300) for one config, timed on the oracle:
    one (batch, head) slice on one thread, as the reference runs it, scaled to
    the config's B*H slices; and min(B*H, threads) slices on that many threads
    (the oracle's multi-head forward and backward), scaled the same way. Inputs
    seeded N(0,1) (x sc for Q/K/V), rounded to bf16 for a bf16 config; fp32
    math either way. Above N = 8192 (cfg3: one slice would take minutes) the
    slices are timed at N = 4096 and scaled by (N / 4096)^2 as well: the
    path's work per slice is N^2 d. Returns the figures and what was sampled."""
    import numpy as np
    import mx230_amd as mx
    import oracle  # the checker; used here only as the timed CPU baseline
    lib = oracle.load()
    nsl = min(B * H, threads)
    n_full = N
    if N > 8192:
        N = 4096
    nscale = (n_full / N) ** 2
    q = oracle.normal(nsl * N * d, 11, sc).reshape(1, nsl, N, d)
    k = oracle.normal(nsl * N * d, 12, sc).reshape(1, nsl, N, d)
    v = oracle.normal(nsl * N * d, 13, sc).reshape(1, nsl, N, d)
    do = oracle.normal(nsl * N * d, 14, 1.0).reshape(1, nsl, N, d)
    if dtype == "bf16":
        q, k, v, do = (oracle.bf16_round(x) for x in (q, k, v, do))
    t0 = time.perf_counter()
    oracle.cpu_attention(q[0, 0], k[0, 0], v[0, 0], N, d, causal, lib=lib)
    oracle.cpu_attention_bwd(q[0, 0], k[0, 0], v[0, 0], do[0, 0], N, d, causal, lib=lib)
    t1 = time.perf_counter() - t0
    t0 = time.perf_counter()
    oracle.mha_fwd(q, k, v, 1, nsl, nsl, N, d, causal, nthreads=nsl, lib=lib)
    oracle.mha_bwd(q, k, v, do, 1, nsl, nsl, N, d, causal, nthreads=nsl, lib=lib)
    tp = time.perf_counter() - t0
    del np
    flops = mx.fwd_flops(B, H, n_full, d, causal) + mx.bwd_flops(B, H, n_full, d, causal)
    whole1 = t1 * B * H * nscale
    wholep = tp * B * H / nsl * nscale
    at = f" at N={N}, scaled x{nscale:g} for N={n_full}," if nscale != 1 else ""
    return {"cpu_1t_s": round(whole1, 2), "cpu_1t_tflops": flops / whole1 / 1e12,
            "cpu_par_s": round(wholep, 2), "cpu_par_tflops": flops / wholep / 1e12, "cpu_threads": nsl,
            "cpu_sample": f"fwd+bwd of 1 slice on 1 thread ({t1:.2f} s) and of {nsl} slices on {nsl} threads "
                          f"({tp:.2f} s){at} each scaled x{B * H}/(slices) to the config's {B * H} slices"}


def config_table(cpu=False):
    """Forward (mxfa_run_flash_lse) and backward from O (mxfa_run_bwd_ws: the
    dQ pass with Delta, then dK/dV, split over the query heads of a GQA group
    through its workspace where that applies) at every BASELINE config, each the median of
    20 event-timed runs after 3 warm-ups, inputs resident. TFLOP/s are the
    algorithmic 4 N^2 d (forward) and 10 N^2 d (backward) per (batch, query
    head), halved when causal; % peak against the dense MFMA peak of the dtype,
    and frac_of_measured against the MFMA probe's rate on this box. cpu: each
    row also carries the reference's CPU path timed on this host (cpu_config:
    one thread, and one thread per slice over up to 16 slices)."""
    import torch
    import mx230_amd as mx
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    stream = torch.cuda.current_stream()
    measured = {"bf16": mx.probe_mfma_tflops(True), "f32": mx.probe_mfma_tflops(False)}
    host = cpu_host()
    threads = max(1, min(16, os.cpu_count() or 1))

    def median_ms(fn, reps=20):
        # warm-up: at least 50 ms of back-to-back calls (the clocks ramp up
        # over the first ~30 ms of load) and at least 3 calls
        t0 = time.perf_counter()
        n = 0
        while n < 3 or time.perf_counter() - t0 < 0.05:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for e0, e1 in evs:
            e0.record(stream)
            fn()
            e1.record(stream)
        torch.cuda.synchronize()
        return sorted(e0.elapsed_time(e1) for e0, e1 in evs)[reps // 2]

    rows = []
    for name, B, H, Hkv, N, d, causal, dtype, sc in CONFIGS:
        dt = torch.bfloat16 if dtype == "bf16" else torch.float32
        gen = torch.Generator(device=dev)
        gen.manual_seed(N + H + d)
        qs, ks = (B, H, N, d), (B, Hkv, N, d)
        q, k, v = (torch.randn(s, generator=gen, device=dev).mul_(sc).to(dt) for s in (qs, ks, ks))
        do = torch.randn(qs, generator=gen, device=dev).to(dt)
        o = torch.empty_like(q)
        lse = torch.empty((B, H, N), device=dev)
        delta = torch.empty_like(lse)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        fwd = median_ms(mx.prepare(mx.run_flash_lse, q, k, v, o, lse, causal))
        nws = mx.bwd_workspace_bytes(q, k, causal)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
        bwd = median_ms(mx.prepare(mx.run_bwd_ws, q, k, v, o, do, lse, delta, dq, dk, dv, ws, causal))
        peak = PEAK_TFLOPS[dtype]
        ftf = mx.fwd_flops(B, H, N, d, causal) / (fwd * 1e-3) / 1e12
        btf = mx.bwd_flops(B, H, N, d, causal) / (bwd * 1e-3) / 1e12
        meas = measured[dtype]
        rows.append({"config": name, "B": B, "Hq": H, "Hkv": Hkv, "N": N, "d": d, "causal": causal,
                     "dtype": dtype, "workspace_mb": round(nws / 1e6, 1), "fwd_ms": round(fwd, 4), "fwd_tflops": round(ftf, 2),
                     "fwd_pct_peak": round(100 * ftf / peak, 1), "fwd_frac_of_measured": round(ftf / meas, 3),
                     "bwd_ms": round(bwd, 4), "bwd_tflops": round(btf, 2), "bwd_pct_peak": round(100 * btf / peak, 1),
                     "bwd_frac_of_measured": round(btf / meas, 3)})
        del q, k, v, do, o, lse, delta, dq, dk, dv, ws
        if cpu:
            c = cpu_config(B, H, Hkv, N, d, causal, dtype, sc, threads)
            c["gpu_vs_cpu_1t"] = round(c["cpu_1t_s"] / ((fwd + bwd) * 1e-3), 1)
            c["cpu_1t_tflops"] = float(f"{c['cpu_1t_tflops']:.3g}")
            c["cpu_par_tflops"] = float(f"{c['cpu_par_tflops']:.3g}")
            rows[-1].update(c)
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    print(json.dumps({"config_table": rows, "peak_tflops": PEAK_TFLOPS,
                      "measured_mfma_tflops": {k: round(x, 1) for k, x in measured.items()}, "host": host,
                      "data": "synthetic (seeded N(0,1) on the GPU; Q/K/V x0.5 where BASELINE says so)",
                      "timing": "median of 20 after >= 50 ms of warm-up calls, HIP events on the launch stream"}), flush=True)


def atomic_probe(a):
    """The alternative to the separate dQ pass, measured: the fp32 atomic adds
    a dQ pass fused into the dK/dV pass would issue at the bench shape (one
    64 x 64 partial tile per (128-key block, 64-query stage), causal, d = 64),
    and plain stores of the same bytes, beside the separate dQ pass's own time
    (with Delta folded in, mean of 20 launches)."""
    import torch
    import mx230_amd as mx
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    bh = a.B * a.H
    at = mx.probe_dq_atomic(bh, a.N, atomic=True)
    st = mx.probe_dq_atomic(bh, a.N, atomic=False)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    qs = (a.B, a.H, a.N, 64)
    q, k, v, do = (torch.randn(qs, generator=gen, device=dev).to(torch.bfloat16) for _ in range(4))
    o = torch.empty_like(q)
    lse = torch.empty((a.B, a.H, a.N), device=dev)
    delta = torch.empty_like(lse)
    dq = torch.empty_like(q)
    mx.run_flash_lse(q, k, v, o, lse, True)
    dq_ms = mx._time_ms(lambda: mx.run_bwd_dq_delta(q, k, v, o, do, lse, delta, dq, True), 20)
    print(json.dumps({"atomic_probe": {"B*H": bh, "N": a.N, "d": 64, "causal": True,
                                       "payload_mb": round(at["payload_bytes"] / 1e6, 1),
                                       "atomic_us": round(at["us"], 1), "atomic_tbps": round(at["tbps"], 3),
                                       "store_us": round(st["us"], 1), "store_tbps": round(st["tbps"], 3),
                                       "separate_dq_pass_us": round(dq_ms * 1e3, 1)}}), flush=True)


def mix_probe(a):
    """Each bf16 kernel's executed MFMA rate at the bench shape beside the
    ceiling of its instruction mix (mxfa_probe_mix: the same per-MFMA counts
    of exp / mul / cvt / LDS reads, issued with no dependencies) at two and
    three waves per SIMD. Kernel times: median of 40 per-launch event pairs
    after >= 150 ms of warm-up launches; ceilings: mean of 10 launches after
    >= 150 ms of warm-up."""
    import time
    import torch
    import mx230_amd as mx
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    stream = torch.cuda.current_stream()

    def warm(fn):
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 0.15:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()

    def median_ms(fn, reps=40):
        warm(fn)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        for i in range(reps):
            ev[i].record(stream)
            fn()
        ev[reps].record(stream)
        torch.cuda.synchronize()
        return sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))[reps // 2]

    B, H, N, d, causal = a.B, a.H, a.N, a.d, bool(a.causal)
    hkv = a.Hkv or a.H
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    q, do = (torch.randn((B, H, N, d), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn((B, hkv, N, d), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    o, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    lse = torch.empty((B, H, N), device=dev)
    delta = torch.empty_like(lse)
    mx.run_flash_lse(q, k, v, o, lse, causal)
    unit = N * N * d * B * H * (0.5 if causal else 1.0)  # x k N^2 d flops per (b, h)
    kern = {"fwd": (4, mx.prepare(mx.run_flash_lse, q, k, v, o, lse, causal)),
            "dq": (6, mx.prepare(mx.run_bwd_dq_delta, q, k, v, o, do, lse, delta, dq, causal)),
            "dkv": (8, mx.prepare(mx.run_bwd_dkv, q, k, v, do, lse, delta, dk, dv, causal)),
            "bwd_one_launch": (14, mx.prepare(mx.run_bwd, q, k, v, o, do, lse, delta, dq, dk, dv, causal))}
    kernels = {}
    for name, (mult, fn) in kern.items():
        ms = median_ms(fn)
        kernels[name] = {"us": round(ms * 1e3, 1), "executed_tflops": round(mult * unit / (ms * 1e-3) / 1e12, 1)}
    ceilings = {}
    for mix in mx.PROBE_MIXES:
        for w in (2, 3):
            warm(lambda: mx.probe_mix_tflops(mix, w, iters=256, reps=1))
            ceilings[f"{mix}_w{w}"] = round(mx.probe_mix_tflops(mix, w, iters=256, reps=10), 1)
    of_ceiling = {name: round(kernels[name]["executed_tflops"] / ceilings[f"{mix}_w3"], 3)
                  for name, mix in (("fwd", "fwd"), ("dq", "dq"), ("dkv", "dkv"))}
    print(json.dumps({"mix_probe": {"shape": {"B": B, "Hq": H, "Hkv": hkv, "N": N, "d": d, "causal": causal},
                                    "kernels": kernels, "ceilings_tflops": ceilings,
                                    "kernel_over_its_mix_ceiling_w3": of_ceiling,
                                    "peak_tflops": PEAK_TFLOPS["bf16"]}}), flush=True)


def _timeline_pass(t, stages, slots):
    """Summary of one kernel's work-groups (t: [groups, 4] microseconds from
    the launch's first start)."""
    pro, loop, epi = t[:, 1] - t[:, 0], t[:, 2] - t[:, 1], t[:, 3] - t[:, 2]
    busy = t[:, 3] - t[:, 0]
    return {"work_groups": int(len(t)), "first_start_us": round(float(t[:, 0].min()), 1),
            "last_start_us": round(float(t[:, 0].max()), 1), "last_end_us": round(float(t[:, 3].max()), 1),
            "prologue_us_mean": round(float(pro.mean()), 2),
            "loop_us_per_stage_mean": round(float((loop / stages).mean()), 3),
            "epilogue_us_mean": round(float(epi.mean()), 2),
            "prologue_share_of_resident_time": round(float(pro.sum() / busy.sum()), 3)}


def _timeline_launch(full, kinds, names):
    """Summary of one launch from its rows of the timeline build's array:
    span, the work-groups resident at once (the most of them is the slots the
    launch had: CUs x work-groups per CU), the work-groups' resident time over
    those slots, per pass (kind) prologue / loop per stage / epilogue, and the
    five work-groups that end last."""
    import numpy as np
    kind, blk, stages = full[:, 4] >> 32, full[:, 4] & 0xffffffff, full[:, 5]
    t = (full[:, :4] - full[:, 0].min()) * 0.01  # microseconds
    span = float(t[:, 3].max())
    ev = np.concatenate([np.stack([t[:, 0], np.ones(len(t))], 1), np.stack([t[:, 3], -np.ones(len(t))], 1)])
    ev = ev[np.lexsort((ev[:, 1], ev[:, 0]))]  # ends before starts at equal times
    slots = int(np.cumsum(ev[:, 1]).max())
    g = np.arange(len(t))
    out = {"span_us": round(span, 1), "slots_observed": slots,
           "resident_time_over_slots_us": round(float((t[:, 3] - t[:, 0]).sum() / slots), 1),
           # work-groups go to the 8 XCDs round robin in dispatch order
           "first_start_by_xcd_us": [round(float(t[g % 8 == x, 0].min()), 1) for x in range(8)]}
    for k, name in zip(kinds, names):
        sel = kind == k
        out[name] = _timeline_pass(t[sel], stages[sel], slots)
    grid = np.linspace(0.0, span, 21)
    out["resident_work_groups_every_5pct_of_span"] = [int(((t[:, 0] <= g) & (t[:, 3] > g)).sum()) for g in grid]
    out["last_to_end"] = [{"kind": names[kinds.index(int(kind[i]))], "block": int(blk[i]), "stages": int(stages[i]),
                           "start_us": round(float(t[i, 0]), 1), "loop_start_us": round(float(t[i, 1]), 1),
                           "end_us": round(float(t[i, 3]), 1)} for i in np.argsort(-t[:, 3])[:5]]
    return out


def timeline(a):
    """One one-launch backward and one forward at the bench shape (bf16,
    causal or not; with --Hkv below --H, the backward through the GQA split's
    workspace) with the timeline build of the code object: for each kernel
    its span, the work-groups resident over the launch, their resident time
    summed over the slots it had (the most resident at once), each pass's
    prologue (start until its first stage is staged), loop time per stage and
    epilogue (until its stores are acknowledged), and the work-groups that end
    last. Each measured launch follows >= 150 ms of calls of the same kind,
    the last eight of them queued back to back with it."""
    import numpy as np
    import torch
    import mx230_amd as mx
    if not os.path.exists(mx.TIMELINE_CODE_OBJECT_PATH):
        sys.exit(f"bench.py --timeline: {mx.TIMELINE_CODE_OBJECT_PATH} is missing (make -C mx230_amd/csrc timeline)")
    mx.set_code_object(mx.TIMELINE_CODE_OBJECT_PATH)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    B, H, N, d, causal = a.B, a.H, a.N, a.d, bool(a.causal)
    Hkv = a.Hkv or H
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    q, do = (torch.randn((B, H, N, d), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn((B, Hkv, N, d), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    o, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(k)
    lse = torch.empty((B, H, N), device=dev)
    delta = torch.empty_like(lse)
    nws = mx.bwd_workspace_bytes(q, k, causal)
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
    assert mx.bwd_one_launch(q, k, causal), "the timeline reads the one-launch backward"

    def warm(fn):
        # >= 150 ms of calls, the last 8 queued back to back with the measured
        # one: after an idle gap (a synchronisation) the first launch has been
        # seen to start on some XCDs up to ~30 us after the others
        t0 = time.perf_counter()
        n = 0
        while n % 8 != 7 or time.perf_counter() - t0 < 0.15:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()

    out = {"shape": {"B": B, "Hq": H, "Hkv": Hkv, "N": N, "d": d, "causal": causal},
           "dkv_partial_planes": int(max(nws // (8 * B * Hkv * N * d), 1))}
    mx.run_flash_lse(q, k, v, o, lse, causal)
    # the backward's work-groups: dQ, then dK/dV, then (GQA split) the reduce;
    # rows past them are zero, an earlier launch's (older stamps) or the
    # forward's
    warm(lambda: mx.run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, ws, causal))
    mx.run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, ws, causal)
    torch.cuda.synchronize()
    full = mx.probe_wg_times().astype(np.int64)
    kind = full[:, 4] >> 32
    ndq = int(np.argmin(kind == 0))
    cur = ((kind[ndq:] == 1) | (kind[ndq:] == 3)) & (full[ndq:, 0] >= full[:ndq, 0].min())
    nwg = len(full) if cur.all() else ndq + int(np.argmin(cur))
    full = full[:nwg]
    red = bool((kind[:nwg] == 3).any())
    out["backward"] = _timeline_launch(full, [0, 1, 3] if red else [0, 1],
                                       ["dq", "dkv", "reduce"] if red else ["dq", "dkv"])
    # the forward's work-groups: the leading rows it stamped (kind 2)
    warm(lambda: mx.run_flash_lse(q, k, v, o, lse, causal))
    mx.run_flash_lse(q, k, v, o, lse, causal)
    torch.cuda.synchronize()
    full = mx.probe_wg_times().astype(np.int64)
    kind = full[:, 4] >> 32
    nwg = len(full) if np.all(kind == 2) else int(np.argmin(kind == 2))
    out["forward"] = _timeline_launch(full[:nwg], [2], ["fwd"])
    print(json.dumps({"timeline": out}), flush=True)


def cpu_host():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu": model}


def cpu_parallel(a, hkv):
    """The oracle's multi-head backward over (batch, head) slices on a thread
    per slice (the parallel CPU figure): 16 slices on up to 16 threads, the
    host share of a one-GPU box."""
    import numpy as np
    import oracle  # the checker; used here only as the timed CPU baseline
    lib = oracle.load()
    threads = max(1, min(16, os.cpu_count() or 1))
    nheads = min(16, a.B * a.H)
    N, d = a.N, a.d
    q = np.stack([oracle.normal(N * d, 5000 + i).reshape(N, d) for i in range(nheads)])[None]
    k = np.stack([oracle.normal(N * d, 6000 + i).reshape(N, d) for i in range(nheads)])[None]
    v = np.stack([oracle.normal(N * d, 7000 + i).reshape(N, d) for i in range(nheads)])[None]
    do = np.stack([oracle.normal(N * d, 8000 + i).reshape(N, d) for i in range(nheads)])[None]
    if a.dtype == "bf16":
        q, k, v, do = (oracle.bf16_round(x) for x in (q, k, v, do))
    t0 = time.perf_counter()
    oracle.mha_bwd(q, k, v, do, 1, nheads, nheads, N, d, bool(a.causal), nthreads=threads, lib=lib)
    dt = time.perf_counter() - t0
    import mx230_amd as mx
    flops = mx.bwd_flops(1, nheads, N, d, bool(a.causal))
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads,
            "sample": f"backward of {nheads} (batch, head) slices at N={N}, d={d}, {threads} threads; {dt:.1f} s"}


def cpu_baseline(a, hkv):
    """Times the CPU oracle on a bounded sample of the same workload: the
    backward of the first 16 (batch, head) slices on one thread (the reference's
    CPU path is single-threaded), inputs bf16-rounded as the GPU sees them."""
    import numpy as np
    import oracle  # the checker; used here only as the timed CPU baseline
    lib = oracle.load()
    nheads = min(16, a.B * a.H)
    N, d = a.N, a.d
    group = a.H // hkv
    tot = 0.0
    for i in range(nheads):
        h = i % a.H
        q = oracle.normal(N * d, 1000 + i).reshape(N, d)
        k = oracle.normal(N * d, 2000 + h // group).reshape(N, d)
        v = oracle.normal(N * d, 3000 + h // group).reshape(N, d)
        do = oracle.normal(N * d, 4000 + i).reshape(N, d)
        if a.dtype == "bf16":
            q, k, v, do = (oracle.bf16_round(x) for x in (q, k, v, do))
        t0 = time.perf_counter()
        oracle.cpu_attention_bwd(q, k, v, do, N, d, bool(a.causal), lib=lib)
        tot += time.perf_counter() - t0
    import mx230_amd as mx
    flops = mx.bwd_flops(1, nheads, N, d, bool(a.causal))
    del np
    return {"value": flops / tot / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"backward of {nheads} of the {a.B * a.H} (batch, head) slices at N={N}, "
                      f"d={d}, causal={bool(a.causal)}, {a.dtype}-rounded inputs, fp32 math, "
                      f"1 thread; {tot:.1f} s"}


def main():
    a = parse()
    if a.copy_probe:
        copy_probe(a.copy_probe)
        return
    if a.naive_table:
        naive_table()
        return
    if a.config_table:
        config_table(cpu=not a.no_cpu)
        return
    if a.prefill_table:
        prefill_table()
        return
    if a.atomic_probe:
        atomic_probe(a)
        return
    if a.mix_probe:
        mix_probe(a)
        return
    if a.timeline:
        timeline(a)
        return
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {a.gpus}); the path shards "
              "over (batch, KV head) with no exchange, so the one-GPU figure is the per-GPU "
              "share. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import mx230_amd as mx

    hkv = a.Hkv or a.H
    causal = bool(a.causal)
    bf16 = a.dtype == "bf16"
    dt = torch.bfloat16 if bf16 else torch.float32
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mx.init(0)
    mx.load_library()

    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    qs, ks = (a.B, a.H, a.N, a.d), (a.B, hkv, a.N, a.d)
    q = torch.randn(qs, generator=gen, device=dev, dtype=torch.float32).to(dt)
    k = torch.randn(ks, generator=gen, device=dev, dtype=torch.float32).to(dt)
    v = torch.randn(ks, generator=gen, device=dev, dtype=torch.float32).to(dt)
    do = torch.randn(qs, generator=gen, device=dev, dtype=torch.float32).to(dt)
    o = torch.empty_like(q)
    lse = torch.empty((a.B, a.H, a.N), device=dev, dtype=torch.float32)
    delta = torch.empty_like(lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    # forward once: O and LSE for the backward (outside the timed region; the
    # forward is timed on its own after the backward regions, with the clocks up)
    stream = torch.cuda.current_stream()
    mx.run_flash_lse(q, k, v, o, lse, causal)
    torch.cuda.synchronize()

    if a.two_launch:
        mx.set_bwd_options(one_launch=False)
    # the backward from O as mxfa_run_bwd runs it: one launch (dQ work-groups
    # publish Delta for the dK/dV work-groups of the same launch) where
    # available, else the dQ pass with Delta then the dK/dV pass; with
    # --separate-delta the reference-shaped sequence preprocess, dQ, dK/dV
    one = not a.separate_delta and mx.bwd_one_launch(q, k, causal)
    if a.separate_delta:
        launches = [("preprocess", mx.prepare(mx.run_preprocess, do, o, delta)),
                    ("dq", mx.prepare(mx.run_bwd_dq, q, k, v, do, lse, delta, dq, causal)),
                    ("dkv", mx.prepare(mx.run_bwd_dkv, q, k, v, do, lse, delta, dk, dv, causal))]
    elif one:
        launches = [("bwd", mx.prepare(mx.run_bwd, q, k, v, o, do, lse, delta, dq, dk, dv, causal))]
    else:
        launches = [("dq", mx.prepare(mx.run_bwd_dq_delta, q, k, v, o, do, lse, delta, dq, causal)),
                    ("dkv", mx.prepare(mx.run_bwd_dkv, q, k, v, do, lse, delta, dk, dv, causal))]

    def step(seq, evs=None):
        # evs: events recorded on the launch stream before each launch and after the last
        for j, (_, launch) in enumerate(seq):
            if evs:
                evs[j].record(stream)
            launch()
        if evs:
            evs[len(seq)].record(stream)

    def per_launch_ms(seq):
        evsets = [[torch.cuda.Event(enable_timing=True) for _ in range(len(seq) + 1)] for _ in range(a.steps)]
        torch.cuda.synchronize()
        for evs in evsets:
            step(seq, evs)
        torch.cuda.synchronize()
        return {n: sum(evs[j].elapsed_time(evs[j + 1]) for evs in evsets) / a.steps for j, (n, _) in enumerate(seq)}

    # clock warm-up, reported on its own: forward launches (the producer of O
    # and LSE) for --clock-warmup-ms, so the clocks are up when the first
    # backward runs and every backward dispatch in the run (the W warm-up
    # steps and the timed ones) is a warm one; then the requested warm-up steps
    cw0 = time.perf_counter()
    cw_steps = 0
    while (time.perf_counter() - cw0) * 1e3 < a.clock_warmup_ms:
        mx.run_flash_lse(q, k, v, o, lse, causal)
        cw_steps += 1
        if cw_steps % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    cw_ms = (time.perf_counter() - cw0) * 1e3
    for _ in range(a.warmup):
        step(launches)
    torch.cuda.synchronize()
    fb0 = mx.bwd_delta_fallbacks() if one else 0
    rt0 = mx.bwd_reduce_timeouts() if one else 0

    # timed region: exactly K backward steps, synchronised on both sides, with
    # an event on the launch stream before each step and after the last: the
    # median of the K per-step times is the headline (the reference's
    # time_median_ms, common/src/lib.rs:22-43), their mean beside it
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps + 1)]
    torch.cuda.synchronize()
    for i in range(a.steps):
        evs[i].record(stream)
        step(launches)
    evs[a.steps].record(stream)
    torch.cuda.synchronize()
    per_step = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(a.steps))
    ms_median = per_step[a.steps // 2] if a.steps % 2 else 0.5 * (per_step[a.steps // 2 - 1] +
                                                                  per_step[a.steps // 2])
    ms_mean = evs[0].elapsed_time(evs[a.steps]) / a.steps
    ms_per_step = ms_median

    # the roofline's basis: each launch's duration from HIP events on the
    # launch stream. With one launch per step that is the timed region itself
    # (one event between consecutive launches; each interval also holds the
    # ~6 us dispatch gap a kernel-trace duration leaves out); otherwise a second
    # region of K steps with events around each launch
    kern = {launches[0][0]: ms_median} if len(launches) == 1 else per_launch_ms(launches)
    # the two passes on their own (two launches), for the breakdown
    passes = None
    if one:
        passes = per_launch_ms([("dq", mx.prepare(mx.run_bwd_dq_delta, q, k, v, o, do, lse, delta, dq, causal)),
                                ("dkv", mx.prepare(mx.run_bwd_dkv, q, k, v, do, lse, delta, dk, dv, causal))])

    # the forward: K launches back to back after a few warm-up ones, one event
    # pair around them (O and LSE are rewritten with the same values)
    fwd_call = mx.prepare(mx.run_flash_lse, q, k, v, o, lse, causal)
    for _ in range(5):
        fwd_call()
    f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    f0.record(stream)
    for _ in range(a.steps):
        fwd_call()
    f1.record(stream)
    torch.cuda.synchronize()
    fwd_avg = f0.elapsed_time(f1) / a.steps

    half = 0.5 if causal else 1.0
    bwd_flops = mx.bwd_flops(a.B, a.H, a.N, a.d, causal)
    # algorithmic MFMA work of each kernel per launch: dK/dV pass computes the
    # S, dP, dV, dK products (8 N^2 d per (batch, query head)); the dQ pass the
    # S, dP, dQ products (6 N^2 d) -- S and dP are recomputed by both passes
    kflops = {"dkv": 8.0 * a.N * a.N * a.d * a.B * a.H * half,
              "dq": 6.0 * a.N * a.N * a.d * a.B * a.H * half}
    executed = kflops["dkv"] + kflops["dq"]
    # the one launch does the algorithmic backward (10 N^2 d) and executes 14
    kflops["bwd"] = bwd_flops
    dom = max((n for n in kern if n in kflops), key=lambda n: kern[n])
    peak = PEAK_TFLOPS[a.dtype]
    achieved = kflops[dom] / (kern[dom] * 1e-3) / 1e12
    value = bwd_flops / (ms_per_step * 1e-3) / 1e12
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{dom}_{a.dtype}_B{a.B}H{a.H}N{a.N}d{a.d}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")

    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_mean": round(ms_mean, 4), "ms_per_step_min_max": [round(per_step[0], 4), round(per_step[-1], 4)],
        "timing": "median of the per-step event pairs of the timed region (mean beside it)",
        "clock_warmup_ms": round(cw_ms, 1), "clock_warmup_fwd_launches": cw_steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": a.dtype,
        "data": "synthetic (seeded N(0,1) on the GPU)",
        "config": {"workload": ("flash-attention backward, one launch (dQ with Delta + dK/dV), fwd outside timing"
                                if one else
                                "flash-attention backward (dQ with Delta folded in + dK/dV), fwd outside timing"
                                if not a.separate_delta else
                                "flash-attention backward (preprocess + dQ + dK/dV), fwd outside timing"),
                   "B": a.B, "Hq": a.H, "Hkv": hkv, "N": a.N, "d": a.d, "causal": causal,
                   "parallelism": "single GPU"},
        "pct_peak": round(100.0 * value / peak, 2),
        # MFMA work the two passes execute per step (the dQ pass recomputes S
        # and dP: 14 N^2 d per (batch, head), halved when causal) over the step
        "executed_tflops": round(executed / (ms_per_step * 1e-3) / 1e12, 2),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic},
        "kernels_ms": {n: round(t, 4) for n, t in kern.items()},
        "fwd": {"ms": round(fwd_avg, 4),
                "tflops": round(mx.fwd_flops(a.B, a.H, a.N, a.d, causal) / (fwd_avg * 1e-3) / 1e12, 2)},
    }
    if dom == "bwd":
        # the one launch executes 14 N^2 d (the dQ pass recomputes S and dP)
        res["roofline"]["executed"] = round(executed / (kern[dom] * 1e-3) / 1e12, 2)
    if one:
        # Delta blocks whose wait ran out in the timed regions (0 expected;
        # results are the same either way)
        res["delta_fallbacks"] = mx.bwd_delta_fallbacks() - fb0
        # GQA split reduce waits that ran out (0 expected; NaN rows otherwise)
        res["reduce_timeouts"] = mx.bwd_reduce_timeouts() - rt0
    if passes is not None:
        res["passes_ms"] = {n: round(t, 4) for n, t in passes.items()}
    if not a.no_probe:
        # measured ceilings (probe kernels, after the timed region): the same
        # MFMA pipe at full occupancy with independent accumulators, and HBM
        # streaming reads; `peak` stays AMD's published figure
        # the MFMA form the backward runs
        mfma = mx.probe_mfma_tflops(bf16=a.dtype == "bf16", iters=256)
        res["roofline"]["measured_peak"] = round(mfma, 1)
        res["roofline"]["measured_peak_mfma"] = ("v_mfma_f32_16x16x32_bf16" if a.dtype == "bf16" else
                                                 "v_mfma_f32_16x16x4_f32")
        res["roofline"]["frac_of_measured"] = round(achieved / mfma, 4)
        res["roofline"]["hbm_measured_gbps"] = round(mx.probe_hbm_gbps(mib=1024), 1)
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(a, hkv)
        res["cpu_baseline"]["parallel"] = cpu_parallel(a, hkv)
        res["cpu_baseline"]["host"] = cpu_host()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
