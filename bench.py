#!/usr/bin/env python3
"""Benchmark of the per-step attention path on one MI355X.

A step is one pass of the hot path over one synthetic batch: GPU pack, fused QK-norm/RoPE/
paged append, decode (split-K + combine) and prefill, for every layer of the config.  The
default workload is config 2 (64 decode sequences, contexts U[512, 4096], one Qwen3-8B
layer); `--config 3|4|5` runs the others.  The step is captured once as a HIP graph and
replayed (as the reference replays decode steps, model_runtime.cu:227-233); inputs are
resident in HBM before timing starts.

Prints ONE JSON line.  `roofline` is for the dominant kernel of the workload (decode: HBM
bytes; prefill: MFMA flops), timed with HIP events around a graph of repeated launches of
that kernel on the stream it is launched on.  `cpu_baseline` is the OpenMP fp32 CPU oracle
(oracle/fqa_oracle.c) timed on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=5, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--no-prefill-lines", action="store_true",
                    help="config 5: skip the config 3/4 prefill measurements added under "
                         "the line's 'prefill' key")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--dec-grid-waves", type=int, default=None,
                    help="decode wavefronts (default: CUs x 4, one per SIMD)")
    ap.add_argument("--dec-min-pages", type=int, default=8)
    ap.add_argument("--pre-tile-q", type=int, default=64, choices=[32, 64])
    ap.add_argument("--layers", type=int, default=None, help="config 5 only (default 36)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only copy 1 GiB device to device 3 times (the reference dispatch "
                         "that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only run the per-kernel graphs (for rocprofv3 passes)")
    ap.add_argument("--sampler", action="store_true",
                    help="only measure fqa_sample (256 rows x 151936 logits: greedy, "
                         "temperature, temperature + top-p 0.9)")
    ap.add_argument("--no-dec-share", action="store_true",
                    help="mixed steps with the second stream: plan the decode for the whole "
                         "device (no dec_share)")
    ap.add_argument("--no-overlap", action="store_true",
                    help="mixed steps: keep the decode on the step's stream (by default it "
                         "runs on a second stream beside the prefill, planned for the CUs "
                         "the prefill leaves: dec_share)")
    ap.add_argument("--dec-prefix-pages", type=int, default=None,
                    help="decode sequences sharing at least this many leading pages attend "
                         "them once per group (fqa_decode_prefix); default 8 on config 5 "
                         "(its 4 groups of 24 sequences on 128-page prefixes), 0 (off) "
                         "elsewhere.  The line also times the decode without it")
    ap.add_argument("--gemm", action="store_true",
                    help="only measure fqa_gemm on the Qwen3-8B projections (decode and "
                         "prefill row counts) beside torch.matmul (hipBLASLt)")
    ap.add_argument("--gemm-rows", type=str, default="128,256,1024,8192",
                    help="row counts for --gemm")
    ap.add_argument("--compat-append", action="store_true",
                    help="also time the compat route's norm/RoPE and append as two launches "
                         "(fqa_qknorm_rope + fqa_store_kv, as fqa_compat.hpp issues them) "
                         "beside the fused fqa_qknorm_rope_append")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the attention path is "
                          "per-GPU work (kv-head or sequence sharding needs no exchange); "
                          "run with --gpus 1"}))
        sys.exit(2)
    if args.copy_calib:
        import torch

        x = torch.ones(2**28, device="cuda", dtype=torch.float32)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": x.numel() * 4, "copies": 3}))
        return

    if args.sampler:
        bench_sampler(args)
        return
    if args.gemm:
        bench_gemm(args)
        return

    device = None if args.profile_kernels else device_info()
    pre = None
    if args.config == 5 and not args.no_prefill_lines and not args.profile_kernels:
        # the metric's second half: prefill MFMA utilisation on the two prefill configs,
        # measured in the same process before config 5 (right after config 5's 36-layer
        # sweep over its 200 GB pool the prefill runs ~10% slower: the clock under sustained
        # load); each config's pool is released before the next is built
        import gc

        import torch

        pre = {}
        for c in (3, 4):
            sub = run_config(args, c, steps=max(args.steps, 20), warmup=args.warmup,
                             with_cpu=not args.no_cpu)
            pre[f"config{c}"] = {"workload": sub["config"]["workload"],
                                 "ms_per_step": sub["ms_per_step"],
                                 "tokens_per_s": sub["value"],
                                 "rows_per_step": sub["config"]["rows_per_step"],
                                 "roofline": sub["roofline"],
                                 "kernels_us": sub["kernels_us"],
                                 "step_floor_us": sub["step_floor_us"],
                                 "step_minus_floor_us": sub["step_minus_floor_us"],
                                 "decode_beside_prefill": sub["decode_beside_prefill"],
                                 "cpu_baseline": sub["cpu_baseline"]}
            gc.collect()
            torch.cuda.empty_cache()
    line = run_config(args, args.config, steps=args.steps, warmup=args.warmup,
                      with_cpu=not args.no_cpu)
    if line is None:  # --profile-kernels
        return
    line["device"] = device
    if pre is not None:
        line["prefill"] = pre
        # the same rooflines, compact, beside the decode's
        line["roofline"]["prefill_configs"] = {
            k: {f: v["roofline"][f] for f in ("achieved", "peak", "unit", "frac", "launch_us",
                                               "flops_per_launch")}
            for k, v in pre.items()}
    print(json.dumps(line))


def device_info():
    """The device's CU count and a measured device-to-device copy rate, beside the datasheet
    peak the rooflines use: 1 GiB copied 10 times after 3 warm-up copies, HIP events on the
    current stream, bytes counted as read + written."""
    import torch

    props = torch.cuda.get_device_properties(0)
    n = 2**28  # fp32 elements: 1 GiB
    x = torch.ones(n, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / 10
    del x, y
    torch.cuda.empty_cache()
    return {"name": props.name, "cus": props.multi_processor_count,
            "copy_GBps": round(2 * n * 4 / sec / 1e9, 1), "copy_bytes": n * 4}


def run_config(args, config, *, steps, warmup, with_cpu):
    """Build config `config`, time `steps` whole steps (after `warmup`) and each kernel, and
    return the JSON line's fields (None in --profile-kernels mode)."""
    import torch

    from flashqwen_amd import synth
    from flashqwen_amd.step import AttnStep, alloc_pool

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if config == 5:
        cfg = synth.config5(layers=args.layers or 36)
    else:
        cfg = synth.CONFIGS[config]()
    layers = cfg.layers
    scheduled = cfg.num_tokens is not None

    # ---- batch as the scheduler would hand it over ------------------------------------
    # Config 4 selects its batch on the GPU (fqa_schedule) from running state: buffers are
    # sized to the token budget, and the selection the GPU made is read back once, before
    # capture, to size grids and to count the algorithmic work.
    T = cfg.token_budget if scheduled else cfg.rows

    rng = np.random.default_rng(1234)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    qkv = t(synth.rand_bf16(rng, (T, synth.QKV_STRIDE)).view(np.int16)).view(torch.bfloat16)
    wq, wk = synth.norm_weights()
    wq_d, wk_d = t(wq), t(wk)
    pool = alloc_pool(cfg.pool_pages, layers, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    flat = pool.view(-1)
    for s in range(0, flat.numel(), 1 << 30):
        e = min(s + (1 << 30), flat.numel())
        flat[s:e].normal_(generator=g)
    out = torch.zeros((T, synth.N_Q * synth.HEAD_DIM), dtype=torch.bfloat16, device=dev)

    prefix_pages = args.dec_prefix_pages
    if prefix_pages is None:
        prefix_pages = 8 if config == 5 else 0

    def make_step(pp):
        return AttnStep(max_rows=T, max_reqs=cfg.n_reqs, max_ctx=cfg.max_ctx,
                        pool_pages=cfg.pool_pages, device=dev,
                        dec_grid_waves=args.dec_grid_waves, dec_min_pages=args.dec_min_pages,
                        pre_tile_q=args.pre_tile_q,
                        dec_share=not (args.no_overlap or args.no_dec_share),
                        dec_prefix_pages=pp)

    step = make_step(prefix_pages)
    d_computed, d_n_new = t(cfg.computed), t(cfg.n_new)
    d_off, d_pages = t(cfg.bt_off), t(cfg.bt_pages)
    d_ntok = t(cfg.num_tokens) if scheduled else None

    if scheduled:
        step.schedule_and_prepare(d_ntok, d_computed, d_off, d_pages, cfg.token_budget,
                                  cfg.prefill_chunk, rows_bound=T)
        torch.cuda.synchronize()
        ns = int(step.n_sel.cpu()[0])
        sel_req = step.sel_req[:ns].cpu().numpy()
        n_sel = step.sel_n[:ns].cpu().numpy()
        comp_sel = cfg.computed[sel_req]
        T = int(n_sel.sum())
    else:
        comp_sel, n_sel = cfg.computed, cfg.n_new
    has_decode = bool((n_sel == 1).any())
    has_prefill = bool((n_sel != 1).any())

    def pack():
        if scheduled:
            step.schedule_and_prepare(d_ntok, d_computed, d_off, d_pages, cfg.token_budget,
                                      cfg.prefill_chunk, rows_bound=T)
        else:
            step.prepare_inputs(d_computed, d_n_new, d_off, d_pages, rows_bound=T)

    side = None if args.no_overlap else torch.cuda.Stream(device=dev)

    def one_step():
        pack()
        for l in range(layers):
            step.run_layer(qkv, pool[l], wq_d, wk_d, out, decode=has_decode,
                           prefill=has_prefill, side_stream=side)

    # eager once (also validates the pack), then capture the step
    one_step()
    torch.cuda.synchronize()
    meta = step.meta_host()
    if meta[7] not in (0,):
        raise SystemExit(f"pack status {meta[7]}")
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        one_step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one_step()
    torch.cuda.synchronize()

    def kernel_graph(fn, reps):
        kg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(kg):
            for _ in range(reps):
                fn()
        return kg

    def time_graph(gr, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    reps = args.kernel_reps
    kernels = {"pack": pack,
               "qknorm_rope_append": lambda: step.head_norm_rope_store_kv(qkv, pool[0], wq_d,
                                                                          wk_d)}
    if args.compat_append:
        import ctypes as C

        from flashqwen_amd import _lib

        lib = _lib.load()

        def two_launch():
            s = step.stream
            _lib.check(lib.fqa_qknorm_rope(
                C.byref(step.dims), qkv.data_ptr(), wq_d.data_ptr(), wk_d.data_ptr(),
                step.cos.data_ptr(), step.sin.data_ptr(), step.max_ctx,
                step.positions.data_ptr(), step.meta.data_ptr(), step.rows_bound, s),
                "fqa_qknorm_rope")
            _lib.check(lib.fqa_store_kv(
                C.byref(step.dims), qkv.data_ptr(), step.positions.data_ptr(),
                step.slot_mapping.data_ptr(), step.meta.data_ptr(), step.rows_bound,
                pool[0].data_ptr(), cfg.pool_pages, s), "fqa_store_kv")
        kernels["compat_norm_then_store"] = two_launch
    if has_decode:
        kernels["decode"] = lambda: step.attn_decode(qkv, pool[0], out)
        # the same plan's pages read with the same loads and no arithmetic: the floor
        kernels["decode_read_floor"] = lambda: step.decode_read_floor(pool[0])
        if prefix_pages > 0 and not scheduled and not args.profile_kernels:
            # the same batch decoded without the shared-prefix groups (fqa_decode), for
            # comparison: its own plan, packed once before capture (not under the profiler,
            # whose per-kernel averages would mix the two plans' split kernels)
            plain = make_step(0)
            plain.prepare_inputs(d_computed, d_n_new, d_off, d_pages, rows_bound=T)
            out_plain = torch.zeros_like(out)
            kernels["decode_no_prefix"] = lambda: plain.attn_decode(qkv, pool[0], out_plain)
            kernels["decode_read_floor_no_prefix"] = lambda: plain.decode_read_floor(pool[0])
    if has_prefill:
        kernels["prefill"] = lambda: step.attn_prefill(qkv, pool[0], out)
    kgraphs = {k: kernel_graph(f, reps) for k, f in kernels.items()}
    torch.cuda.synchronize()
    if args.profile_kernels:
        # Clocks ramp up over the first tens of ms of sustained work: ten replays per
        # kernel keep the cold first one a small part of the profiler's average
        for k, kg in kgraphs.items():
            for _ in range(10):
                kg.replay()
        torch.cuda.synchronize()
        print(json.dumps({"profile_kernels": list(kgraphs)}))
        return None

    # ---- timed region: K whole steps -----------------------------------------------------
    # The GPU clock ramps over the first tens of milliseconds of sustained work, so steps
    # much shorter than that (configs 1-4) get more warmup: at least `warmup` steps and
    # ~50 ms in all.  The line reports the number of warmup steps run.
    warm_ms = time_graph(graph, warmup) if warmup > 0 else 0.0
    extra = max(0, math.ceil(50.0 / max(warm_ms, 1e-3)) - warmup) if warmup > 0 else 0
    for _ in range(extra):
        graph.replay()
    torch.cuda.synchronize()
    warmup += extra
    t0 = time.perf_counter()
    ms_events = time_graph(graph, steps)
    wall = time.perf_counter() - t0
    ms_step = ms_events

    kern_ms = {}
    for k, kg in kgraphs.items():
        kg.replay()
        torch.cuda.synchronize()
        kern_ms[k] = time_graph(kg, 5) / reps

    # ---- roofline of the dominant kernel ---------------------------------------------------
    meta = step.meta_host()
    if has_decode and (not has_prefill or config == 5):
        logical, unique = synth.decode_bytes(_selected(cfg, comp_sel, n_sel))
        bt_bytes = int(meta[9]) * 4
        bytes_per = logical + bt_bytes
        achieved = bytes_per / (kern_ms["decode"] * 1e-3) / 1e9
        dec_kernels = ["decode_split_kernel", "decode_combine_kernel"]
        name = "fqa_decode (decode_split_kernel + decode_combine_kernel)"
        if prefix_pages > 0:
            name = ("fqa_decode_prefix (decode_split_kernel, its workgroups past the "
                    "shares running the prefix items, + decode_combine_kernel)")
        traffic, tsrc = _profile_traffic(config, dec_kernels)
        roof = {"kernel": name,
                "bound": "hbm",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": tsrc,
                "bytes_per_launch": bytes_per, "unique_kv_bytes": unique,
                "launch_us": round(kern_ms["decode"] * 1e3, 2),
                "read_floor_us": round(kern_ms["decode_read_floor"] * 1e3, 2),
                "frac_of_read_floor": round(kern_ms["decode_read_floor"] / kern_ms["decode"], 4)}
        if prefix_pages > 0:
            # achieved counts a shared prefix's bytes once per reading sequence (the metric's
            # definition); the plan reads each group's prefix once per 8 members, so the
            # bytes the plan reads and their rate are stated beside it
            items = step.dec_pre_items[:int(meta[10])].cpu().numpy()
            item_runs = int((items[:, 3] - items[:, 2]).sum()) if len(items) else 0
            run_bytes = synth.PAGE_BYTES // synth.N_KV
            n_dec = int(meta[1])
            plan_bytes = ((int(meta[9]) * synth.N_KV + item_runs) * run_bytes + bt_bytes +
                          n_dec * 2 * synth.N_Q * synth.HEAD_DIM * 2)
            roof["plan_read_bytes"] = plan_bytes
            roof["plan_read_GBps"] = round(plan_bytes / (kern_ms["decode"] * 1e-3) / 1e9, 1)
            roof["prefix_groups"] = int(meta[11])
            roof["prefix_items"] = int(meta[10])
            if "decode_no_prefix" in kern_ms:
                roof["no_prefix_launch_us"] = round(kern_ms["decode_no_prefix"] * 1e3, 2)
                roof["no_prefix_frac"] = round(
                    bytes_per / (kern_ms["decode_no_prefix"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    else:
        flops = synth.prefill_flops(comp_sel, n_sel)
        achieved = flops / (kern_ms["prefill"] * 1e-3) / 1e12
        traffic, tsrc = _profile_traffic(config, ["prefill_kernel"])
        roof = {"kernel": "fqa_prefill (prefill_kernel)", "bound": "mfma",
                "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                "traffic_source": tsrc,
                "flops_per_launch": flops, "launch_us": round(kern_ms["prefill"] * 1e3, 2),
                "counters": _profile_mfma_util(config)}
        if has_decode:
            logical, _ = synth.decode_bytes(_selected(cfg, comp_sel, n_sel))
            # the decode alone on the step's plan (with dec_share: the waves it gets beside
            # the prefill, so less than the whole device)
            roof["decode_GBps_alone"] = round(logical / (kern_ms["decode"] * 1e-3) / 1e9, 1)
            roof["decode_waves"] = int(meta[4])

    # ---- CPU baseline (OpenMP fp32 oracle, bounded sample) ------------------------------
    cpu = None
    if with_cpu:
        cpu = cpu_baseline(cfg, comp_sel, n_sel, T, args.cpu_seconds)

    # the step's floor: its kernels back to back at their isolated durations, the decode at
    # its read floor (the same pages read with no arithmetic); the rest of the step time is
    # launch gaps and what the kernels lose to each other.  A mixed step whose decode runs
    # beside the prefill (dec_share) can end below it: the two kernels overlap.
    floor_us = (kern_ms["pack"] + layers * (kern_ms["qknorm_rope_append"] +
                                            kern_ms.get("decode_read_floor", 0.0) +
                                            kern_ms.get("prefill", 0.0))) * 1e3
    tokens_per_step = T
    value = tokens_per_step / (ms_step * 1e-3)
    line = {
        "metric": "attn-step tokens/s",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/k/v and pool, seeded page placement)",
        "config": {"workload": f"config{config}: {_describe(config)}",
                   "rows_per_step": T, "requests": int(len(n_sel)), "layers": layers,
                   "pool_pages_per_layer": cfg.pool_pages, "head_shape": "32q/8kv/128",
                   "dec_wave_cost": int(meta[6]), "dec_waves": int(meta[4]),
                   "pre_items": int(meta[5]), "dec_prefix_pages": prefix_pages},
        "roofline": roof,
        "kernels_us": {k: round(v * 1e3, 2) for k, v in kern_ms.items()},
        "step_floor_us": round(floor_us, 2),
        "step_minus_floor_us": round(ms_step * 1e3 - floor_us, 2),
        "decode_beside_prefill": bool(side is not None and has_decode and has_prefill),
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    return line



def bench_sampler(args):
    """fqa_sample on 256 rows of 151936 fp32 logits (one sampling row per request of a
    256-sequence decode step): greedy, temperature 1, temperature 1 + top-p 0.9.  The
    roofline is HBM: one read of the logits (B*N*4 bytes) per launch; the kernel reads a
    row once for greedy and temperature-only sampling, 4 times with top-p."""
    import torch

    from flashqwen_amd.sample import sample

    B, N = 256, 151936
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    logits = torch.randn(B, N, device="cuda", generator=g) * 3
    u = torch.rand(B, device="cuda", generator=g)
    out = torch.empty(B, dtype=torch.int32, device="cuda")
    res = {}
    for name, it, tp in (("greedy", 0.0, 1.0), ("temperature", 1.0, 1.0),
                         ("top_p_0.9", 1.0, 0.9)):
        itv = torch.full((B,), it, device="cuda")
        tpv = torch.full((B,), tp, device="cuda")
        for _ in range(5):
            sample(logits, itv, tpv, u, out)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(20):
                sample(logits, itv, tpv, u, out)
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 200
        res[name] = {"us": round(us, 2), "rows_per_s": round(B / (us * 1e-6), 1),
                     "logit_GBps": round(B * N * 4 / (us * 1e-6) / 1e9, 1)}
    print(json.dumps({"sampler": res, "rows": B, "vocab": N, "peak_GBps": HBM_PEAK_GBS}))


GEMM_SHAPES = {"qkv": (6144, 4096), "o_proj": (4096, 4096), "gate_up": (24576, 4096),
               "down": (4096, 12288), "lm_head": (151936, 4096)}


def bench_gemm(args):
    """fqa_gemm on the Qwen3-8B projections (N, K) at several row counts M, beside
    torch.matmul (hipBLASLt) on the same tensors.  Algorithmic work: 2MNK FLOP; bytes
    (M K + N K + M N) * 2 (fp32 logits for lm_head).  lm_head only at M <= 256 (sampling
    rows).  Each timing replays a graph of 20 calls 10 times."""
    import torch

    from flashqwen_amd.gemm import gemm

    def timed(fn):
        for _ in range(3):
            fn()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(20):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / 200

    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    rows = [int(v) for v in args.gemm_rows.split(",")]
    out = {}
    for name, (N, K) in GEMM_SHAPES.items():
        w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        f32 = name == "lm_head"
        for M in rows:
            if f32 and M > 256:
                continue
            x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
            y = torch.empty(M, N, device="cuda", dtype=torch.float32 if f32 else torch.bfloat16)
            us = timed(lambda: gemm(x, w, out=y, out_f32=f32))
            if f32:
                # hipBLASLt has no bf16 x bf16 -> fp32 path in torch.matmul: bf16 + cast
                ut = timed(lambda: torch.matmul(x, w.t()).float())
            else:
                yt = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
                ut = timed(lambda: torch.matmul(x, w.t(), out=yt))
            fl = 2.0 * M * N * K
            by = (M * K + N * K) * 2 + M * N * (4 if f32 else 2)
            out[f"{name}_M{M}"] = {
                "us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                "GBps": round(by / us / 1e3, 1), "torch_us": round(ut, 2),
                "speedup": round(ut / us, 2)}
            print(name, M, out[f"{name}_M{M}"], flush=True)
            del x, y
        del w
    # the QKV projection with the norm/RoPE/append fused (fqa_qkv_proj_append) against
    # fqa_gemm + fqa_qknorm_rope_append: up to 256 rows one decode row per sequence on its
    # own page, above that 512-token prompts on full pages
    import ctypes as C

    from flashqwen_amd import _lib
    from flashqwen_amd.gemm import workspace_bytes
    from flashqwen_amd.step import alloc_pool, make_dims, rope_tables

    lib = _lib.load()
    dims = make_dims()
    N, K = GEMM_SHAPES["qkv"]
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    qn = torch.ones(128, device="cuda")
    cos, sin = (torch.from_numpy(t).cuda() for t in rope_tables(4096))
    for M in rows:
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        qkv = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        pool = alloc_pool(M + 16)[0]
        if M <= 256:  # decode rows: one row per sequence, each on its own page
            pos = torch.arange(M, dtype=torch.int32, device="cuda") + 1000
            slots = torch.arange(M, dtype=torch.int32, device="cuda") * 16 + 7
        else:  # prefill rows: 512-token prompts on scattered full pages
            r = torch.arange(M, dtype=torch.int32, device="cuda")
            pos = r % 512
            pages = torch.randperm(M + 16, generator=g, device="cuda")[: (M + 15) // 16]
            slots = (pages[r // 16] * 16 + r % 16).to(torch.int32)
        meta = torch.zeros(16, dtype=torch.int32, device="cuda")
        meta[_lib.META_ROWS] = M
        nb = workspace_bytes(M, N, K)
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")

        def unfused():
            gemm(x, w, out=qkv, workspace=ws)
            lib.fqa_qknorm_rope_append(C.byref(dims), qkv.data_ptr(), qn.data_ptr(), qn.data_ptr(),
                                       cos.data_ptr(), sin.data_ptr(), 4096, pos.data_ptr(),
                                       slots.data_ptr(), meta.data_ptr(), M, pool.data_ptr(),
                                       M + 16, 0, torch.cuda.current_stream().cuda_stream)

        def fused():
            lib.fqa_qkv_proj_append(C.byref(dims), x.data_ptr(), K, w.data_ptr(), K, M, K,
                                    qkv.data_ptr(), qn.data_ptr(), qn.data_ptr(), cos.data_ptr(),
                                    sin.data_ptr(), 4096, pos.data_ptr(), slots.data_ptr(),
                                    meta.data_ptr(), pool.data_ptr(), M + 16, 0,
                                    ws.data_ptr() if nb else None, nb,
                                    torch.cuda.current_stream().cuda_stream)

        uf, fu = timed(unfused), timed(fused)
        out[f"qkv_append_M{M}"] = {"fused_us": round(fu, 2), "unfused_us": round(uf, 2)}
        print("qkv+append", M, out[f"qkv_append_M{M}"], flush=True)
    # lm_head + greedy pick: fused (no logits written) against fqa_gemm (fp32) + fqa_sample
    from flashqwen_amd.gemm import gemm_argmax
    from flashqwen_amd.sample import sample

    N, K = GEMM_SHAPES["lm_head"]
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    for M in [r for r in rows if r <= 256]:
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        logits = torch.empty(M, N, device="cuda", dtype=torch.float32)
        zero = torch.zeros(M, device="cuda")
        one = torch.ones(M, device="cuda")
        tok = torch.empty(M, dtype=torch.int32, device="cuda")
        fu = timed(lambda: gemm_argmax(x, w, out=tok))
        uf = timed(lambda: sample(gemm(x, w, out=logits, out_f32=True), zero, one, zero, tok))
        out[f"lm_head_greedy_M{M}"] = {"fused_us": round(fu, 2), "unfused_us": round(uf, 2)}
        print("lm_head+greedy", M, out[f"lm_head_greedy_M{M}"], flush=True)
    print(json.dumps({"gemm": out, "peak_TFLOPs": 2516.6, "peak_GBps": HBM_PEAK_GBS}))


def _profile_traffic(config: int, kernels: list[str]):
    """HBM bytes per launch of `kernels` (summed) from the committed rocprofv3 summary of
    this config (profiles/*_config<N>.txt, calibrated FETCH_SIZE + WRITE_SIZE), or None."""
    prof = Path(__file__).resolve().parent / "profiles"
    for f in sorted(prof.glob(f"*_config{config}.txt")):
        got = {}
        for line in f.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes":
                got[parts[1]] = int(parts[2])
        if all(k in got for k in kernels):
            return sum(got[k] for k in kernels), f"profiles/{f.name}"
    return None, None


def _profile_mfma_util(config: int):
    """The prefill kernel's MFMA busy fraction of the active cycles, and the clock while it
    ran, from the committed rocprofv3 counter summary of this config (or None)."""
    prof = Path(__file__).resolve().parent / "profiles"
    for f in sorted(prof.glob(f"*_config{config}.txt")):
        util = clock = None
        for line in f.read_text().splitlines():
            if "MfmaUtil" in line and "=" in line:
                util = float(line.rsplit("=", 1)[1].strip().rstrip("%")) / 100
            if "clock while the kernel ran" in line:
                clock = float(line.rsplit("=", 1)[1].split()[0])
        if util is not None:
            return {"mfma_busy_of_active_cycles": util, "clock_ghz_under_load": clock,
                    "source": f"profiles/{f.name}"}
    return None


def _selected(cfg, comp_sel, n_sel):
    """A StepConfig view of the batch actually run (config 4 is selected on the GPU)."""
    from flashqwen_amd import synth

    if cfg.num_tokens is None:
        return cfg
    return synth.StepConfig(cfg.name, comp_sel, n_sel, np.zeros(len(n_sel) + 1, np.int32),
                            np.zeros(0, np.int32), cfg.pool_pages, cfg.max_ctx)


def _describe(n):
    return {1: "4 decode seqs, L in {17,100,255,512}",
            2: "64 decode seqs, L~U[512,4096], 1 layer, pool 200k tokens",
            3: "16 log-normal prompts (median 400) within 8192 tokens, causal varlen prefill",
            4: "mixed 8192-token budget: 2x2048 chunks on 3000 prefixes + 512/700/900 fresh + "
               "256 decodes, selection on GPU",
            5: "36 layers, 32x32768 + 96 shared-prefix decodes, ~200 GB pool"}[n]


def cpu_baseline(cfg, comp_sel, n_sel, T, seconds):
    """The OpenMP fp32 oracle on the same step: (selection for a scheduled config) + pack +
    norm/rope/append + decode + prefill, one layer, repeated for about `seconds` (at least 3
    repetitions); tokens/s = rows / (time per step x layers).  Only the oracle's C calls
    are timed: the q/k/v rows the append normalises in place are restored from a pristine
    copy between repetitions outside the timer, and the pool is copied once, before the
    first repetition (the append rewrites the same slots with the same values each time)."""
    from flashqwen_amd import synth
    from oracle import oracle as orc
    from tests import stepcase as sc

    sub = cfg
    scheduled = cfg.num_tokens is not None
    if scheduled:
        sel_req, _ = orc.schedule(cfg.num_tokens, cfg.computed, cfg.token_budget,
                                  cfg.prefill_chunk)
        tabs = cfg.tables()
        sub = synth._assemble(cfg.name, comp_sel, n_sel, [tabs[i] for i in sel_req],
                              cfg.pool_pages, cfg.max_ctx)
    # the pages the step reads, renumbered into a compact pool (shared pages stay shared):
    # the oracle's time does not depend on where in the pool a page sits
    sample = "full step, one layer"
    keep = list(range(len(sub.computed)))
    if cfg.name == "config5":
        # a sample of 8 long and 24 shared-prefix sequences
        keep = list(range(8)) + list(range(32, 56))
        sample = "8 of 32 long + 24 of 96 shared-prefix seqs, 1 layer"
    sub = _compact(sub, keep)
    rng = np.random.default_rng(5)
    kw = sc.pack_kwargs(sub)
    qkv0 = synth.rand_bf16(rng, (sub.rows, synth.QKV_STRIDE))
    # the pool: a 4M-value N(0,1) bf16 block tiled over the pages (the oracle's time does not
    # depend on the values; drawing ~1e9 normals would take minutes)
    block = synth.rand_bf16(rng, 1 << 22)
    pool = np.resize(block, sc.pool_elems(sub.pool_pages))
    wq, wk = synth.norm_weights()
    cos, sin = orc.rope_tables(sub.max_ctx)
    parts = {k: [] for k in (["schedule"] if scheduled else []) +
             ["pack", "qknorm_rope_append", "decode", "prefill"]}
    totals = []
    t_end = time.perf_counter() + seconds
    while True:
        q = qkv0.copy()  # untimed restore
        out = np.zeros((max(sub.rows, 1), synth.N_Q * synth.HEAD_DIM), np.uint16)
        tot = 0.0
        if scheduled:
            t0 = time.perf_counter()
            orc.schedule(cfg.num_tokens, cfg.computed, cfg.token_budget, cfg.prefill_chunk)
            dt = time.perf_counter() - t0
            parts["schedule"].append(dt)
            tot += dt
        t0 = time.perf_counter()
        pk = orc.pack(sub.computed, sub.n_new, sub.bt_off, sub.bt_pages, **kw)
        dt = time.perf_counter() - t0
        parts["pack"].append(dt)
        tot += dt
        Tn = int(pk["meta"][0])
        t0 = time.perf_counter()
        orc.qknorm_rope_append(q, wq, wk, cos, sin, pk["positions"], pk["slot_mapping"], Tn,
                               pool, sub.pool_pages)
        dt = time.perf_counter() - t0
        parts["qknorm_rope_append"].append(dt)
        tot += dt
        t0 = time.perf_counter()
        orc.decode(q, pool, sub.pool_pages, pk["block_tables"], kw["max_blocks"],
                   pk["cu_seqlens"], pk["positions"], pk["decode_rids"], int(pk["meta"][1]), out)
        dt = time.perf_counter() - t0
        parts["decode"].append(dt)
        tot += dt
        t0 = time.perf_counter()
        orc.prefill(q, pool, sub.pool_pages, pk["block_tables"], kw["max_blocks"],
                    pk["cu_seqlens"], pk["positions"], pk["prefill_rids"], int(pk["meta"][2]),
                    out)
        dt = time.perf_counter() - t0
        parts["prefill"].append(dt)
        tot += dt
        totals.append(tot)
        if (time.perf_counter() > t_end and len(totals) >= 3) or len(totals) >= 50:
            break
    per = float(np.median(totals))
    rows = sub.rows
    value = rows / (per * cfg.layers)
    if cfg.layers > 1:
        sample += f"; x{cfg.layers} layers extrapolated"
    return {"value": round(value, 2), "unit": "tokens/s", "cores": orc.num_threads(),
            "kind": "port",
            "sample": f"{sample}; {len(totals)} reps, median {per * 1e3:.1f} ms of oracle C "
                      "calls only (input restores and copies outside the timer)",
            "parts_ms": {k: round(float(np.median(v)) * 1e3, 3) for k, v in parts.items()},
            "nproc": os.cpu_count()}


def _compact(cfg, keep):
    """The requests `keep` of a step with their pages (the new tokens' pages included)
    renumbered into a small pool; pages shared between requests stay shared."""
    from flashqwen_amd import synth

    all_tabs = cfg.tables()
    tabs = [all_tabs[i] for i in keep]
    uniq = {p: i for i, p in enumerate(dict.fromkeys(np.concatenate(tabs).tolist()))}
    new = [np.array([uniq[p] for p in tb], np.int32) for tb in tabs]
    return synth._assemble(cfg.name, cfg.computed[keep], cfg.n_new[keep], new, max(len(uniq), 1),
                           cfg.max_ctx, layers=cfg.layers)


if __name__ == "__main__":
    main()
