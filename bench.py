#!/usr/bin/env python3
"""Benchmark of the BD3LM denoise step on one MI355X.

Workload (one GPU): BD3LM on the Qwen3-0.6B architecture with q4 affine g64
weights (seed 4), an 8192-token random prefix already committed to the K/V
cache, then blocks of 32 masked tokens, 8 denoise steps per block, 4 tokens
unmasked per step (greedy max-probability). A *step* is one denoise step: the
forward of the active block over the cached prefix, the fused LM head with the
frontier's float64 scoring, and the step's fixed-quota choice and commit, all
on the device through the library's native loop (``--host-loop``: the choice
on the host through propose / commit). A finished block's K/V-writing forward
runs merged into the next block's first step and is counted there.

Prints one JSON line. ``value`` is generated tokens/s over the timed steps,
which replay the captured HIP graphs of the step and block-commit forwards.
``roofline`` is the dominant kernel (the block-over-prefix decode attention,
``attn_decode_kernel``): its dispatches are timed one by one with HIP events
(hipExtLaunchKernelGGL start/stop events on the launch stream) over a second
timed region of the same number of steps run eagerly, since a graph replay
cannot carry per-dispatch events; ``roofline.op`` is the same over the kernel
and its range combine. ``cpu_baseline`` times the oracle's
reference-semantics CPU path (full prefix recompute) on a bounded sample.

``--calibrate-copy`` instead times a plain device copy of a known size (the
scale for rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and prints its line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "generated tokens/sec + ms/denoise step on 1 MI355X; % HBM roofline"
HBM_PEAK_GBS = 8000.0
PREFIX = 8192
BLOCK = 32
STEPS_PER_BLOCK = 8
SEED = 4


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed denoise steps")
    ap.add_argument("--warmup", type=int, default=8, help="untimed denoise steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-loop", action="store_true",
                    help="drive the step loop from Python (propose/commit per step) instead of "
                         "the library's native loop")
    ap.add_argument("--cpu-sample-layers", type=int, default=1)
    ap.add_argument("--profile-steps", type=int, default=None,
                    help="eager steps timed per dispatch for the roofline (default: --steps; 0 = none)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="time a 256 MiB device-to-device copy and exit")
    ap.add_argument("--workload", default="bd3_q4_8k",
                    choices=["bd3_q4_8k", "bd3_bf16", "dream_q4", "dream_q4_threshold",
                             "attention", "q4_linear"],
                    help="bd3_q4_8k is the headline line; the others print one JSON line per "
                         "case of the remaining configurations")
    return ap.parse_args()


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def cpu_baseline(model, prefix_ids, mask_id, layers_sampled: int):
    """Reference-semantics CPU step (oracle), bounded sample.

    The reference recomputes the whole visible prefix every denoise step
    (S = prefix + block rows through all layers). The sample times the
    embedding, ``layers_sampled`` decoder layers and the final norm + LM head on
    the 32 frontier rows at S = 8224, and scales the layer time to all layers."""
    import numpy as np

    from diffusorrt_amd import synthetic as syn
    from oracle import forward as F
    from oracle import ops as O

    g = model.geometry
    W = {}
    for k, v in syn.to_oracle_weights(model).items():
        W[k] = O.Q4Weight(*v) if isinstance(v, tuple) else v
    cfg = syn.oracle_config(g, "q4")
    ids = np.asarray(list(prefix_ids) + [mask_id] * BLOCK)
    s = len(ids)
    # weight dequantization is load-time work: do it before the clock starts
    for i in range(layers_sampled):
        for suf in syn.LINEAR_SUFFIXES:
            W[f"model.layers.{i}.{suf}.weight"].dense()
    W["lm_head.weight"].dense()
    t0 = time.perf_counter()
    hidden = np.asarray(W["model.embed_tokens.weight"][ids], dtype=np.float32)
    cos, sin = O.rope_tables(np.arange(s), g.head_dim, g.rope_theta)
    visible = O.d2f_visible(np.arange(s), s, prompt_len=0, block_size=BLOCK)
    t1 = time.perf_counter()
    for i in range(layers_sampled):
        hidden = F.layer_forward(W, cfg, i, hidden, cos, sin, visible)
    t2 = time.perf_counter()
    rows = list(range(PREFIX, PREFIX + BLOCK))
    h = O.rms_norm(hidden[rows], W["model.norm.weight"], g.rms_norm_eps)
    logits = O.linear(h, W["lm_head.weight"], None, weight_kind="q4")
    O.raw_max_prob(logits)
    t3 = time.perf_counter()
    per_layer = (t2 - t1) / layers_sampled
    step_s = (t1 - t0) + per_layer * g.layer_count + (t3 - t2)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.environ.get("OPENBLAS_NUM_THREADS",
                                                                      os.cpu_count() or 1)))
    return {
        "value": round(4.0 / step_s, 4),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "ms_per_step": round(step_s * 1e3, 1),
        "sample": (f"oracle (numpy fp32, reference semantics: full recompute of S={s} rows) "
                   f"timed for embedding + {layers_sampled} of {g.layer_count} decoder layers + "
                   f"final norm/LM head/float64 scoring of 32 rows; layer time scaled x"
                   f"{g.layer_count / layers_sampled:g}; 4 tokens per step"),
    }


def calibrate_copy(steps: int) -> None:
    """A plain copy kernel of known size: 256 MiB read + 256 MiB written."""
    import torch

    n = 256 << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": steps,
                      "ms_per_copy": round(dt * 1e3, 4),
                      "GBps_read_plus_write": round(2 * n / dt / 1e9, 1)}), flush=True)


def read_traffic():
    """HBM bytes per decode-attention dispatch measured with rocprofv3 counters
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading for the
    plain copy), recorded as ``traffic_bytes_per_launch = N`` in the profile
    summary; None when that file is absent."""
    path = os.path.join(ROOT, "profiles", "attn_decode_kernel_bd3_q4_8k_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch ="):
                    return float(line.split("=", 1)[1].strip().split()[0])
    except OSError:
        return None
    return None


def _event_time_us(fn, reps: int) -> float:
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3


def _graph_time_us(fn, reps: int) -> float:
    """Per-call device time of `reps` calls captured in one HIP graph and replayed
    (no host work between the calls: what a graph-capturing caller sees)."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (5 * reps) * 1e3


def bench_attention() -> None:
    """Isolated block-over-prefix attention: 32 query rows x 16 heads x 128, bf16,
    K/V of L prefix + 32 block keys x 8 heads, N(0, 1) from seed 1, prefix fully
    visible and the block bidirectional; fp32 accumulate, bf16 output. Timed per
    call (Q planes, decode attention, range combine) on the torch stream: 50 calls
    captured in a HIP graph and replayed, and 50 eager calls."""
    import ctypes as C

    import torch

    from diffusorrt_amd import _lib, kernels

    lib = _lib.load()
    rows, hq, hkv = 32, 16, 8
    gen = torch.Generator().manual_seed(1)
    for L in (512, 2048, 8192):
        n = L + 32
        cache = kernels.PrefixKVCache(1, hkv, n, dtype="bf16")
        k = torch.randn((n, hkv, 128), generator=gen).bfloat16().cuda()
        v = torch.randn((n, hkv, 128), generator=gen).bfloat16().cuda()
        cache.store(0, k, v, 0)
        q = torch.randn((rows, hq, 128), generator=gen).bfloat16().cuda()
        out = torch.empty((rows, hq * 128), dtype=torch.bfloat16, device="cuda")
        ws_b = lib.drt_op_attention_workspace_bytes(rows, hq, hkv, n)
        ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
        def run():
            st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(lib.drt_op_attention(
                C.c_void_p(q.data_ptr()), C.c_void_p(cache.data.data_ptr()), cache.head_stride,
                _lib.BF16, rows, hq, hkv, n, L, 0, 0, 1, C.c_void_p(out.data_ptr()), _lib.BF16,
                C.c_void_p(ws.data_ptr()), ws_b, st))

        us_eager = _event_time_us(run, 50)
        us = _graph_time_us(run, 50)
        byts = 4.0 * rows * hq * 128 + 4096.0 * n
        print(json.dumps({"workload": "attention", "prefix": L, "rows": rows, "heads": [hq, hkv],
                          "dtype": "bf16", "us_per_call": round(us, 2),
                          "timed": "50 calls in a HIP graph",
                          "us_per_call_eager": round(us_eager, 2),
                          "algorithmic_bytes": byts,
                          "achieved_GBps": round(byts / us / 1e3, 1),
                          "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)


def bench_q4_linear() -> None:
    """Isolated q4 g64 linear (MLX packing): nibbles U{0..15}, scales U(0.005, 0.02),
    biases U(-0.1, 0.1) (bf16), x bf16 N(0, 1), seed 2. Timed per call on the
    per-op entry point: 30 calls captured in a HIP graph and replayed (device
    time per call), and 30 eager calls (host launch rate included)."""
    import ctypes as C

    import torch

    from diffusorrt_amd import _lib, kernels
    from diffusorrt_amd import synthetic as syn

    lib = _lib.load()
    gen = torch.Generator().manual_seed(2)
    for (N, K) in ((1024, 1024), (3072, 1024), (1024, 3072), (18944, 3584), (3584, 18944)):
        qt = syn.random_q4(gen, N, K, scale_lo=0.005, scale_hi=0.02, centred=False,
                           bias_lo=-0.1, bias_hi=0.1)
        w = kernels.DeviceQ4Weight(qt.w_q.cuda(), qt.scales.cuda(), qt.biases.cuda())
        for M in (32, 128):
            x = torch.randn((M, K), generator=gen).bfloat16().cuda()
            us_eager = _event_time_us(lambda: kernels.linear(x, w), 30)
            us = _graph_time_us(lambda: kernels.linear(x, w), 30)
            byts = N * K / 2 + N * K / 16 + 2.0 * M * K + 4.0 * M * N
            flops = 2.0 * M * N * K
            print(json.dumps({"workload": "q4_linear", "M": M, "N": N, "K": K,
                              "us_per_call": round(us, 2), "timed": "30 calls in a HIP graph",
                              "us_per_call_eager": round(us_eager, 2),
                              "algorithmic_bytes": byts,
                              "achieved_GBps": round(byts / us / 1e3, 1),
                              "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4),
                              "achieved_TFLOPs": round(flops / us / 1e6, 2),
                              "mfma_frac_fp16": round(flops / us / 1e6 / 2500.0, 4)}), flush=True)


def bench_decode_config(args, which: str) -> None:
    """Whole-decode configurations: `bd3_bf16` (Qwen3-0.6B BD3, bf16 N(0, 0.02) seed 0,
    64-token prompt, 4 blocks x 32 masks, 32 steps = 8 rounds of 4 per block) and
    `dream_q4` (Qwen2.5-7B Dream, q4 seed 3, 256-token prompt + 256 masks, 64
    steps of 4, bidirectional full canvas). One untimed decode, then one timed."""
    import torch

    from diffusorrt_amd import decode
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import (Runtime, bd3_session_config, block_threshold_session_config,
                                        fixed_quota_session_config)

    if which == "bd3_bf16":
        g, kind, seed, prompt_len, gen_len, steps, block = syn.BD3_QWEN3_06B, "bf16", 0, 64, 128, 32, 32
    elif which == "dream_q4_threshold":
        # Dream's own policy: 8-token blocks over the exact prompt + frozen-block
        # K/V, threshold 0.9 (random weights never reach it: one token per step)
        g, kind, seed, prompt_len, gen_len, steps, block = syn.DREAM_QWEN25_7B, "q4", 3, 256, 64, 512, 8
    else:
        g, kind, seed, prompt_len, gen_len, steps, block = syn.DREAM_QWEN25_7B, "q4", 3, 256, 256, 64, 256
    t = time.perf_counter()
    model = syn.build_model(g, kind, seed=seed)
    prompt = syn.prompt_ids(seed, prompt_len)
    log(f"{which}: model generated in {time.perf_counter() - t:.1f}s")
    rt = Runtime(model, max_forward_rows=max(512, prompt_len + gen_len),
                 max_positions=prompt_len + gen_len + 64)
    strategy = {"bd3_bf16": "bd3_fixed_quota", "dream_q4": "fixed_quota",
                "dream_q4_threshold": "block_threshold"}[which]
    make = {"bd3_fixed_quota": bd3_session_config, "fixed_quota": fixed_quota_session_config,
            "block_threshold": block_threshold_session_config}[strategy]
    cfg = make(block, steps, prompt_len + gen_len)

    def run():
        with rt.session(cfg) as s:
            return decode.generate_device_tokens(
                s, prompt, max_tokens=gen_len, mask_token_id=g.mask_token_id,
                eos_token_id=g.eos_token_id, steps=steps, block_size=block,
                decode_strategy=strategy)

    run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    res = run()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out = {"workload": which, "tokens_per_s": round(res.committed_token_count / dt, 2),
           "ms_per_step": round(dt / max(1, res.forward_count) * 1e3, 4),
           "forwards": res.forward_count, "committed_tokens": res.committed_token_count,
           "hit_eos": res.hit_eos, "weights": kind}
    if which == "dream_q4":
        params = g.layer_count * sum(n * k for n, k in syn.linear_shapes(g).values())
        flops = 2.0 * (prompt_len + gen_len) * params
        out["mfma_frac_fp16_linears"] = round(flops / (dt / res.forward_count) / 2.5e15, 4)
    print(json.dumps(out), flush=True)
    rt.close()


def main():
    args = parse_args()
    if args.calibrate_copy:
        calibrate_copy(max(1, args.steps))
        return
    if args.workload != "bd3_q4_8k":
        if args.workload == "attention":
            bench_attention()
        elif args.workload == "q4_linear":
            bench_q4_linear()
        else:
            bench_decode_config(args, args.workload)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path (the step is measured on one GPU's share of the work).",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from diffusorrt_amd import decode
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import Runtime, bd3_session_config

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    g = syn.BD3_QWEN3_06B
    prof_steps = args.steps if args.profile_steps is None else args.profile_steps
    total = args.warmup + args.steps + prof_steps
    n_blocks = max(1, math.ceil(total / STEPS_PER_BLOCK))
    max_tokens = n_blocks * BLOCK
    steps_budget = n_blocks * STEPS_PER_BLOCK
    t = time.perf_counter()
    model = syn.build_model(g, "q4", seed=SEED)
    prefix = syn.prompt_ids(SEED, PREFIX)
    log(f"model generated in {time.perf_counter() - t:.1f}s; {n_blocks} blocks")
    rt = Runtime(model, max_forward_rows=2048, max_positions=PREFIX + max_tokens + 64)
    sess = rt.session(bd3_session_config(BLOCK, steps_budget, PREFIX + max_tokens))
    state = decode.MaskState(x=list(prefix) + [g.mask_token_id] * max_tokens, prompt_len=PREFIX,
                             mask_token_id=g.mask_token_id, eos_token_id=g.eos_token_id)
    policy = decode.QuotaSchedule(prompt_len=PREFIX, generated=max_tokens, block_size=BLOCK,
                                  steps=steps_budget, absolute=True)
    sess.start_device(state.x, prompt_len=0, block_size=BLOCK, mask_token_id=g.mask_token_id,
                      exact_kv=False, steps=steps_budget)
    step_iter = iter(range(policy.iteration_limit))

    def native_steps(k: int) -> int:
        """k steps of the library's own loop in one call (as the product runs it)."""
        fwd, com, _done = sess.bd3_decode(prompt_len=PREFIX, max_tokens=max_tokens,
                                          steps=steps_budget, eos_token_id=g.eos_token_id,
                                          max_forwards=k)
        if fwd != k:
            raise RuntimeError("decode stopped early (EOS at a block boundary)")
        return com

    def one_step() -> int:
        if not args.host_loop:
            return native_steps(1)
        for step in step_iter:
            plan = policy.plan(state=state, step=step)
            if plan.stop:
                raise RuntimeError("decode stopped early (EOS at a block boundary)")
            if plan.skip:
                continue
            frozen = (min(plan.frontier) // BLOCK) * BLOCK
            scores, toks, _ = sess.propose_device(plan.frontier, window_end=plan.window_end,
                                                  frozen_prefix=frozen)
            chosen = policy.select(scores=scores, step=step)
            pos = [plan.frontier[r] for r in chosen]
            tk = [toks[r] for r in chosen]
            sess.commit_device(pos, tk)
            for p, tok in zip(pos, tk):
                state.commit(position=p, token_id=tok)
            return len(chosen)
        raise RuntimeError("ran out of scheduled steps")

    t = time.perf_counter()
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    log(f"warmup ({args.warmup} steps, incl. the {PREFIX}-row prefix commit) "
        f"{time.perf_counter() - t:.2f}s")
    m0 = sess.device_metrics()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    committed = 0
    if args.host_loop:
        for _ in range(args.steps):
            committed += one_step()
    else:
        committed = native_steps(args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    m1 = sess.device_metrics()
    log(f"timed {args.steps} steps (graph replay) {elapsed * 1e3:.1f} ms")
    if prof_steps > 0:
        # per-dispatch events force eager launches (no graph replay)
        sess.set_profiling(True)
        torch.cuda.synchronize()
        tp = time.perf_counter()
        for _ in range(prof_steps):
            one_step()
        torch.cuda.synchronize()
        prof_elapsed = time.perf_counter() - tp
        mp = sess.device_metrics()
        sess.set_profiling(False)
        log(f"profiled {prof_steps} eager steps {prof_elapsed * 1e3:.1f} ms")
    sess.close()
    rt.close()

    ms_step = elapsed / args.steps * 1e3
    tok_s = committed / elapsed
    dev_ms = (m1["rocm_total_forward_ms"] - m0["rocm_total_forward_ms"]) / args.steps
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "bd3lm-qwen3-0.6b-q4g64 denoise step, 8192-token committed "
                               "prefix, block 32, 8 steps/block, 4 tokens/step",
                   "prefix_len": PREFIX, "block_size": BLOCK, "steps_per_block": STEPS_PER_BLOCK,
                   "tokens_per_step": 4, "weights": "q4 affine g64 (MLX packing), seed 4",
                   "kv_cache": "fp16", "mfma_operands": "fp16, fp32 accumulate",
                   "parallelism": "single GPU"},
        "ms_per_denoise_step": round(ms_step, 4),
        "device_forward_ms_per_step": round(dev_ms, 4),
        "committed_tokens": committed,
    }
    if prof_steps > 0:
        names = ("attention", "attention_combine", "linear", "lm_head")
        comp = {}
        for n in names:
            ms = mp[f"rocm_prof_ms_{n}"]
            launches = mp[f"rocm_prof_launches_{n}"]
            byts = mp[f"rocm_prof_bytes_{n}"]
            comp[n] = {"ms_per_step": round(ms / prof_steps, 4), "launches": int(launches),
                       "avg_launch_us": round(ms / max(1, launches) * 1e3, 3),
                       "algorithmic_GBps": round(byts / max(ms, 1e-9) / 1e6, 1)}
        out["components"] = comp
        out["profiled_eager_ms_per_step"] = round(prof_elapsed / prof_steps * 1e3, 4)
        a = comp["attention"]
        achieved = mp["rocm_prof_bytes_attention"] / max(mp["rocm_prof_ms_attention"], 1e-9) / 1e6
        per_launch = mp["rocm_prof_bytes_attention"] / max(1, mp["rocm_prof_launches_attention"])
        out["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                           "traffic": read_traffic(), "kernel": "attn_decode_kernel",
                           "algorithmic_bytes_per_launch": round(per_launch),
                           "avg_launch_us": a["avg_launch_us"], "launches": a["launches"],
                           "timed_over": f"{prof_steps} eager steps after the graph-timed region"}
        # the attention op: the kernel and its range combine, over the same bytes
        op_ms = mp["rocm_prof_ms_attention"] + mp["rocm_prof_ms_attention_combine"]
        op_achieved = mp["rocm_prof_bytes_attention"] / max(op_ms, 1e-9) / 1e6
        out["roofline"]["op"] = {"kernels": "attn_decode_kernel + attn_decode_combine_kernel",
                                 "achieved": round(op_achieved, 1),
                                 "frac": round(op_achieved / HBM_PEAK_GBS, 4),
                                 "avg_op_us": round(op_ms / max(1, a["launches"]) * 1e3, 3)}
    if not args.no_cpu_baseline:
        t = time.perf_counter()
        out["cpu_baseline"] = cpu_baseline(model, prefix, g.mask_token_id, args.cpu_sample_layers)
        log(f"cpu baseline sample took {time.perf_counter() - t:.1f}s")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
