#!/usr/bin/env python3
"""Benchmark of the ragged-batch decode hot path on one MI355X.

Workload: paged decode attention for 64 ragged sequences,
L ~ U[128, 2048], 32 query heads / 8 KV heads, head_dim 128, block size 16, block ids drawn
from a seeded permutation of an 8192-block pool, f32 Q/K/V ~ N(0, 1).  One step = one
fi_attn_decode_paged launch over the whole batch (one layer's decode attention), inputs
already resident in HBM.

Prints ONE JSON line: value = decode tokens/s (64 query tokens per step); ``roofline`` is the
decode kernel's achieved HBM bandwidth from hipEvents on the launch stream over the timed
region (algorithmic bytes / average launch time); ``cpu_baseline`` is the CPU oracle (the
reference's paged decode: gather by block table + cached-prefixed attention, one thread as
the reference uses for a single query row) on the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec
METRIC = "decode tokens/sec @ ragged batch 64; paged-attn achieved HBM GB/s (% peak)"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--kv-dtype", choices=["f32", "bf16"], default="f32")
    p.add_argument("--cpu-reps", type=int, default=0,
                   help="CPU baseline repetitions of the full batch (0 = auto, ~10 s)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--pmc-copy-reference", action="store_true",
                   help="only run a plain 512 MiB device copy (5 launches): the known-size "
                        "reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return p.parse_args()


def pmc_copy_reference():
    import torch

    n = 512 * 1024 * 1024 // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_copy_reference_bytes_per_launch": n * 4, "launches": 5}))


def traffic_from_profile(kv_dtype):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    the copy reference), committed under profiles/ for this workload; None if absent."""
    path = os.path.join(ROOT, "profiles", f"decode_c2_{kv_dtype}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        data = json.load(f)
    return data.get("traffic_bytes_per_launch"), os.path.relpath(path, ROOT)


def cpu_baseline(wl, reps):
    """Times the oracle's restatement of the reference paged decode on the host."""
    import oracle

    oracle.build()
    oracle.set_threads(1)
    kp = wl.pages_reference_layout(wl.k_pool)
    vp = wl.pages_reference_layout(wl.v_pool)
    t0 = time.perf_counter()
    oracle.paged_decode_gather_attention(wl.q, kp, vp, wl.block_tables, wl.context_lens,
                                         wl.block_size)
    one = time.perf_counter() - t0
    if reps <= 0:
        reps = max(1, min(30, int(10.0 / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.paged_decode_gather_attention(wl.q, kp, vp, wl.block_tables, wl.context_lens,
                                             wl.block_size)
    dt = time.perf_counter() - t0
    return {
        "value": round(wl.num_seqs * reps / dt, 2),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full C2 batch ({wl.num_seqs} seqs, sum L={int(wl.context_lens.sum())}) x {reps} "
                  f"reps, f32, 1 thread (the reference runs a 1-row query single-threaded, "
                  f"kernel/cpu/attention.rs:1185-1201); host {os.cpu_count()} cpus",
        "ms_per_step": round(dt / reps * 1e3, 3),
    }


def main():
    args = parse_args()
    if args.pmc_copy_reference:
        pmc_copy_reference()
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(no multi-GPU path exists; see DESIGN.md for how the path would shard)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32, Context
    from ferrisinfer_amd.workloads import paged_decode_c2

    wl = paged_decode_c2(seed=args.seed)
    ctx = Context(0)
    info = ctx.device_info()
    if args.kv_dtype == "bf16":
        def to_bf16(x):
            # round-to-nearest-even, the append kernel's rule (inputs are finite)
            w = x.view(np.uint32).astype(np.uint64)
            w = (w + 0x7FFF + ((w >> 16) & 1)) >> 16
            return w.astype(np.uint16).view(np.int16)

        kp = torch.from_numpy(to_bf16(wl.k_pool)).cuda()
        vp = torch.from_numpy(to_bf16(wl.v_pool)).cuda()
        dt, kv_bytes = DTYPE_BF16, 2
    else:
        kp = torch.from_numpy(wl.k_pool).cuda()
        vp = torch.from_numpy(wl.v_pool).cuda()
        dt, kv_bytes = DTYPE_F32, 4
    q = torch.from_numpy(wl.q).cuda()
    bt = torch.from_numpy(wl.block_tables).cuda()
    cl = torch.from_numpy(wl.context_lens).cuda()
    out = torch.empty_like(q)

    def step():
        ctx.attn_decode_paged(q, kp, vp, dt, bt, cl, wl.max_context_len, wl.num_kv_heads,
                              wl.block_size, wl.num_blocks, wl.scale, out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ctx.check_faults()

    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ctx.check_faults()

    wall = t1 - t0
    kernel_ms = ev0.elapsed_time(ev1) / args.steps
    alg_bytes = wl.algorithmic_bytes(kv_bytes)
    achieved = alg_bytes / (kernel_ms * 1e-3) / 1e9
    traffic, traffic_src = traffic_from_profile(args.kv_dtype)
    result = {
        "metric": METRIC,
        "value": round(wl.num_seqs * args.steps / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.kv_dtype == "f32" else "f32 compute, bf16 KV",
        "data": "synthetic (seeded numpy PCG64, N(0,1) Q/K/V)",
        "config": {
            "workload": "C2 paged decode attention: 64 ragged seqs, L~U[128,2048] "
                        f"(sum L={int(wl.context_lens.sum())}), Hq=32, Hkv=8, D=128, block 16, "
                        f"8192-block pool, {args.kv_dtype} KV",
            "global_batch": wl.num_seqs,
            "kv_dtype": args.kv_dtype,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partition_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": alg_bytes,
            "avg_launch_us": round(kernel_ms * 1e3, 3),
        },
        "device": info,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_reps)
    print(json.dumps(result), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
