#!/usr/bin/env python3
"""Benchmark of the ragged-batch decode hot path on one MI355X.

Workload: paged decode attention for 64 ragged sequences,
L ~ U[128, 2048], 32 query heads / 8 KV heads, head_dim 128, block size 16, block ids drawn
from a seeded permutation of an 8192-block pool, f32 Q/K/V ~ N(0, 1).  One step = one
fi_attn_decode_paged launch over the whole batch (one layer's decode attention), inputs
already resident in HBM.

A second measurement, ``c4``, serves BASELINE config C4 (the Qwen2-0.5B-shaped model under
continuous batching at max batch 64) through the GPU runtime and reports decode tokens/s by
the reference's definition next to the CPU oracle on a declared subset.

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
FP32_PEAK_TFS = 157.3  # MI355X dense fp32 (vector and MFMA), AMD public spec
BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA, AMD public spec
# 5.81 TB/s: read-only kernels over C2's f32 pools at their best decomposition (per-kv-head
# 8 KiB runs, partitions of <= 128 tokens), measured on MI355X
C2_F32_READ_CEILING_FRAC = 0.727
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
    p.add_argument("--no-c4", action="store_true",
                   help="skip the C4 (Qwen2-0.5B-shaped) continuous-batching measurement")
    p.add_argument("--c4-requests", type=int, default=128)
    p.add_argument("--c4-variants", default="graph,ahead,eager,sampled,bf16",
                   help="C4 runs to make (comma list of graph, ahead, eager, sampled, bf16); graph "
                        "(else eager) fills the top-level c4 figures; ahead runs the top-level "
                        "configuration with FR_TICK_RUN_AHEAD")
    p.add_argument("--no-c5", action="store_true",
                   help="skip the C5 (Llama-3-8B-shaped, bf16 weights and KV) decode-step measurement")
    p.add_argument("--c5-steps", type=int, default=5)
    p.add_argument("--c5-runtime-ticks", type=int, default=20,
                   help="C5 decode ticks at batch 256 timed through the runtime (0 skips that leg)")
    p.add_argument("--no-kernels", action="store_true",
                   help="skip the C3 prefill/append and projection-GEMM kernel measurements")
    p.add_argument("--hf-load", action="store_true",
                   help="also time importing a Qwen2-0.5B-shaped BF16 HF checkpoint")
    p.add_argument("--gemm-shapes", action="store_true",
                   help="only time the projection GEMMs at the C4 shapes (packed-weight path "
                        "against fi_gemm), one JSON line per shape")
    p.add_argument("--pmc-copy-reference", action="store_true",
                   help="only run a plain 512 MiB device copy (5 launches): the known-size "
                        "reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    p.add_argument("--c4-layer-ops", action="store_true",
                   help="only run one C4 decode-tick layer's ops at batch 64 (Qwen2-0.5B shape: the "
                        "M = 64 projections, the q|k|v consumer, KV append, residual norm, SwiGLU "
                        "split sum, greedy head), 10 launches each: the command the C4 counter "
                        "profiles run under rocprofv3")
    return p.parse_args()


def c4_layer_ops(seed):
    """One C4 decode-tick layer's kernels at batch 64 on random inputs, 10 launches each."""
    import numpy as np
    import torch

    from ferrisinfer_amd import DTYPE_F32, Context

    from ferrisinfer_amd.workloads import paged_decode_c2

    ctx = Context(0)
    g = torch.Generator(device="cuda").manual_seed(seed)
    m, h, f, v, hq, hkv, d = 64, 896, 4864, 151936, 14, 2, 64
    nb, bs = 12288, 16
    # the tick's attention: 64 sequences with C4-like contexts; each new token is the last
    # position of its sequence, at the slot its block table gives
    wl = paged_decode_c2(seed=seed, num_seqs=m, min_len=64, max_len=2300, num_q_heads=hq,
                         num_kv_heads=hkv, head_dim=d, block_size=bs, num_blocks=nb)

    def rn(*shape):
        return torch.randn(*shape, device="cuda", generator=g)

    x = rn(m, h)
    nqkv = h + 2 * hkv * d
    pw = 32  # the runtime's pack width for q|k|v, wo and w2
    w_qkv = ctx.weight_pack(rn(h, nqkv) * 0.02, h, nqkv, pw)
    w_o = ctx.weight_pack(rn(h, h) * 0.02, h, h, pw)
    w_2 = ctx.weight_pack(rn(f, h) * 0.02, f, h, pw)
    pair = ctx.weight_pack_pair(rn(h, f) * 0.02, rn(h, f) * 0.02, h, f)
    head = ctx.weight_pack(rn(v, h) * 0.02, h, v, 2, src_layout=1)
    s_qkv = ctx.gemm_packed_splits(m, h, nqkv, pw)
    s_o = ctx.gemm_packed_splits(m, h, h, pw)
    s_w2 = ctx.gemm_packed_splits(m, f, h, pw)
    p_qkv = torch.empty(s_qkv, m, nqkv, device="cuda")
    p_o = torch.empty(s_o, m, h, device="cuda")
    p_w2 = torch.empty(s_w2, m, h, device="cuda")
    act = torch.empty(m, f, device="cuda")
    tok = torch.empty(m, dtype=torch.int32, device="cuda")
    prob = torch.empty(m, device="cuda")
    kp = torch.from_numpy(wl.k_pool).cuda()
    vp = torch.from_numpy(wl.v_pool).cuda()
    last = wl.context_lens.astype(np.int64) - 1
    pos = torch.from_numpy(last.astype(np.int32)).cuda()
    slots = torch.from_numpy(np.array([int(wl.block_tables[b, p // bs]) * bs + p % bs
                                       for b, p in enumerate(last)], np.int64)).cuda()
    bt, cl = torch.from_numpy(wl.block_tables).cuda(), torch.from_numpy(wl.context_lens).cuda()
    attn = torch.empty(m, hq, d, device="cuda")
    cos = torch.empty(4096, d // 2, device="cuda")
    sin = torch.empty_like(cos)
    ctx.rope_table(4096, d, d, 1e6, cos, sin)
    q = torch.empty(m, hq, d, device="cuda")
    kn, vn = rn(m, hkv, d), rn(m, hkv, d)
    res = rn(m, h)
    ssum = torch.empty(m, h, device="cuda")
    nw = torch.ones(h, device="cuda")
    nout = torch.empty(m, h, device="cuda")
    for _ in range(10):
        ctx.gemm_packed(x, w_qkv, h, nqkv, pw, s_qkv, p_qkv)
        ctx.qkv_rope_append(p_qkv, s_qkv, None, pos, cos, sin, d, 4096, slots, kp, vp, DTYPE_F32, nb, bs,
                            hq, hkv, d, q)
        ctx.kv_append(kn, vn, slots, kp, vp, DTYPE_F32, nb, bs, hkv, d)
        # the decode tick's attention: the q|k|v consumer folded in (decode_partition_kernel
        # merging in its last-arriving workgroups), as the runtime runs it
        ctx.attn_decode_paged_qkv(p_qkv, s_qkv, None, pos, cos, sin, d, 4096, slots, kp, vp, DTYPE_F32, bt, cl,
                                  wl.max_context_len, hq, hkv, d, bs, nb, wl.scale, attn, q_out=q)
        ctx.gemm_packed(x, w_o, h, h, pw, s_o, p_o)
        ctx.splitk_residual_rms_norm(p_o, s_o, None, res, ssum, nw, nout, 1e-6)
        ctx.gemm_packed_swiglu(x, pair, h, f, act)
        ctx.gemm_packed(act, w_2, f, h, pw, s_w2, p_w2)
        ctx.lm_head_argmax_packed(x, head, v, tok, prob)
    torch.cuda.synchronize()
    ctx.check_faults()
    print(json.dumps({"c4_layer_ops": "done", "splits": {"qkv": s_qkv, "wo": s_o, "w2": s_w2}}), flush=True)
    ctx.close()


def pmc_copy_reference():
    import torch

    n = 512 * 1024 * 1024 // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_copy_reference_bytes_per_launch": n * 4, "launches": 5}))


def gemm_shapes(seed):
    """Projection GEMMs at the C4 (Qwen2-0.5B) shapes: the packed-weight kernel at every
    pack width against fi_gemm (checked equal within 1e-5 normwise), the SwiGLU pair and the
    packed greedy head; M = 64 (a decode tick) and M = 1024 (a prefill chunk)."""
    import torch

    from ferrisinfer_amd import Context

    ctx = Context(0)
    g = torch.Generator(device="cuda").manual_seed(seed)

    def ms(fn, reps=50):
        return timed(fn, reps, warmup=5)

    for m in (64, 1024):
        for name, k, n in (("qkv", 896, 1152), ("wo", 896, 896), ("w2", 4864, 896), ("w13", 896, 9728)):
            a = torch.randn(m, k, device="cuda", generator=g)
            w = torch.randn(k, n, device="cuda", generator=g) * 0.02
            c = torch.empty(m, n, device="cuda")
            row = {"shape": name, "m": m, "k": k, "n": n,
                   "fi_gemm_us": round(ms(lambda: ctx.gemm(a, w, c)) * 1e3, 2)}
            for pw in (1, 2, 4, 32):
                bp = ctx.weight_pack(w, k, n, pw)
                s = ctx.gemm_packed_splits(m, k, n, pw)
                out = torch.empty(s, m, n, device="cuda")
                us = ms(lambda: ctx.gemm_packed(a, bp, k, n, pw, s, out)) * 1e3
                err = float((out.sum(0) - c).abs().max() / c.abs().max())
                assert err < 1e-5, (name, m, pw, err)
                row[f"packed_pw{pw}"] = {"us": round(us, 2), "splits": s,
                                         "tflops": round(2 * m * n * k / us / 1e6, 1),
                                         "weight_gbs": round(4 * k * n / us / 1e3, 1)}
            print(json.dumps(row), flush=True)
        k, f = 896, 4864
        a = torch.randn(m, k, device="cuda", generator=g)
        w1 = torch.randn(k, f, device="cuda", generator=g) * 0.02
        w3 = torch.randn(k, f, device="cuda", generator=g) * 0.02
        bp = ctx.weight_pack_pair(w1, w3, k, f)
        out = torch.empty(m, f, device="cuda")
        us = ms(lambda: ctx.gemm_packed_swiglu(a, bp, k, f, out)) * 1e3
        print(json.dumps({"shape": "w1/w3 pair + swiglu", "m": m, "k": k, "n": f, "us": round(us, 2),
                          "tflops": round(2 * m * k * 2 * f / us / 1e6, 1)}), flush=True)
    h, v = 896, 151936
    w = torch.randn(v, h, device="cuda", generator=g) * 0.02
    bp = ctx.weight_pack(w, h, v, 2, src_layout=1)
    for m in (1, 16, 64):
        hid = torch.randn(m, h, device="cuda", generator=g)
        tok = torch.empty(m, dtype=torch.int32, device="cuda")
        prob = torch.empty(m, device="cuda")
        old = ms(lambda: ctx.lm_head_argmax(hid, w, tok, prob), 20) * 1e3
        us = ms(lambda: ctx.lm_head_argmax_packed(hid, bp, v, tok, prob), 20) * 1e3
        print(json.dumps({"shape": "lm_head argmax", "m": m, "k": h, "n": v,
                          "fi_lm_head_argmax_us": round(old, 2), "packed_us": round(us, 2),
                          "weight_gbs": round(4 * h * v / us / 1e3, 1),
                          "tflops": round(2 * m * h * v / us / 1e6, 1)}), flush=True)
    ctx.close()


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


def timed(fn, reps, warmup=3):
    """Average device time (ms) of fn over reps launches, hipEvents on torch's current
    stream (the stream the library's context follows)."""
    import torch

    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def gemm_row(m, k, n, ms, splits, pw):
    """One projection leg: MFMA fraction (2·M·K·N) and weight-stream HBM fraction (4·K·N)."""
    fl = 2 * m * n * k
    wb = 4 * k * n
    return {"m": m, "k": k, "n": n, "pack_width": pw, "splits": splits,
            "avg_launch_us": round(ms * 1e3, 2),
            "achieved_tflops": round(fl / (ms * 1e-3) / 1e12, 2),
            "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / FP32_PEAK_TFS, 4),
            "weight_gbs": round(wb / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(wb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def kernel_legs(ctx, seed):
    """C3 varlen prefill attention (MFMA f32) and KV append (HBM) at full size, and the
    packed projection GEMMs at the C4 shapes: a decode tick (M = 64, where f32 weight
    streaming and MFMA are balanced) and a prefill chunk (M = 1024, MFMA-bound)."""
    import numpy as np
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32
    from ferrisinfer_amd.workloads import prefill_c3

    out = {}
    wl = prefill_c3(seed=seed)
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    shape = (wl.num_blocks, wl.num_kv_heads, wl.block_size, wl.head_dim)
    kp = torch.zeros(shape, device="cuda")
    vp = torch.zeros(shape, device="cuda")
    k_new, v_new, slots, q = d(wl.k_new), d(wl.v_new), d(wl.slot_mapping), d(wl.q)
    bt, cu, cl = d(wl.block_tables), d(wl.cu_seqlens), d(wl.context_lens)
    o = torch.empty_like(q)
    T = int(wl.cu_seqlens[-1])

    def append():
        ctx.kv_append(k_new, v_new, slots, kp, vp, DTYPE_F32, wl.num_blocks, wl.block_size,
                      wl.num_kv_heads, wl.head_dim)

    def prefill():
        ctx.attn_prefill_paged(q, kp, vp, DTYPE_F32, bt, cu, cl, int(wl.query_lens.max()),
                               wl.num_kv_heads, wl.block_size, wl.num_blocks, wl.scale, o)

    ms_a = timed(append, 50)
    ms_p = timed(prefill, 20)
    ctx.check_faults()
    flops = wl.attention_flops()
    ab = wl.append_bytes(4)
    # f32 arithmetic as six bf16 MFMAs per product (three-piece operands): frac is against the
    # f32 dense peak; frac_of_three_piece_peak against the bf16 peak / 6, the kernel's own ceiling
    out["c3_prefill_attention"] = {
        "kernel": "prefill_x3_kernel", "bound": "mfma (f32 accuracy on bf16 MFMA, six products each)",
        "tokens": T, "flops_per_launch": flops, "avg_launch_us": round(ms_p * 1e3, 2),
        "achieved_tflops": round(flops / (ms_p * 1e-3) / 1e12, 2), "peak_tflops": FP32_PEAK_TFS,
        "frac": round(flops / (ms_p * 1e-3) / 1e12 / FP32_PEAK_TFS, 4),
        "frac_of_three_piece_peak": round(flops / (ms_p * 1e-3) / 1e12 / (BF16_PEAK_TFS / 6), 4)}
    # the same workload on a bf16 pool through the bf16-MFMA variant
    kb = torch.zeros(shape, dtype=torch.int16, device="cuda")
    vb = torch.zeros(shape, dtype=torch.int16, device="cuda")
    ctx.kv_append(k_new, v_new, slots, kb, vb, DTYPE_BF16, wl.num_blocks, wl.block_size,
                  wl.num_kv_heads, wl.head_dim)

    def prefill_bf16():
        ctx.attn_prefill_paged_bf16(q, kb, vb, bt, cu, cl, int(wl.query_lens.max()), wl.num_kv_heads,
                                    wl.block_size, wl.num_blocks, wl.scale, o)

    ms_b = timed(prefill_bf16, 20)
    ctx.check_faults()
    out["c3_prefill_attention_bf16_mfma"] = {
        "kernel": "prefill_bf16_kernel", "bound": "mfma (bf16)", "kv_dtype": "bf16",
        "tokens": T, "flops_per_launch": flops, "avg_launch_us": round(ms_b * 1e3, 2),
        "achieved_tflops": round(flops / (ms_b * 1e-3) / 1e12, 2), "peak_tflops": BF16_PEAK_TFS,
        "frac": round(flops / (ms_b * 1e-3) / 1e12 / BF16_PEAK_TFS, 4)}
    del kb, vb
    out["c3_kv_append"] = {
        "kernel": "kv_append4_kernel", "bound": "hbm", "tokens": T,
        "bytes_per_launch": ab, "avg_launch_us": round(ms_a * 1e3, 2),
        "achieved_gbs": round(ab / (ms_a * 1e-3) / 1e9, 1), "peak_gbs": HBM_PEAK_GBS,
        "frac": round(ab / (ms_a * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del kp, vp, k_new, v_new, slots, q, o

    # the projections as the runtime runs them: packed weights, pack widths of
    # DeviceModel (q|k|v, wo and w2 32, w1/w3 SwiGLU pair, lm_head 2), C4 shapes
    g = torch.Generator(device="cuda").manual_seed(seed)
    for m in (64, 1024):
        tag = "decode" if m == 64 else "prefill"
        for name, k, n, pw in (("qkv", 896, 1152, 32), ("wo", 896, 896, 32), ("w2", 4864, 896, 32)):
            a = torch.randn(m, k, device="cuda", generator=g)
            w = torch.randn(k, n, device="cuda", generator=g) * 0.02
            bp = ctx.weight_pack(w, k, n, pw)
            splits = ctx.gemm_packed_splits(m, k, n, pw)
            parts = torch.empty(splits, m, n, device="cuda")
            ms = timed(lambda: ctx.gemm_packed(a, bp, k, n, pw, splits, parts), 50)
            out[f"gemm_c4_{tag}_{name}"] = gemm_row(m, k, n, ms, splits, pw)
        k, f = 896, 4864
        a = torch.randn(m, k, device="cuda", generator=g)
        w1 = torch.randn(k, f, device="cuda", generator=g) * 0.02
        w3 = torch.randn(k, f, device="cuda", generator=g) * 0.02
        bp = ctx.weight_pack_pair(w1, w3, k, f)
        act = torch.empty(m, f, device="cuda")
        ms = timed(lambda: ctx.gemm_packed_swiglu(a, bp, k, f, act), 50)
        out[f"gemm_c4_{tag}_w13_swiglu"] = gemm_row(m, k, 2 * f, ms, 1, 2)
    h, v = 896, 151936
    w = torch.randn(v, h, device="cuda", generator=g) * 0.02
    bp = ctx.weight_pack(w, h, v, 2, src_layout=1)
    for m in (1, 64):
        hid = torch.randn(m, h, device="cuda", generator=g)
        tok = torch.empty(m, dtype=torch.int32, device="cuda")
        prob = torch.empty(m, device="cuda")
        ms = timed(lambda: ctx.lm_head_argmax_packed(hid, bp, v, tok, prob), 20)
        out[f"lm_head_argmax_c4_m{m}"] = gemm_row(m, h, v, ms, 1, 2)
    del w, bp
    # device sampling (sample_last_token per row, one workgroup per row): the logits are
    # read once, so the bound is HBM at rows * vocab * 4 bytes per launch; N(0, 2.5) logits
    # under the reference's chat_default sampler (top-k 20) and a greedy configuration.  Then
    # the paths off the fast one: top-k 1024 on N(0, 1) rows (equal values among the 1025
    # largest in about a fifth of them), top-k 20 on bf16-rounded logits (equal values nearly
    # everywhere), and top-k above 1024 (the reserved-area launch: a radix sort of each row and
    # sequential walks over up to `vocab` weights, so not an HBM-bound figure; the reservation
    # comes last, as a reserved context launches that kernel on every call)
    for tag, rows, vocab, cfg, scale, bf16 in (
            ("c4_m64_topk20", 64, 151936, (0.7, 20, 0.9), 2.5, False),
            ("c5_m257_topk20", 257, 128256, (0.7, 20, 0.9), 2.5, False),
            ("c4_m64_greedy", 64, 151936, (0.0, 1, 1.0), 2.5, False),
            ("c4_m64_topk1024", 64, 151936, (1.0, 1024, 0.95), 1.0, False),
            ("c4_m64_topk20_bf16_logits", 64, 151936, (0.7, 20, 0.9), 2.5, True),
            ("c4_m64_topk2000", 64, 151936, (0.7, 2000, 0.9), 2.5, False),
            ("c4_m64_topk_vocab", 64, 151936, (1.0, 151936, 1.0), 1.0, False)):
        logits = torch.randn(rows, vocab, device="cuda", generator=g) * scale
        if bf16:
            logits = logits.to(torch.bfloat16).float()
        if cfg[1] > 1024:
            ctx.sample_reserve(rows, vocab)
        temp = torch.full((rows,), cfg[0], device="cuda")
        topk = torch.full((rows,), cfg[1], dtype=torch.int32, device="cuda")
        topp = torch.full((rows,), cfg[2], device="cuda")
        st = torch.arange(1, rows + 1, dtype=torch.int64, device="cuda")
        tok = torch.empty(rows, dtype=torch.int32, device="cuda")
        prob = torch.empty(rows, device="cuda")
        ms = timed(lambda: ctx.sample_tokens(logits, temp, topk, topp, st, tok, prob), 20)
        b = rows * vocab * 4
        out[f"sample_tokens_{tag}"] = {
            "kernel": ("sample_row_kernel<4>" if rows >= 256 else "sample_scan_kernel<4> + sample_finish_kernel<4>") +
                      (" + sample_large_kernel<4>" if cfg[1] > 1024 else ""),
            "bound": "hbm", "rows": rows, "vocab": vocab,
            "temperature": cfg[0], "top_k": cfg[1], "top_p": cfg[2], "bytes_per_launch": b,
            "avg_launch_us": round(ms * 1e3, 2), "achieved_gbs": round(b / (ms * 1e-3) / 1e9, 1),
            "peak_gbs": HBM_PEAK_GBS, "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del logits
    # checkpoint import (fi_convert_to_f32): HBM-bound, 2 bytes read + 4 written per element;
    # a Qwen2 MLP weight [4864, 896] bf16 transposed to [896, 4864] f32, and the [151936, 896]
    # embedding widened in place order
    from ferrisinfer_amd import DTYPE_F16
    for tag, rows, cols, dt, tr in (("bf16_t_4864x896", 4864, 896, DTYPE_BF16, True),
                                    ("f16_t_4864x896", 4864, 896, DTYPE_F16, True),
                                    ("bf16_151936x896", 151936, 896, DTYPE_BF16, False)):
        src = torch.randint(-32768, 32767, (rows * cols,), dtype=torch.int16, device="cuda", generator=g)
        dst = torch.empty(rows * cols, device="cuda")
        ms = timed(lambda: ctx.convert_to_f32(src, dt, rows, cols, tr, dst), 20)
        b = rows * cols * 6
        out[f"convert_to_f32_{tag}"] = {
            "kernel": "widen_transpose_kernel" if tr else "widen_kernel", "bound": "hbm",
            "bytes_per_launch": b, "avg_launch_us": round(ms * 1e3, 2),
            "achieved_gbs": round(b / (ms * 1e-3) / 1e9, 1), "peak_gbs": HBM_PEAK_GBS,
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del src, dst
    ctx.check_faults()
    return out


def hf_load(seed):
    """A Qwen2-0.5B-shaped checkpoint (BF16, tied, q/k/v biases, random values; 988 MB of
    safetensors in 2 shards) written to a temporary directory, then imported by the runtime:
    config + every tensor to HBM with on-device widening / transposes (Runtime.from_hf), and
    the first submit, which packs the projections for the GEMM kernels."""
    import shutil
    import tempfile

    import numpy as np

    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, write_qwen2_checkpoint

    cfg = dict(QWEN2_05B_C4)
    tmp = tempfile.mkdtemp(prefix="fi_hf_")
    try:
        t0 = time.perf_counter()
        written = write_qwen2_checkpoint(tmp, cfg, "BF16", seed=seed, shards=2, biases=True, std=0.02)
        t_write = time.perf_counter() - t0
        nbytes = sum(len(raw) for *_, raw in written.values())
        del written
        t0 = time.perf_counter()
        rt = Runtime.from_hf(tmp, num_blocks=64, block_size=16)
        t_load = time.perf_counter() - t0
        t0 = time.perf_counter()
        rt.submit(np.arange(8, dtype=np.uint32), max_new_tokens=1)
        t_pack = time.perf_counter() - t0
        rt.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return {"workload": "Qwen2-0.5B-shaped HF checkpoint, BF16, 2 shards, tied, q/k/v biases",
            "safetensors_bytes": nbytes, "write_s": round(t_write, 2), "load_s": round(t_load, 3),
            "load_gbs": round(nbytes / t_load / 1e9, 2), "first_submit_pack_s": round(t_pack, 3)}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def c4_model_bytes_flops(cfg, weight_bytes):
    """Per decode token: the projection and head weights every tick streams (bytes at the given
    storage width) and their multiply-adds (2 FLOPs per weight per token)."""
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])
    per_layer = h * (h + 2 * kvw) + h * h + 2 * h * f + f * h
    params = cfg["layers"] * per_layer + v * h
    return params * weight_bytes, 2 * params


def c4_roofline(cfg, ticks, weight_bytes, peak_tfs):
    """Roofline of the decode ticks at batch 64: algorithmic bytes = the weights once per tick +
    every sequence's K/V (ctx tokens x layers x 2 x Hkv x D x 4 bytes, f32 pool) + the new K/V rows;
    FLOPs = 2 x params x 64 + attention 4 x Hq x D x ctx per layer.  The bound is whichever of
    HBM (8 TB/s) and the MFMA peak of the weight dtype needs more time."""
    full = [t for t in ticks if t["kind"] == 1 and t["batch"] == 64 and "ctx_sum" in t]
    if not full:
        return None
    d = cfg["hidden"] // cfg["heads"]
    wbytes, wflops_per_tok = c4_model_bytes_flops(cfg, weight_bytes)
    kv_per_tok = cfg["layers"] * 2 * cfg["kv_heads"] * d * 4
    secs = sum(t["seconds"] for t in full)
    byt = sum(wbytes + t["ctx_sum"] * kv_per_tok for t in full)
    flops = sum(64 * wflops_per_tok + cfg["layers"] * 4 * cfg["heads"] * d * t["ctx_sum"] for t in full)
    t_hbm = byt / (HBM_PEAK_GBS * 1e9)
    t_mfma = flops / (peak_tfs * 1e12)
    bound = "hbm" if t_hbm >= t_mfma else "mfma"
    return {
        "bound": bound,
        "ticks": len(full),
        "bytes_per_tick": int(byt / len(full)),
        "flops_per_tick": int(flops / len(full)),
        "achieved_gbs": round(byt / secs / 1e9, 1),
        "achieved_tflops": round(flops / secs / 1e12, 2),
        "roofline_ms_per_tick": round(max(t_hbm, t_mfma) / len(full) * 1e3, 4),
        "ms_per_tick": round(secs / len(full) * 1e3, 4),
        "frac": round(max(t_hbm, t_mfma) / secs, 4),
        "peaks": {"hbm_gbs": HBM_PEAK_GBS, "mfma_tflops": peak_tfs},
    }


_C4_WEIGHTS = {}


def c4_weights(seed):
    """The C4 model's seeded weights, generated once per seed for every leg that serves them."""
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, random_weights

    if seed not in _C4_WEIGHTS:
        _C4_WEIGHTS.clear()
        _C4_WEIGHTS[seed] = random_weights(QWEN2_05B_C4, seed=seed, qkv_bias=True)
    return _C4_WEIGHTS[seed]


def c4_continuous(seed, n_requests, sampler=None, graph=True, weight_dtype="f32", run_ahead=False):
    """C4: the Qwen2-0.5B-shaped model (f32, tied, q/k/v biases, random N(0, 0.02) weights)
    served by the GPU runtime under continuous batching (max batch 64, block 16, the
    reference scheduler's other defaults), Poisson arrivals at 8 req/s on 50 ms virtual
    ticks.  Decode tok/s = generated tokens / summed decode-tick wall time, the reference's
    continuous-batching definition (cli/main.rs:1502-1512, 1619-1622).  sampler: None for
    greedy sessions, or (temperature, top_k, top_p, seed) for sampled ones; graph: decode ticks
    replayed from HIP graphs; weight_dtype: storage of the packed projections and head;
    run_ahead: each tick followed by no arrival enqueues the next decode tick before it returns
    (FR_TICK_RUN_AHEAD), and such a tick's seconds run from the previous tick's return, the
    driver's own time in between included."""
    import numpy as np

    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, c4_requests, run_continuous

    cfg = QWEN2_05B_C4
    weights = c4_weights(seed)
    rt = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                 cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=True, max_seq=4096,
                 max_gen=512, max_batch=64, num_blocks=16384, block_size=16, sampler=sampler,
                 graph_decode=graph, weight_dtype=weight_dtype)
    rt.set_weights(weights)
    del weights
    # warm-up: one short request through prefill and decode (module load, first launches)
    run_continuous(rt, [dict(prompt=np.arange(300, dtype=np.uint32), max_new_tokens=3,
                             arrival_tick=0)])
    reqs = c4_requests(seed=seed, n=n_requests)
    t0 = time.perf_counter()
    rep = run_continuous(rt, reqs, run_ahead=run_ahead)
    wall = time.perf_counter() - t0
    full = [t for t in rep["ticks"] if t["kind"] == 1 and t["batch"] == 64]
    full_s = sum(t["seconds"] for t in full)
    dec = [t for t in rep["ticks"] if t["kind"] == 1]
    split = {k: round(sum(t["profile"][k] for t in dec) / max(len(dec), 1) * 1e3, 3)
             for k in ("schedule", "enqueue", "wait", "total")}
    out = {
        "workload": f"C4 Qwen2-0.5B shape, {n_requests} requests, Poisson 8/s on 50 ms virtual "
                    "ticks, prompts lognormal(median 512, sigma 0.5) clipped [1,2048], outputs "
                    "U[64,256], " + ("greedy" if sampler is None else
                                     "sampled (temperature, top_k, top_p, seed) = " + str(sampler))
                    + f", max batch 64, block 16, {weight_dtype} weights, f32 KV, decode ticks "
                    + ("replayed from HIP graphs" if graph else "enqueued eagerly")
                    + (", the next decode tick enqueued before each tick returns when no request "
                       "arrives in between" if run_ahead else ""),
        "decode_tok_s": round(rep["decode_tok_s"], 1),
        "decode_tok_s_at_batch_64": round(64 * len(full) / full_s, 1) if full_s > 0 else None,
        "ms_per_decode_tick_at_batch_64": round(full_s / len(full) * 1e3, 3) if full else None,
        "prefill_tok_s": round(rep["prefill_tok_s"], 1),
        "generated_tokens": rep["generated_tokens"],
        "decode_ticks": rep["decode_ticks"],
        "prefill_ticks": rep["prefill_ticks"],
        "avg_decode_batch": round(rep["avg_decode_batch"], 2),
        "decode_ticks_at_batch_64": len(full),
        "decode_tick_host_ms": split,
        "wall_s": round(wall, 3),
        "roofline_at_batch_64": c4_roofline(cfg, rep["ticks"], 4 if weight_dtype == "f32" else 2,
                                            FP32_PEAK_TFS if weight_dtype == "f32" else BF16_PEAK_TFS),
    }
    if graph:
        out["graph_counters"] = rt.graph_counters()
    if run_ahead:
        out["run_ahead_counters"] = rt.run_ahead_counters()
    # generated ids per request, for the graph-versus-eager comparison (not printed)
    out["_tokens"] = [rt.generated(s) for s in rep["sequence_ids"]]
    rt.close()
    return out


C5_LAYER_SHAPES = ("attention.wq.weight", "attention.wk.weight", "attention.wv.weight", "attention.wo.weight",
                   "feed_forward.w1.weight", "feed_forward.w2.weight", "feed_forward.w3.weight")


def c5_shape_of(cfg, name):
    h, f = cfg["hidden"], cfg["intermediate"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])
    return {"attention.wq.weight": (h, h), "attention.wk.weight": (h, kvw), "attention.wv.weight": (h, kvw),
            "attention.wo.weight": (h, h), "feed_forward.w1.weight": (h, f), "feed_forward.w2.weight": (f, h),
            "feed_forward.w3.weight": (h, f)}[name]


def c5_seeded_layers(seed, cfg):
    """Every layer's projection weights, N(0, 0.02) from ferrisinfer_amd.seeded (tag = CRC-32 of
    "layers.<l>.<name>", the names and [in, out] layout of workloads.random_weights), drawn on
    the device and held as bf16: {name: [layers, in, out] bf16}."""
    import torch

    from ferrisinfer_amd import seeded
    from ferrisinfer_amd.seeded import tag_of

    return {name: seeded.normals_torch(seed, [tag_of(f"layers.{li}.{name}") for li in range(cfg["layers"])],
                                       c5_shape_of(cfg, name), scale=0.02, out_dtype=torch.bfloat16)
            for name in C5_LAYER_SHAPES}


def c5_seeded_matrix(seed, name, shape):
    """One N(0, 0.02) seeded matrix (tag = CRC-32 of `name`) as bf16 on the device."""
    import torch

    from ferrisinfer_amd import seeded
    from ferrisinfer_amd.seeded import tag_of

    return seeded.normals_torch(seed, [tag_of(name)], shape, scale=0.02, out_dtype=torch.bfloat16)[0]


def fill_tiled(flat, tile):
    """flat[i] = tile[i % len(tile)] (device tensors)."""
    n, t = flat.numel(), tile.numel()
    full = n // t
    if full:
        flat[:full * t].view(full, t).copy_(tile.expand(full, t))
    if n - full * t:
        flat[full * t:].copy_(tile[:n - full * t])


def c5_runtime_decode(seed, ticks, warmup=8, groups=16):
    """C5 through the runtime ABI: the full 32-layer Llama-3-8B-shaped model with bf16 weights
    and a bf16 KV pool (fr_create / fr_set_weight_device / fr_submit / fr_execute_next_tick,
    decode ticks replayed from HIP graphs), 256 sequences with contexts U[512, 8192]
    (ferrisinfer_amd.seeded).  Sequence i's prompt is a prefix of group (i mod 16)'s seeded
    token stream: the group's longest prompt is prefilled first (2048-token chunks, the C5
    tick budget), then the other 240 share its blocks through the scheduler's prefix sharing
    and compute one token each.  Times `ticks` decode ticks at batch 256 after `warmup`."""
    import numpy as np
    import torch

    from ferrisinfer_amd import seeded
    from ferrisinfer_amd.bf16_decoder import LLAMA3_8B_C5
    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.seeded import tag_of

    cfg = LLAMA3_8B_C5
    h, v = cfg["hidden"], cfg["vocab"]
    n = 256
    lens = seeded.integers(seed, tag_of("c5.runtime.context_lens"), n, 512, 8192)
    members = [[i for i in range(n) if i % groups == g] for g in range(groups)]
    source = [max(m, key=lambda i: lens[i]) for m in members]
    streams = [seeded.integers(seed, tag_of(f"c5.runtime.prompt.{g}"), int(lens[source[g]]), 0, v - 1)
               .astype(np.uint32) for g in range(groups)]
    prompts = [streams[i % groups][:int(lens[i])] for i in range(n)]
    # no sequence may finish before the timed ticks: the sources decode between their prefill
    # chunks (two prefill ticks, then a decode tick) and every sequence while the others are
    # admitted
    gen = 512
    unique = sum(int(lens[s]) for s in source)
    num_blocks = (unique + n * 160) // 16 + 2 * n
    t0 = time.time()
    rt = Runtime(h, cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"], v, cfg["max_pos"], cfg["eps"],
                 cfg["theta"], tie=False, max_seq=cfg["max_pos"], max_gen=gen, max_batch=n, max_chunk=2048,
                 max_batch_tokens=2048, num_blocks=num_blocks, block_size=16, kv_dtype="bf16",
                 weight_dtype="bf16", graph_decode=True)
    layers = c5_seeded_layers(seed, cfg)
    for name, stack in layers.items():
        for li in range(cfg["layers"]):
            rt.set_weight_device(f"layers.{li}.{name}", stack[li])
    del layers
    ones = torch.ones(h, device="cuda")
    for li in range(cfg["layers"]):
        rt.set_weight_device(f"layers.{li}.attention_norm.weight", ones)
        rt.set_weight_device(f"layers.{li}.ffn_norm.weight", ones)
    rt.set_weight_device("norm.weight", ones)
    for name in ("tok_embeddings.weight", "output.weight"):
        rt.set_weight_device(name, c5_seeded_matrix(seed, name, (v, h)))
    torch.cuda.empty_cache()
    t_weights = time.time() - t0
    print(f"bench: C5 runtime weights set in {t_weights:.1f} s; prefilling {groups} sources", file=sys.stderr,
          flush=True)
    t0 = time.time()
    seqs = {}
    for g in range(groups):
        seqs[source[g]] = rt.submit(prompts[source[g]], max_new_tokens=gen)
    while any(len(rt.generated(seqs[s])) == 0 for s in source):
        rt.execute_next_tick()
    for i in range(n):
        if i not in seqs:
            seqs[i] = rt.submit(prompts[i], max_new_tokens=gen)
    while any(len(rt.generated(seqs[i])) == 0 for i in range(n)):
        rt.execute_next_tick()
    t_setup = time.time() - t0
    print(f"bench: C5 runtime sequences admitted in {t_setup:.1f} s; timing decode ticks", file=sys.stderr,
          flush=True)
    times, batches, ctx_sums = [], [], []
    while len(times) < warmup + ticks:
        tick = rt.execute_next_tick()
        if tick is None:
            break
        if tick[0] == 1:  # decode
            times.append(rt.last_tick_seconds)
            batches.append(len(tick[1]))
            ctx_sums.append(rt.last_batch_context_sum())
    timed = times[warmup:]
    ms = 1e3 * sum(timed) / max(len(timed), 1)
    counters = rt.graph_counters()
    res = {
        "workload": "C5 model through the runtime ABI: 32 layers, bf16 weights (N(0,0.02), seeded, widened on the "
                    "device), bf16 activations into the projections, bf16 KV; 256 sequences, contexts "
                    "U[512,8192] (seeded) as prefixes of 16 seeded prompts sharing pool blocks; decode ticks "
                    "replayed from HIP graphs, wall time of fr_execute_next_tick",
        "ms_per_tick": round(ms, 3),
        "decode_tok_s": round(sum(batches[warmup:]) / max(sum(timed), 1e-9), 1),
        "batch_min_max": [min(batches[warmup:]), max(batches[warmup:])] if len(batches) > warmup else None,
        "ticks": len(timed),
        "avg_context": round(float(np.sum(ctx_sums[warmup:])) / max(sum(batches[warmup:]), 1), 1),
        # KV rows every tick reads (K and V, bf16, every layer), many of them from blocks the
        # sequences share
        "kv_read_gb_per_tick": round(float(np.mean(ctx_sums[warmup:])) * cfg["layers"] * cfg["kv_heads"] *
                                     (h // cfg["heads"]) * 2 * 2 / 1e9, 1) if len(ctx_sums) > warmup else None,
        "unique_kv_tokens": unique,
        "graph_counters": counters,
        "setup_s": {"weights": round(t_weights, 1), "prefill_and_admission": round(t_setup, 1)},
    }
    rt.close()
    torch.cuda.empty_cache()
    return res


def c5_step(seed, steps):
    """C5: the Llama-3-8B-shaped decoder (32 layers, hidden 4096, Hq 32 / Hkv 8, D 128, FFN
    14336, vocab 128256, untied head) with N(0, 0.02) bf16 weights (ferrisinfer_amd.seeded) and
    a bf16 KV pool per layer sized for the step's 257 sequences (about 147 GB over the 32 layers,
    N(0, 1) contents from a seeded tile).
    One step = 256 decode tokens (contexts U[512, 8192]) + one 2048-token prefill chunk (2048
    tokens already cached) through every layer and the greedy head.  Also times layer 0's ops
    one by one for their roofline fractions."""
    import numpy as np
    import torch

    from ferrisinfer_amd import Context, seeded
    from ferrisinfer_amd.bf16_decoder import LLAMA3_8B_C5, Bf16Decoder, build_step_batch, c5_step_shape
    from ferrisinfer_amd.seeded import tag_of

    cfg = LLAMA3_8B_C5
    h, f, v, hq, hkv = cfg["hidden"], cfg["intermediate"], cfg["vocab"], cfg["heads"], cfg["kv_heads"]
    d = h // hq
    bs = 16
    decode_ctx, prefill = c5_step_shape(seed)
    lens = list(decode_ctx) + [p + n for p, n in prefill]
    num_blocks = sum((n + bs - 1) // bs for n in lens)
    t = len(decode_ctx) + sum(n for _, n in prefill)
    ctx = Context(0)
    dec = Bf16Decoder(ctx, cfg, num_blocks, bs, max_tokens=t, max_last_rows=len(lens))
    layers = c5_seeded_layers(seed, cfg)
    ones = torch.ones(h, device="cuda")
    for li in range(cfg["layers"]):
        lw = {k: layers[k][li] for k in layers}
        dec.set_layer(lw["attention.wq.weight"], lw["attention.wk.weight"], lw["attention.wv.weight"],
                      lw["attention.wo.weight"], lw["feed_forward.w1.weight"], lw["feed_forward.w2.weight"],
                      lw["feed_forward.w3.weight"], ones, ones)
    del layers
    dec.set_head(ones, c5_seeded_matrix(seed, "output.weight", (v, h)))
    for li, (kp, vp) in enumerate(zip(dec.k_pools, dec.v_pools)):  # N(0, 1) contents, a seeded 2^20-value tile
        for name, pool in (("k", kp), ("v", vp)):
            fill_tiled(pool.view(torch.bfloat16).view(-1),
                       seeded.normals_torch(seed, [tag_of(f"c5.kv_pool.{li}.{name}")], (1 << 20,),
                                            out_dtype=torch.bfloat16)[0])
    kv_bytes = sum(p.numel() * 2 for p in dec.k_pools + dec.v_pools)
    batch, _ = build_step_batch(decode_ctx, prefill, bs, num_blocks, seed)
    # synthetic embeddings of the step's tokens
    x = seeded.normals_torch(seed, [tag_of("c5.step_input")], (t, h), scale=0.02)[0]
    torch.cuda.synchronize()

    dec.step(x, batch)  # warm-up
    torch.cuda.synchronize()
    ctx.check_faults()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        dec.step(x, batch)
    e1.record(stream)
    torch.cuda.synchronize()
    ctx.check_faults()
    step_ms = e0.elapsed_time(e1) / steps

    # layer 0's ops one by one (repeated launches; the K/V append rewrites the same slots)
    nd = batch.num_decode
    lw = dec.layers[0]
    normed, q, attn, act = dec.normed[:t], dec.q[:t], dec.attn[:t], dec.act[:t]
    # the projections' inputs as the step hands them over (bf16 bits)
    xin, ain = dec.normed16[:t], dec.attn16[:t]
    ops = {}
    s_qkv = ctx.gemm_bf16_splits(t, h, dec.nqkv)
    parts = dec._parts(t, dec.nqkv, s_qkv)
    ops["qkv_gemm"] = (timed(lambda: ctx.gemm_bf16(xin, lw["qkv"], h, dec.nqkv, s_qkv, parts), 10),
                       2.0 * t * h * dec.nqkv, "mfma")
    ops["qkv_rope_append"] = (timed(lambda: ctx.qkv_rope_append(
        parts, s_qkv, None, batch.positions, dec.cos, dec.sin, d, dec.max_pos, batch.slot_mapping,
        dec.k_pools[0], dec.v_pools[0], 1, num_blocks, bs, hq, hkv, d, q), 10), None, None)
    scale = 1.0 / d ** 0.5
    dec_bytes = sum(decode_ctx) * hkv * d * 2 * 2 + nd * hq * d * 8 + sum((c + bs - 1) // bs for c in decode_ctx) * 4
    ops["decode_attention"] = (timed(lambda: ctx.attn_decode_paged(
        q[:nd], dec.k_pools[0], dec.v_pools[0], 1, batch.dec_block_tables, batch.dec_context_lens,
        batch.dec_max_context, hkv, bs, num_blocks, scale, attn[:nd]), 10), dec_bytes, "hbm")
    pf_flops = sum(4.0 * hq * d * sum(range(p + 1, p + n + 1)) for p, n in prefill)
    ops["prefill_attention_bf16_mfma"] = (timed(lambda: ctx.attn_prefill_paged_bf16(
        q[nd:], dec.k_pools[0], dec.v_pools[0], batch.pf_block_tables, batch.pf_cu_seqlens,
        batch.pf_context_lens, batch.pf_max_query, hkv, bs, num_blocks, scale, attn[nd:]), 10),
        pf_flops, "mfma")
    ops["attn_out_to_bf16"] = (timed(lambda: ctx.convert_f32_to_bf16(attn, ain), 10), t * h * 6, "hbm")
    s_o = ctx.gemm_bf16_splits(t, h, h)
    parts = dec._parts(t, h, s_o)
    ops["wo_gemm"] = (timed(lambda: ctx.gemm_bf16(ain, lw["wo"], h, h, s_o, parts), 10),
                      2.0 * t * h * h, "mfma")
    ops["w13_swiglu_gemm"] = (timed(lambda: ctx.gemm_bf16_swiglu(xin, lw["w13"], h, f, act), 10),
                              4.0 * t * h * f, "mfma")
    s_w2 = ctx.gemm_bf16_splits(t, f, h)
    parts = dec._parts(t, h, s_w2)
    ops["w2_gemm"] = (timed(lambda: ctx.gemm_bf16(act, lw["w2"], f, h, s_w2, parts), 10),
                      2.0 * t * f * h, "mfma")
    r = int(batch.last_rows.numel())
    ops["lm_head_argmax"] = (timed(lambda: ctx.lm_head_argmax_bf16(dec.last16[:r], dec.lm_head, v, dec.tok[:r],
                                                                   dec.prob[:r]), 10), 2.0 * r * h * v, "mfma")
    ctx.check_faults()
    out_ops = {}
    for name, (ms, work, bound) in ops.items():
        row = {"avg_launch_us": round(ms * 1e3, 1)}
        if bound == "hbm":
            row.update(bytes_per_launch=int(work), achieved_gbs=round(work / (ms * 1e-3) / 1e9, 1),
                       hbm_frac=round(work / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        elif bound == "mfma":
            tf = work / (ms * 1e-3) / 1e12
            row.update(flops=work, achieved_tflops=round(tf, 1), bf16_mfma_frac=round(tf / BF16_PEAK_TFS, 4))
        elif bound == "mfma_f32":
            tf = work / (ms * 1e-3) / 1e12
            row.update(flops=work, achieved_tflops=round(tf, 1), f32_mfma_frac=round(tf / FP32_PEAK_TFS, 4))
        out_ops[name] = row
    res = {
        "workload": "C5 Llama-3-8B shape composed from the kernel ABI, bf16 weights (N(0,0.02), seeded), bf16 "
                    "activations (projection inputs rounded to bf16: bf16 x bf16 products with f32 accumulation, "
                    "where the reference multiplies f32 activations by bf16-widened weights) and bf16 KV; "
                    f"step = {nd} decode "
                    f"tokens (ctx U[512,8192], sum {sum(decode_ctx)}) + {sum(n for _, n in prefill)}-token "
                    "prefill chunk after a 2048-token cached prefix; 32 layers + greedy head; block 16",
        "kv_pool_gb": round(kv_bytes / 1e9, 1),
        "ms_per_step": round(step_ms, 3),
        "decode_tok_s": round(nd / (step_ms * 1e-3), 1),
        "step_tok_s": round(t / (step_ms * 1e-3), 1),
        "steps": steps,
        "layer0_ops": out_ops,
    }
    del dec, x, batch
    ctx.close()
    torch.cuda.empty_cache()
    return res


def c4_cpu_baseline(seed, threads):
    """The oracle's restatement of the reference (per-sequence sessions, its thread fan-out)
    on a fixed 64-sequence decode window: the first 64 C4 requests with prompts cut to 16 tokens
    (one prefill tick) and 2 new tokens each, so both decode ticks run at batch 64 like the GPU
    figure it sits next to; tok/s by the reference's definition (generated / decode-tick time)."""
    import oracle
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, c4_requests, run_continuous

    oracle.build()
    oracle.set_threads(threads)
    cfg = QWEN2_05B_C4
    model = oracle.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                         cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                         tie=True)
    model.set_weights(c4_weights(seed))
    reqs = c4_requests(seed=seed)[:64]
    for r in reqs:
        r["prompt"] = r["prompt"][:16]
        r["max_new_tokens"] = 2
        r["arrival_tick"] = 0
    rep = run_continuous(oracle.Scheduler(model, max_batch=64, max_seq=64), reqs)
    return {
        "value": round(rep["decode_tok_s"], 3),
        "unit": "decode tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": "C4 model, fixed 64-sequence decode window: the first 64 C4 requests with prompts "
                  f"cut to 16 tokens, 2 decode ticks at batch 64 ({rep['generated_tokens']} decode "
                  f"tokens over {rep['decode_ticks']} ticks); host {os.cpu_count()} cpus, "
                  f"{cpu_model()}",
        "avg_decode_batch": round(rep["avg_decode_batch"], 2),
        "prefill_tok_s": round(rep["prefill_tok_s"], 2),
    }


def main():
    args = parse_args()
    if args.pmc_copy_reference:
        pmc_copy_reference()
        return
    if args.gemm_shapes:
        gemm_shapes(args.seed)
        return
    if args.c4_layer_ops:
        c4_layer_ops(args.seed)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(no multi-GPU path exists in this build)",
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
        "data": "synthetic: N(0,1) Q/K/V from the reference sampler's xorshift64* (splitmix64-seeded "
                f"streams, Box-Muller), seed {args.seed}",
        "value_is": "C2 paged-attention op rate: 64 query tokens per fi_attn_decode_paged launch "
                    "(one layer's decode attention over the batch) / wall time per launch; the model-"
                    "level decode rate is c4_decode_tok_s_at_batch_64",
        "config": {
            "workload": "C2 paged decode attention (one layer's op): 64 ragged seqs, L~U[128,2048] "
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
            # the fastest pure read of C2's f32 K/V bytes measured on MI355X (read-only kernels,
            # per-kv-head chunks of <= 128 tokens, no arithmetic): the rate this access pattern allows
            "ceiling_frac": C2_F32_READ_CEILING_FRAC if args.kv_dtype == "f32" else None,
            "ceiling_source": "profiles/decode_c2_read_ceiling.md" if args.kv_dtype == "f32" else None,
        },
        "device": dict(info, host_cpu=cpu_model(), host_cpus=os.cpu_count()),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_reps)
    del q, kp, vp, bt, cl, out
    if not args.no_kernels:
        print("bench: C3 prefill/append and GEMM kernels", file=sys.stderr, flush=True)
        result["kernels"] = kernel_legs(ctx, args.seed)
    ctx.close()
    if not args.no_c4:
        print("bench: C4 continuous batching on the GPU runtime", file=sys.stderr, flush=True)
        keys = ("workload", "decode_tok_s", "decode_tok_s_at_batch_64", "ms_per_decode_tick_at_batch_64",
                "prefill_tok_s", "generated_tokens", "decode_tick_host_ms", "roofline_at_batch_64")
        variants = [v for v in args.c4_variants.split(",") if v]
        main_graph = "graph" in variants or "eager" not in variants
        result["c4"] = c4_continuous(args.seed, args.c4_requests, graph=main_graph)
        tokens = result["c4"].pop("_tokens")
        if main_graph and "eager" in variants:
            # the same requests with every decode tick enqueued launch by launch; greedy decode
            # from replayed graphs must generate exactly the eager run's ids
            eager = c4_continuous(args.seed, args.c4_requests, graph=False)
            result["c4"]["eager"] = {k: eager[k] for k in keys}
            differ = sum(1 for a, b in zip(tokens, eager["_tokens"]) if a != b)
            result["c4"]["graph_tokens_equal_eager"] = differ == 0 and len(tokens) == len(eager["_tokens"])
            result["c4"]["graph_eager_differing_requests"] = differ
            if differ:
                print(f"bench: C4 graph and eager runs differ on {differ} requests", file=sys.stderr, flush=True)
        if "ahead" in variants:
            # the same requests with each decode tick enqueued while the previous one runs
            # (stream overlap of host planning with the device); the ids must equal the serial run's
            ahead = c4_continuous(args.seed, args.c4_requests, graph=main_graph, run_ahead=True)
            result["c4"]["run_ahead"] = {k: ahead[k] for k in keys + ("run_ahead_counters",)}
            differ = sum(1 for a, b in zip(tokens, ahead["_tokens"]) if a != b)
            result["c4"]["run_ahead"]["tokens_equal_serial"] = differ == 0 and len(tokens) == len(ahead["_tokens"])
        if "sampled" in variants:
            # the same requests under the reference's chat_default sampler (sampler.rs:30-37):
            # logits head + device sampling in every tick
            sampled = c4_continuous(args.seed, args.c4_requests, sampler=(0.7, 20, 0.9, 42), graph=main_graph)
            result["c4"]["sampled_chat_default"] = {k: sampled[k] for k in keys}
            if "ahead" in variants:
                # the same sampled pass run ahead: each tick's sampler states continue on the
                # device; the ids must equal the serial sampled run's
                sa = c4_continuous(args.seed, args.c4_requests, sampler=(0.7, 20, 0.9, 42), graph=main_graph,
                                   run_ahead=True)
                result["c4"]["sampled_chat_default_run_ahead"] = {k: sa[k] for k in keys + ("run_ahead_counters",)}
                differ = sum(1 for a, b in zip(sampled["_tokens"], sa["_tokens"]) if a != b)
                result["c4"]["sampled_chat_default_run_ahead"]["tokens_equal_serial"] = (
                    differ == 0 and len(sampled["_tokens"]) == len(sa["_tokens"]))
        if "bf16" in variants:
            # bf16-stored projections and head (the storage of the real Qwen2.5-0.5B checkpoints)
            b16 = c4_continuous(args.seed, args.c4_requests, graph=main_graph, weight_dtype="bf16")
            result["c4"]["bf16_weights"] = {k: b16[k] for k in keys}
        result["c4_decode_tok_s_at_batch_64"] = result["c4"]["decode_tok_s_at_batch_64"]
        if not args.no_cpu_baseline:
            print("bench: C4 CPU baseline (oracle, declared subset)", file=sys.stderr, flush=True)
            result["c4"]["cpu_baseline"] = c4_cpu_baseline(args.seed, min(16, os.cpu_count() or 1))
    if not args.no_c5:
        print("bench: C5 bf16 decoder step", file=sys.stderr, flush=True)
        result["c5"] = c5_step(args.seed, args.c5_steps)
        if args.c5_runtime_ticks > 0:
            print("bench: C5 decode ticks through the runtime", file=sys.stderr, flush=True)
            result["c5"]["runtime_decode_tick"] = c5_runtime_decode(args.seed, args.c5_runtime_ticks)
    if args.hf_load:
        print("bench: hf checkpoint import", file=sys.stderr, flush=True)
        result["hf_load"] = hf_load(args.seed)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
