"""GPU parity of KV append + varlen causal prefill attention over the paged pool against the
CPU oracle's cached-prefixed attention (the reference's prefill with a cached prefix,
runtime/reference.rs:425-465).  f32: 1e-4 normwise; bf16 KV: 2e-2 (here also 1e-4, since
the oracle attends the same widened bf16 values)."""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu


def run_prefill(ctx, wl, kv_dtype, bf16_mfma=False):
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    dt = DTYPE_F32 if kv_dtype == "f32" else DTYPE_BF16
    tdt = torch.float32 if kv_dtype == "f32" else torch.int16
    shape = (wl.num_blocks, wl.num_kv_heads, wl.block_size, wl.head_dim)
    kp = torch.zeros(shape, dtype=tdt, device="cuda")
    vp = torch.zeros(shape, dtype=tdt, device="cuda")
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    ctx.kv_append(d(wl.k_new), d(wl.v_new), d(wl.slot_mapping), kp, vp, dt, wl.num_blocks,
                  wl.block_size, wl.num_kv_heads, wl.head_dim)
    q = d(wl.q)
    out = torch.empty_like(q)
    if bf16_mfma:
        ctx.attn_prefill_paged_bf16(q, kp, vp, d(wl.block_tables), d(wl.cu_seqlens),
                                    d(wl.context_lens), int(wl.query_lens.max()), wl.num_kv_heads,
                                    wl.block_size, wl.num_blocks, wl.scale, out)
    else:
        ctx.attn_prefill_paged(q, kp, vp, dt, d(wl.block_tables), d(wl.cu_seqlens),
                               d(wl.context_lens), int(wl.query_lens.max()), wl.num_kv_heads,
                               wl.block_size, wl.num_blocks, wl.scale, out)
    torch.cuda.synchronize()
    ctx.check_faults()
    return out.cpu().numpy()


def oracle_prefill(orc, wl, kv_dtype):
    outs = []
    for b in range(len(wl.context_lens)):
        k, v = wl.full_kv(b)
        if kv_dtype == "bf16":
            k = orc.bf16_to_f32(orc.f32_to_bf16(k))
            v = orc.bf16_to_f32(orc.f32_to_bf16(v))
        start = int(wl.context_lens[b]) - int(wl.query_lens[b])
        qb = wl.q[wl.cu_seqlens[b]:wl.cu_seqlens[b + 1]]
        outs.append(orc.cached_prefixed_causal_attention(qb, k[:start], v[:start], start,
                                                         k[start:], v[start:]))
    return np.concatenate(outs)


CASES = [
    # (num_seqs, min_len, max_len, groups, group_size, shared, hq, hkv, d, bs)
    (4, 1, 70, 0, 1, 0, 4, 4, 32, 16),        # no prefix, tiny, includes 1-token prompts
    (8, 20, 200, 2, 4, 64, 8, 2, 32, 16),     # C1-shaped heads, block-shared prefixes
    (6, 30, 300, 2, 3, 128, 14, 2, 64, 16),   # Qwen2-shaped GQA 7
    (4, 100, 400, 1, 4, 96, 32, 8, 128, 8),   # block size 8
    (3, 1, 150, 0, 1, 0, 4, 2, 128, 32),      # GQA 2, block size 32, 1-token prompts
    # grids large enough for two row groups a wave (the launch picks them when every CU gets
    # two workgroups): Qwen2-shaped GQA 7 at D 64, C1-shaped heads at D 32
    (32, 200, 300, 2, 4, 96, 14, 2, 64, 16),
    (48, 150, 200, 0, 1, 0, 8, 2, 32, 16),
]


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", CASES)
def test_prefill_small(orc, gpu_ctx, case, kv_dtype):
    from ferrisinfer_amd.workloads import prefill_c3

    b, lo, hi, g, gs, sh, hq, hkv, d, bs = case
    print(f"prefill case={case} dtype={kv_dtype}", flush=True)
    wl = prefill_c3(seed=5, num_seqs=b, min_len=lo, max_len=hi, groups=g, group_size=gs,
                    shared_prefix=sh, num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                    block_size=bs, num_blocks=1024)
    got = run_prefill(gpu_ctx, wl, kv_dtype)
    err = normwise_error(got, oracle_prefill(orc, wl, kv_dtype))
    assert err <= 1e-4, err


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_prefill_c3_full_size(orc, gpu_ctx, kv_dtype):
    """16 seqs, L ~ U[32, 1024], 4 groups of 4 sharing 512-token
    prefixes by block id, Hq 32 / Hkv 8, D 128."""
    from ferrisinfer_amd.workloads import prefill_c3

    print(f"prefill C3 full dtype={kv_dtype}", flush=True)
    wl = prefill_c3(seed=0)
    assert (wl.shared_lens > 0).sum() >= 8  # the shared-prefix path is exercised
    got = run_prefill(gpu_ctx, wl, kv_dtype)
    err = normwise_error(got, oracle_prefill(orc, wl, kv_dtype))
    assert err <= (1e-4 if kv_dtype == "f32" else 2e-2), err


@pytest.mark.parametrize("case", CASES)
def test_prefill_bf16_mfma_small(orc, gpu_ctx, case):
    """fi_attn_prefill_paged_bf16 (bf16 MFMA, Q and P rounded to bf16) on a bf16 pool: within
    the bf16-storage bound of the oracle, and within 5e-3 of the f32-math kernel on the same
    pool (the rounding of Q and of the probabilities is the only difference)."""
    from ferrisinfer_amd.workloads import prefill_c3

    b, lo, hi, g, gs, sh, hq, hkv, d, bs = case
    print(f"prefill bf16 mfma case={case}", flush=True)
    wl = prefill_c3(seed=5, num_seqs=b, min_len=lo, max_len=hi, groups=g, group_size=gs,
                    shared_prefix=sh, num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                    block_size=bs, num_blocks=1024)
    got = run_prefill(gpu_ctx, wl, "bf16", bf16_mfma=True)
    f32_math = run_prefill(gpu_ctx, wl, "bf16")
    assert normwise_error(got, f32_math) <= 5e-3
    assert normwise_error(got, oracle_prefill(orc, wl, "bf16")) <= 2e-2


def test_prefill_bf16_mfma_rising_scores(orc, gpu_ctx):
    """Keys whose norms grow along the sequence (row i scaled by 1 + i / 16), so the row maxima
    rise chunk after chunk by far more than the kernel's exponent headroom (8 in log2 units):
    the reference point moves and the accumulators are rescaled on most chunks.  Compared with
    the f64 closed form on the kernel's own operands (Q rounded to bf16, bf16-stored K/V), which
    leaves the bf16 rounding of the probabilities and the summation order: 5e-3.  (Against
    unrounded Q the scores here, up to ~40, move by ~0.08 with Q's rounding.)"""
    from ferrisinfer_amd.workloads import prefill_c3

    print("prefill bf16 mfma rising scores", flush=True)
    wl = prefill_c3(seed=7, num_seqs=3, min_len=300, max_len=600, groups=0, group_size=1,
                    shared_prefix=0, num_q_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
                    num_blocks=1024)
    for b in range(len(wl.context_lens)):
        lo, hi = int(wl.cu_seqlens[b]), int(wl.cu_seqlens[b + 1])
        wl.k_new[lo:hi] *= (1.0 + np.arange(hi - lo, dtype=np.float32) / 16.0)[:, None, None]
    got = run_prefill(gpu_ctx, wl, "bf16", bf16_mfma=True)
    assert np.isfinite(got).all()
    rb = lambda x: orc.bf16_to_f32(orc.f32_to_bf16(x)).astype(np.float64)  # noqa: E731
    group = wl.num_q_heads // wl.num_kv_heads
    ref = np.empty(got.shape, np.float64)
    for b in range(len(wl.context_lens)):
        lo, hi = int(wl.cu_seqlens[b]), int(wl.cu_seqlens[b + 1])
        n = hi - lo
        q, k, v = rb(wl.q[lo:hi]), rb(wl.k_new[lo:hi]), rb(wl.v_new[lo:hi])
        causal = np.tril(np.ones((n, n), bool))
        for h in range(wl.num_q_heads):
            s = q[:, h] @ k[:, h // group].T * wl.scale
            s = np.where(causal, s, -np.inf)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            ref[lo:hi, h] = (p / p.sum(axis=1, keepdims=True)) @ v[:, h // group]
    assert normwise_error(got, ref) <= 5e-3


def rise_keys(wl, step):
    """Scale each key row by 1 + position / step (position within its sequence; a shared
    prefix is scaled where its source computes it), so scores grow along the sequence."""
    for b in range(len(wl.context_lens)):
        lo, hi = int(wl.cu_seqlens[b]), int(wl.cu_seqlens[b + 1])
        pos = int(wl.shared_lens[b]) + np.arange(hi - lo, dtype=np.float32)
        wl.k_new[lo:hi] *= (1.0 + pos / np.float32(step))[:, None, None]


def lazy_point_moves(wl, chunk=32, headroom=8.0):
    """Host replay of the f32-pool prefill kernel's exponent reference point: keys in chunks of
    `chunk` from position 0, the point set by the first chunk and moved only when a later
    chunk's maximum score (log2 units) passes it by more than `headroom`; every move after the
    first chunk rescales the accumulators by alpha in (0, 1).  Returns the fraction of (query
    row, head) pairs whose point moves at least once after the first chunk."""
    c2 = wl.scale * np.log2(np.e)
    group = wl.num_q_heads // wl.num_kv_heads
    moved = total = 0
    for b in range(len(wl.context_lens)):
        k, _ = wl.full_kv(b)
        lo, hi = int(wl.cu_seqlens[b]), int(wl.cu_seqlens[b + 1])
        start = int(wl.context_lens[b]) - (hi - lo)
        n = int(wl.context_lens[b])
        nch = (n + chunk - 1) // chunk
        for h in range(wl.num_q_heads):
            s = (wl.q[lo:hi, h].astype(np.float64) @ k[:, h // group].astype(np.float64).T) * c2
            s[np.arange(n)[None, :] > (start + np.arange(hi - lo))[:, None]] = -np.inf
            pad = np.full((hi - lo, nch * chunk), -np.inf)
            pad[:, :n] = s
            cmax = pad.reshape(hi - lo, nch, chunk).max(axis=2)
            m = cmax[:, 0].copy()
            any_move = np.zeros(hi - lo, bool)
            for c in range(1, nch):
                mv = cmax[:, c] > m + headroom
                any_move |= mv
                m = np.where(mv, cmax[:, c], m)
            moved += int(any_move.sum())
            total += hi - lo
    return moved / total


RISING_CASES = [
    # (num_seqs, min_len, max_len, groups, group_size, shared, hq, hkv, d, step)
    (3, 300, 600, 0, 1, 0, 8, 2, 64, 16),           # GQA 4, D 64, no prefix
    (4, 1500, 1600, 1, 4, 512, 14, 2, 64, 64),      # Qwen2 heads: ~1000-token prompts after a shared 512
    (32, 200, 300, 2, 4, 96, 14, 2, 64, 16),        # GQA 7 at D 64 with two row groups a wave
    (4, 300, 500, 1, 4, 128, 32, 8, 128, 16),       # C2/C3 heads at D 128
]


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", RISING_CASES)
def test_prefill_rising_scores(orc, gpu_ctx, case, kv_dtype):
    """fi_attn_prefill_paged with keys whose norms grow along the sequence, so later chunks'
    maxima pass the running reference point and the accumulators are rescaled (the
    s > m branch of the reference's online softmax, kernel/cpu/attention.rs:1125-1149).  The f32
    pool runs the three-piece kernel, whose point moves lazily (asserted to move on the host);
    the bf16 pool runs the f32-math kernel on widened values.  Both within 1e-4 of the oracle's
    cached-prefixed attention and of the f64 closed form on the same stored values."""
    from ferrisinfer_amd.workloads import prefill_c3

    b, lo, hi, g, gs, sh, hq, hkv, d, step = case
    print(f"prefill rising scores case={case} dtype={kv_dtype}", flush=True)
    wl = prefill_c3(seed=7, num_seqs=b, min_len=lo, max_len=hi, groups=g, group_size=gs,
                    shared_prefix=sh, num_q_heads=hq, num_kv_heads=hkv, head_dim=d, block_size=16,
                    num_blocks=1024)
    rise_keys(wl, step)
    assert lazy_point_moves(wl) >= 0.5
    got = run_prefill(gpu_ctx, wl, kv_dtype)
    assert np.isfinite(got).all()
    assert normwise_error(got, oracle_prefill(orc, wl, kv_dtype)) <= 1e-4
    rb = (lambda x: orc.bf16_to_f32(orc.f32_to_bf16(x))) if kv_dtype == "bf16" else (lambda x: x)
    ref = np.empty(got.shape, np.float64)
    for s in range(len(wl.context_lens)):
        k, v = wl.full_kv(s)
        r0, r1 = int(wl.cu_seqlens[s]), int(wl.cu_seqlens[s + 1])
        ref[r0:r1] = brute_force_f64(wl.q[r0:r1], rb(k), rb(v), int(wl.context_lens[s]) - (r1 - r0))
    assert normwise_error(got, ref) <= 1e-4


def test_prefill_bf16_mfma_c3_full_size(orc, gpu_ctx):
    from ferrisinfer_amd.workloads import prefill_c3

    print("prefill bf16 mfma C3 full", flush=True)
    wl = prefill_c3(seed=0)
    got = run_prefill(gpu_ctx, wl, "bf16", bf16_mfma=True)
    f32_math = run_prefill(gpu_ctx, wl, "bf16")
    assert normwise_error(got, f32_math) <= 5e-3
    assert normwise_error(got, oracle_prefill(orc, wl, "bf16")) <= 2e-2


def test_prefill_one_token_matches_decode(gpu_ctx):
    """A 1-token prefill chunk is a decode step: both kernels agree within f32 rounding."""
    import torch

    from ferrisinfer_amd import DTYPE_F32
    from ferrisinfer_amd.workloads import paged_decode_c2

    wl = paged_decode_c2(seed=4, num_seqs=8, min_len=1, max_len=900, num_blocks=512)
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    kp, vp, q = d(wl.k_pool), d(wl.v_pool), d(wl.q)
    bt, cl = d(wl.block_tables), d(wl.context_lens)
    out_d = torch.empty_like(q)
    out_p = torch.empty_like(q)
    gpu_ctx.attn_decode_paged(q, kp, vp, DTYPE_F32, bt, cl, wl.max_context_len, wl.num_kv_heads,
                              wl.block_size, wl.num_blocks, wl.scale, out_d)
    cu = d(np.arange(wl.num_seqs + 1, dtype=np.int32))
    gpu_ctx.attn_prefill_paged(q, kp, vp, DTYPE_F32, bt, cu, cl, 1, wl.num_kv_heads,
                               wl.block_size, wl.num_blocks, wl.scale, out_p)
    torch.cuda.synchronize()
    assert normwise_error(out_p.cpu().numpy(), out_d.cpu().numpy()) <= 1e-5


def brute_force_f64(q, k, v, start):
    """f64 causal attention of the rows of q at positions start + t over keys [0, start + t]
    (the closed form the oracle is pinned to in tests/test_oracle_invariants.py)."""
    t, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((t, hq, d), np.float64)
    n = start + t
    mask = np.arange(n)[None, :] > (start + np.arange(t))[:, None]
    for kv in range(hkv):
        qg = q[:, kv * g:(kv + 1) * g].astype(np.float64).transpose(1, 0, 2)  # [g, t, d]
        s = qg @ k[:n, kv].astype(np.float64).T / np.sqrt(d)                   # [g, t, n]
        s[:, mask] = -np.inf
        s -= s.max(axis=2, keepdims=True)
        w = np.exp(s)
        w /= w.sum(axis=2, keepdims=True)
        out[:, kv * g:(kv + 1) * g] = (w @ v[:n, kv].astype(np.float64)).transpose(1, 0, 2)
    return out


def test_prefill_c5_chunk_after_cached_prefix(orc, gpu_ctx):
    """BASELINE config C5's prefill chunk: 2048 new tokens after a 2048-token cached prefix
    (Hq 32 / Hkv 8 / D 128), batched with a ragged 37-token chunk after 1500 cached tokens, on
    f32 and bf16 pools through fi_attn_prefill_paged and fi_attn_prefill_paged_bf16.  Every row
    is compared with the f64 closed form (1e-4 f32, 2e-2 bf16 storage) and the first and last 16
    rows of the long chunk with the oracle's cached-prefixed attention."""
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    print("prefill C5 chunk 2048 after 2048", flush=True)
    rng = np.random.default_rng(55)
    hq, hkv, d, bs = 32, 8, 128, 16
    ctx_lens = np.array([4096, 1537], np.int32)
    qlens = np.array([2048, 37], np.int32)
    nblk = (ctx_lens + bs - 1) // bs
    num_blocks = 512
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.zeros((2, nblk.max()), np.int32)
    tables[0, :nblk[0]] = perm[:nblk[0]]
    tables[1, :nblk[1]] = perm[nblk[0]:nblk[0] + nblk[1]]
    k_seq = [rng.standard_normal((L, hkv, d), dtype=np.float32) for L in ctx_lens]
    v_seq = [rng.standard_normal((L, hkv, d), dtype=np.float32) for L in ctx_lens]
    q = rng.standard_normal((int(qlens.sum()), hq, d), dtype=np.float32)
    cu = np.array([0, qlens[0], qlens.sum()], np.int32)
    scale = float(1.0 / np.sqrt(np.float32(d)))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    for kv_dtype in ("f32", "bf16"):
        pool_k = np.zeros((num_blocks, hkv, bs, d), np.float32)
        pool_v = np.zeros_like(pool_k)
        ks, vs = [], []
        for b in range(2):
            kb, vb = k_seq[b], v_seq[b]
            if kv_dtype == "bf16":
                kb = orc.bf16_to_f32(orc.f32_to_bf16(kb))
                vb = orc.bf16_to_f32(orc.f32_to_bf16(vb))
            ks.append(kb)
            vs.append(vb)
            for p in range(int(ctx_lens[b])):
                pool_k[tables[b, p // bs], :, p % bs] = kb[p]
                pool_v[tables[b, p // bs], :, p % bs] = vb[p]
        if kv_dtype == "f32":
            kp, vp, dt = dev(pool_k), dev(pool_v), DTYPE_F32
        else:
            kp = dev(orc.f32_to_bf16(pool_k).view(np.int16))
            vp = dev(orc.f32_to_bf16(pool_v).view(np.int16))
            dt = DTYPE_BF16
        refs = [brute_force_f64(q[cu[b]:cu[b + 1]], ks[b], vs[b], int(ctx_lens[b] - qlens[b]))
                for b in range(2)]
        ref = np.concatenate(refs)
        qd, out = dev(q), torch.empty((q.shape[0], hq, d), device="cuda")
        gpu_ctx.attn_prefill_paged(qd, kp, vp, dt, dev(tables), dev(cu), dev(ctx_lens),
                                   int(qlens.max()), hkv, bs, num_blocks, scale, out)
        torch.cuda.synchronize()
        gpu_ctx.check_faults()
        got = out.cpu().numpy()
        assert normwise_error(got, ref) <= 1e-4, (kv_dtype, normwise_error(got, ref))
        start = int(ctx_lens[0] - qlens[0])
        for r0 in (0, int(qlens[0]) - 16):
            o = orc.cached_prefixed_causal_attention(q[r0:r0 + 16], ks[0][:start + r0], vs[0][:start + r0],
                                                     start + r0, ks[0][start + r0:start + r0 + 16],
                                                     vs[0][start + r0:start + r0 + 16])
            assert normwise_error(got[r0:r0 + 16], o) <= 1e-4
        if kv_dtype == "bf16":
            gpu_ctx.attn_prefill_paged_bf16(qd, kp, vp, dev(tables), dev(cu), dev(ctx_lens),
                                            int(qlens.max()), hkv, bs, num_blocks, scale, out)
            torch.cuda.synchronize()
            gpu_ctx.check_faults()
            got16 = out.cpu().numpy()
            assert normwise_error(got16, ref) <= 2e-2
            assert normwise_error(got16, got) <= 5e-3


@pytest.mark.parametrize("prefixes,qlen", [((256, 768, 1280, 1792), 256), ((1536,), 256), ((0, 40, 1000), 130)])
def test_prefill_key_splits_small_launch(orc, gpu_ctx, prefixes, qlen):
    """A C4-shaped prefill tick (Qwen2 heads 14/2, D 64) on an f32 pool: so few (tile, kv head)
    workgroups that the launch splits each tile's key chunks over up to four workgroups and
    merges their partials.  Rows whose keys all lie in later splits, splits with no chunk and
    a chunk with no prefix are included.  Every row against the f64 closed form and the first
    and last rows of each chunk against the oracle's cached-prefixed attention, at 1e-4."""
    import torch

    from ferrisinfer_amd import DTYPE_F32

    print(f"prefill key splits prefixes={prefixes} qlen={qlen}", flush=True)
    rng = np.random.default_rng(61)
    hq, hkv, d, bs = 14, 2, 64, 16
    n = len(prefixes)
    ctx_lens = np.array([p + qlen for p in prefixes], np.int32)
    qlens = np.full(n, qlen, np.int32)
    nblk = (ctx_lens + bs - 1) // bs
    num_blocks = int(nblk.sum()) + 8
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.zeros((n, nblk.max()), np.int32)
    o = 0
    for b in range(n):
        tables[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    ks = [rng.standard_normal((L, hkv, d), dtype=np.float32) for L in ctx_lens]
    vs = [rng.standard_normal((L, hkv, d), dtype=np.float32) for L in ctx_lens]
    pool_k = np.zeros((num_blocks, hkv, bs, d), np.float32)
    pool_v = np.zeros_like(pool_k)
    for b in range(n):
        for p in range(int(ctx_lens[b])):
            pool_k[tables[b, p // bs], :, p % bs] = ks[b][p]
            pool_v[tables[b, p // bs], :, p % bs] = vs[b][p]
    q = rng.standard_normal((int(qlens.sum()), hq, d), dtype=np.float32)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    scale = float(1.0 / np.sqrt(np.float32(d)))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    out = torch.empty((q.shape[0], hq, d), device="cuda")
    gpu_ctx.attn_prefill_paged(dev(q), dev(pool_k), dev(pool_v), DTYPE_F32, dev(tables), dev(cu), dev(ctx_lens),
                               qlen, hkv, bs, num_blocks, scale, out)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    got = out.cpu().numpy()
    ref = np.concatenate([brute_force_f64(q[cu[b]:cu[b + 1]], ks[b], vs[b], int(prefixes[b])) for b in range(n)])
    assert normwise_error(got, ref) <= 1e-4, normwise_error(got, ref)
    for b in range(n):
        start = int(prefixes[b])
        for r0 in (0, qlen - 8):
            rows = slice(int(cu[b]) + r0, int(cu[b]) + r0 + 8)
            ref_o = orc.cached_prefixed_causal_attention(q[rows], ks[b][:start + r0], vs[b][:start + r0], start + r0,
                                                         ks[b][start + r0:start + r0 + 8],
                                                         vs[b][start + r0:start + r0 + 8])
            assert normwise_error(got[rows], ref_o) <= 1e-4


def test_prefill_query_beyond_max_query_len_reported(gpu_ctx):
    """A cu_seqlens entry longer than max_query_len: the tiles max_query_len sized are computed,
    the sequence's rows past them are not, and the host gets Runtime with its own message; the
    other sequence is unaffected."""
    import torch

    from ferrisinfer_amd import DTYPE_F32, FerrisError

    nb, bs, hkv, hq, d = 64, 16, 2, 4, 64
    g = torch.Generator().manual_seed(3)
    kc = torch.randn((nb, hkv, bs, d), generator=g).cuda()
    vc = torch.randn((nb, hkv, bs, d), generator=g).cuda()
    qlens = [20, 300]  # the second exceeds max_query_len = 20 by more than any tile size
    q = torch.randn((sum(qlens), hq, d), generator=g).cuda()
    cu = torch.tensor([0, 20, 320], dtype=torch.int32).cuda()
    ctxl = torch.tensor([20, 300], dtype=torch.int32).cuda()
    bt = torch.arange(2 * 20, dtype=torch.int32).reshape(2, 20).cuda()
    out = torch.zeros_like(q)
    gpu_ctx.attn_prefill_paged(q, kc, vc, DTYPE_F32, bt, cu, ctxl, 20, hkv, bs, nb, d ** -0.5, out)
    torch.cuda.synchronize()
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert e.value.kind == "Runtime" and "max_query_len" in str(e.value)
    gpu_ctx.check_faults()  # flags were cleared
    solo = torch.zeros_like(q[:20])
    gpu_ctx.attn_prefill_paged(q[:20].contiguous(), kc, vc, DTYPE_F32, bt[:1].contiguous(), cu[:2].contiguous(),
                               ctxl[:1].contiguous(), 20, hkv, bs, nb, d ** -0.5, solo)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    assert torch.equal(out[:20], solo)
