"""GPU parity of paged decode attention and KV append against the CPU oracle.

The oracle runs the reference's paged decode exactly: gather the committed prefix by block
table, then cached-prefixed attention with the current token last
(runtime/reference.rs:497-508).  Tolerances: f32 outputs within 1e-4
normwise relative error, bf16-storage within 2e-2.
"""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2


def _dev(x, torch):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run_decode(ctx, wl, kv_dtype, torch):
    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    if kv_dtype == "bf16":
        import oracle

        kp = torch.from_numpy(oracle.f32_to_bf16(wl.k_pool).view(np.int16)).cuda()
        vp = torch.from_numpy(oracle.f32_to_bf16(wl.v_pool).view(np.int16)).cuda()
        dt = DTYPE_BF16
    else:
        kp, vp, dt = _dev(wl.k_pool, torch), _dev(wl.v_pool, torch), DTYPE_F32
    q = _dev(wl.q, torch)
    bt = _dev(wl.block_tables, torch)
    cl = _dev(wl.context_lens, torch)
    out = torch.empty_like(q)
    ctx.attn_decode_paged(q, kp, vp, dt, bt, cl, wl.max_context_len, wl.num_kv_heads,
                          wl.block_size, wl.num_blocks, wl.scale, out)
    torch.cuda.synchronize()
    ctx.check_faults()
    return out.cpu().numpy()


def oracle_decode(orc, wl, kv_dtype):
    k, v = wl.k_pool, wl.v_pool
    if kv_dtype == "bf16":
        k = orc.bf16_to_f32(orc.f32_to_bf16(k))
        v = orc.bf16_to_f32(orc.f32_to_bf16(v))
    return orc.paged_decode_gather_attention(wl.q, wl.pages_reference_layout(k),
                                             wl.pages_reference_layout(v), wl.block_tables,
                                             wl.context_lens, wl.block_size)


SMALL_CASES = [
    # (num_seqs, min_len, max_len, hq, hkv, d, block_size, num_blocks)
    (3, 1, 40, 4, 4, 32, 16, 64),      # L=1 possible, MHA
    (5, 200, 300, 8, 2, 32, 16, 128),  # crosses the 256-token partition
    (4, 250, 770, 14, 2, 64, 16, 256),  # Qwen2-shaped GQA 7
    (6, 1, 600, 8, 1, 64, 8, 512),      # group 8, block size 8
    (4, 500, 1100, 32, 8, 128, 16, 512),
    (2, 255, 258, 4, 2, 128, 32, 64),   # partition edges, block size 32
]


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", SMALL_CASES)
def test_decode_small_cases(orc, gpu_ctx, case, kv_dtype):
    import torch

    from ferrisinfer_amd.workloads import paged_decode_c2

    b, lo, hi, hq, hkv, d, bs, nb = case
    print(f"decode case={case} dtype={kv_dtype}", flush=True)
    wl = paged_decode_c2(seed=11, num_seqs=b, min_len=lo, max_len=hi, num_q_heads=hq,
                         num_kv_heads=hkv, head_dim=d, block_size=bs, num_blocks=nb)
    got = run_decode(gpu_ctx, wl, kv_dtype, torch)
    ref = oracle_decode(orc, wl, kv_dtype)
    err = normwise_error(got, ref)
    assert err <= (F32_TOL if kv_dtype == "f32" else BF16_TOL), err
    if kv_dtype == "bf16":
        # the oracle attends the same widened bf16 values, so only summation order differs
        assert err <= F32_TOL, err


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_decode_c2_full_size(orc, gpu_ctx, kv_dtype):
    """BASELINE config C2 at its full size: 64 ragged sequences, L ~ U[128, 2048]."""
    import torch

    from ferrisinfer_amd.workloads import paged_decode_c2

    print(f"decode C2 full dtype={kv_dtype}", flush=True)
    wl = paged_decode_c2(seed=0)
    got = run_decode(gpu_ctx, wl, kv_dtype, torch)
    ref = oracle_decode(orc, wl, kv_dtype)
    err = normwise_error(got, ref)
    assert err <= (F32_TOL if kv_dtype == "f32" else BF16_TOL), err


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_decode_c5_context_range(orc, gpu_ctx, kv_dtype):
    """BASELINE config C5's decode attention range: contexts up to 8192 (8 to 16 partitions of
    512 tokens through the split-KV merge), Hq 32 / Hkv 8 / D 128, 10 sequences."""
    import torch

    from ferrisinfer_amd.workloads import paged_decode_c2

    print(f"decode C5 context range dtype={kv_dtype}", flush=True)
    wl = paged_decode_c2(seed=7, num_seqs=10, min_len=4000, max_len=8192, num_blocks=5200)
    assert wl.max_context_len > 7680  # the longest sequence spans 16 partitions
    got = run_decode(gpu_ctx, wl, kv_dtype, torch)
    ref = oracle_decode(orc, wl, kv_dtype)
    err = normwise_error(got, ref)
    assert err <= F32_TOL, err  # bf16: the oracle attends the same widened values


def test_decode_batch_invariance(gpu_ctx):
    """A sequence's output does not depend on the batch around it (bit-identical)."""
    import torch

    from ferrisinfer_amd.workloads import paged_decode_c2

    wl = paged_decode_c2(seed=3, num_seqs=16, num_blocks=4096)
    full = run_decode(gpu_ctx, wl, "f32", torch)
    for i in (0, 7, 15):
        one = paged_decode_c2(seed=3, num_seqs=16, num_blocks=4096)
        one.q = wl.q[i:i + 1].copy()
        one.block_tables = wl.block_tables[i:i + 1].copy()
        one.context_lens = wl.context_lens[i:i + 1].copy()
        alone = run_decode(gpu_ctx, one, "f32", torch)
        assert np.array_equal(alone[0], full[i])


@pytest.mark.parametrize("shape", [(32, 8, 128), (14, 2, 64)])
def test_decode_split_merge_repeatable(gpu_ctx, shape):
    """Sequences spanning several partitions go through the split-KV partials and the merge
    kernel.  Thirty back-to-back launches sharing one workspace must give bit-identical
    outputs: the partition size depends only on the model shape and every summation order is
    fixed."""
    import torch

    from ferrisinfer_amd import DTYPE_F32
    from ferrisinfer_amd.workloads import paged_decode_c2

    hq, hkv, d = shape
    wl = paged_decode_c2(seed=5, num_seqs=48, min_len=600, max_len=2048, num_q_heads=hq,
                         num_kv_heads=hkv, head_dim=d, num_blocks=8192)
    kp, vp = _dev(wl.k_pool, torch), _dev(wl.v_pool, torch)
    q, bt, cl = _dev(wl.q, torch), _dev(wl.block_tables, torch), _dev(wl.context_lens, torch)
    outs = [torch.empty_like(q) for _ in range(30)]
    for o in outs:
        gpu_ctx.attn_decode_paged(q, kp, vp, DTYPE_F32, bt, cl, wl.max_context_len, hkv,
                                  wl.block_size, wl.num_blocks, wl.scale, o)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [
    (64, 1, 2300, 14, 2, 64),    # a C4 decode tick at batch 64: up to 9 partitions of 256 tokens
    (6, 600, 4096, 32, 8, 128),  # few long sequences at the C5 head shape: up to 8 of 512
])
def test_decode_in_kernel_merge_matches_merge_launch(orc, gpu_ctx, kv_dtype, shape):
    """Small launches (at most six workgroups a CU) merge the split-KV partials in the
    partition kernel's last-arriving workgroup, with device-coherent stores and loads and a
    per-(sequence, kv head) arrival counter.  The no-allocation entry point always merges in
    a separate launch: both must give bit-identical outputs, three launches in a row (the
    counters are reset by each launch's last arrivers), and match the oracle."""
    import torch

    import oracle
    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32
    from ferrisinfer_amd.workloads import paged_decode_c2

    n, lo, hi, hq, hkv, d = shape
    wl = paged_decode_c2(seed=31, num_seqs=n, min_len=lo, max_len=hi, num_q_heads=hq,
                         num_kv_heads=hkv, head_dim=d, num_blocks=12288)
    parts = -(-int(wl.max_context_len) // (256 if hkv * d < 512 else 512))
    assert parts > 1 and n * hkv * parts <= 6 * 256, "the shape must take the in-kernel merge"
    if kv_dtype == "bf16":
        kp = torch.from_numpy(oracle.f32_to_bf16(wl.k_pool).view(np.int16)).cuda()
        vp = torch.from_numpy(oracle.f32_to_bf16(wl.v_pool).view(np.int16)).cuda()
        dt = DTYPE_BF16
    else:
        kp, vp, dt = _dev(wl.k_pool, torch), _dev(wl.v_pool, torch), DTYPE_F32
    q, bt, cl = _dev(wl.q, torch), _dev(wl.block_tables, torch), _dev(wl.context_lens, torch)
    args = (wl.max_context_len, wl.num_kv_heads, wl.block_size, wl.num_blocks, wl.scale)
    sep = torch.full_like(q, float("nan"))
    gpu_ctx.attn_decode_paged_noalloc(q, kp, vp, dt, bt, cl, *args, sep)
    outs = [torch.full_like(q, float("nan")) for _ in range(3)]
    for o in outs:
        gpu_ctx.attn_decode_paged(q, kp, vp, dt, bt, cl, *args, o)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    for o in outs:
        assert torch.equal(o, sep)
    ref = oracle_decode(orc, wl, kv_dtype)
    assert normwise_error(outs[0].cpu().numpy(), ref) < (F32_TOL if kv_dtype == "f32" else BF16_TOL)


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("d,misaligned", [(64, False), (6, False), (64, True)])
def test_kv_append_scatter_exact(orc, gpu_ctx, kv_dtype, d, misaligned):
    """fi_kv_append writes each token row to block_id*bs+offset, bit-exact (bf16: RNE): the
    16-byte path (head dim a multiple of 4, aligned sources) and the element path (head dim 6,
    or sources one float off 16-byte alignment)."""
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    rng = np.random.default_rng(5)
    nb, bs, hkv, t = 64, 16, 4, 300
    slots = rng.permutation(nb * bs)[:t].astype(np.int64)
    slots[::37] = -1  # padding rows are skipped
    key = rng.standard_normal((t, hkv, d), dtype=np.float32)
    val = rng.standard_normal((t, hkv, d), dtype=np.float32)
    torch_dt = torch.float32 if kv_dtype == "f32" else torch.int16
    kc = torch.zeros((nb, hkv, bs, d), dtype=torch_dt, device="cuda")
    vc = torch.zeros_like(kc)

    def src(x):
        if not misaligned:
            return _dev(x, torch)
        buf = torch.empty(x.size + 1, dtype=torch.float32, device="cuda")
        view = buf[1:].view(x.shape)
        view.copy_(torch.from_numpy(x))
        return view

    gpu_ctx.kv_append(src(key), src(val), _dev(slots, torch), kc, vc,
                      DTYPE_F32 if kv_dtype == "f32" else DTYPE_BF16, nb, bs, hkv, d)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    exp_k = np.zeros((nb, hkv, bs, d), np.float32)
    exp_v = np.zeros_like(exp_k)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        exp_k[s // bs, :, s % bs, :] = key[i]
        exp_v[s // bs, :, s % bs, :] = val[i]
    if kv_dtype == "f32":
        assert np.array_equal(kc.cpu().numpy(), exp_k)
        assert np.array_equal(vc.cpu().numpy(), exp_v)
    else:
        assert np.array_equal(kc.cpu().numpy().view(np.uint16), orc.f32_to_bf16(exp_k))
        assert np.array_equal(vc.cpu().numpy().view(np.uint16), orc.f32_to_bf16(exp_v))


def test_kv_append_out_of_range_slot_reported(gpu_ctx):
    """A slot beyond the pool is skipped on device and reported as Runtime by the host."""
    import torch

    from ferrisinfer_amd import DTYPE_F32, FerrisError

    nb, bs, hkv, d = 4, 16, 2, 32
    kc = torch.zeros((nb, hkv, bs, d), device="cuda")
    vc = torch.zeros_like(kc)
    key = torch.ones((2, hkv, d), device="cuda")
    slots = torch.tensor([3, nb * bs + 5], dtype=torch.int64, device="cuda")
    gpu_ctx.kv_append(key, key, slots, kc, vc, DTYPE_F32, nb, bs, hkv, d)
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert e.value.kind == "Runtime"
    assert float(kc[0, :, 3].sum()) == hkv * d
    gpu_ctx.check_faults()  # flags were cleared


def test_decode_context_beyond_max_context_len_reported(gpu_ctx):
    """A context_lens entry beyond the partitions that max_context_len sizes is clamped to them
    on device (the block table covers it, so every read stays in the pool and the partials
    in their stripe) and reported as Runtime; the other sequences are unaffected."""
    import torch

    from ferrisinfer_amd import DTYPE_F32, FerrisError

    nb, bs, hkv, hq, d, max_len = 320, 16, 2, 4, 64, 600
    lens = [max_len, 5000]  # 5000 > 600 rounded up to whole partitions, for any partition size
    g = torch.Generator().manual_seed(11)
    kc = torch.randn((nb, hkv, bs, d), generator=g).cuda()
    vc = torch.randn((nb, hkv, bs, d), generator=g).cuda()
    q = torch.randn((2, hq, d), generator=g).cuda()
    max_blocks = (lens[1] + bs - 1) // bs
    bt = torch.arange(2 * max_blocks, dtype=torch.int32).reshape(2, max_blocks) % nb
    bt = bt.cuda()
    out = torch.empty_like(q)
    gpu_ctx.attn_decode_paged(q, kc, vc, DTYPE_F32, bt, torch.tensor(lens, dtype=torch.int32).cuda(),
                              max_len, hkv, bs, nb, d ** -0.5, out)
    torch.cuda.synchronize()
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert e.value.kind == "Runtime"
    assert "context length beyond max_context_len" in str(e.value)
    gpu_ctx.check_faults()  # flags were cleared
    assert torch.isfinite(out).all()
    solo = torch.empty_like(q[:1])
    gpu_ctx.attn_decode_paged(q[:1].contiguous(), kc, vc, DTYPE_F32, bt[:1].contiguous(),
                              torch.tensor(lens[:1], dtype=torch.int32).cuda(), max_len, hkv, bs,
                              nb, d ** -0.5, solo)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    assert torch.equal(out[0], solo[0])


def test_kv_copy_blocks(gpu_ctx):
    import torch

    from ferrisinfer_amd import DTYPE_F32

    nb, bs, hkv, d = 8, 16, 2, 64
    kc = torch.randn((nb, hkv, bs, d), device="cuda")
    vc = torch.randn((nb, hkv, bs, d), device="cuda")
    k0, v0 = kc.clone(), vc.clone()
    src = torch.tensor([1, 4], dtype=torch.int32, device="cuda")
    dst = torch.tensor([6, 2], dtype=torch.int32, device="cuda")
    cnt = torch.tensor([5, 16], dtype=torch.int32, device="cuda")
    gpu_ctx.kv_copy_blocks(kc, vc, DTYPE_F32, src, dst, cnt, nb, bs, hkv, d)
    torch.cuda.synchronize()
    exp_k, exp_v = k0.clone(), v0.clone()
    exp_k[6, :, :5] = k0[1, :, :5]
    exp_v[6, :, :5] = v0[1, :, :5]
    exp_k[2] = k0[4]
    exp_v[2] = v0[4]
    assert torch.equal(kc, exp_k) and torch.equal(vc, exp_v)


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("length,read", [(300, 300), (300, 113), (16, 16), (1, 1), (37, 0)])
def test_kv_gather_matches_read_prefix(orc, gpu_ctx, kv_dtype, length, read):
    """fi_kv_gather against the oracle's PagedKvCacheStorage::read_prefix_f32 (pages concatenated
    by block table, runtime/paged_kv.rs:769-791): a sequence of `length` rows written to the
    oracle's paged storage and, through the same block table mapped onto a permuted device
    pool, appended with fi_kv_append; the first `read` rows gathered back are bit-identical
    (bf16 pool: the oracle's rows rounded to nearest even and widened)."""
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    print(f"kv gather length={length} read={read} dtype={kv_dtype}", flush=True)
    rng = np.random.default_rng(length * 7 + read)
    hkv, d, bs, nb = 2, 64, 16, 64
    store = orc.PagedKvStorage(1, hkv, d, 1024, bs)
    key = rng.standard_normal((length, hkv, d), dtype=np.float32)
    val = rng.standard_normal((length, hkv, d), dtype=np.float32)
    store.write_sequence(0, 0, key, val)
    entries = store.block_table(0, length)
    perm = rng.permutation(nb).astype(np.int32)
    table = np.array([perm[block] for _, block, _, _ in entries], np.int32)
    slots = np.array([int(table[p // bs]) * bs + p % bs for p in range(length)], np.int64)
    dt = DTYPE_F32 if kv_dtype == "f32" else DTYPE_BF16
    tdt = torch.float32 if kv_dtype == "f32" else torch.int16
    kc = torch.zeros((nb, hkv, bs, d), dtype=tdt, device="cuda")
    vc = torch.zeros_like(kc)
    gpu_ctx.kv_append(_dev(key, torch), _dev(val, torch), _dev(slots, torch), kc, vc, dt, nb, bs, hkv, d)
    k_out = torch.full((max(read, 1), hkv, d), float("nan"), device="cuda")
    v_out = torch.full_like(k_out, float("nan"))
    gpu_ctx.kv_gather(kc, vc, dt, _dev(table, torch), read, nb, bs, hkv, d, k_out, v_out)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    if read == 0:
        assert torch.isnan(k_out).all() and torch.isnan(v_out).all()  # nothing written
        return
    ref_k, ref_v = store.read_prefix(0, read)
    if kv_dtype == "bf16":
        ref_k = orc.bf16_to_f32(orc.f32_to_bf16(ref_k))
        ref_v = orc.bf16_to_f32(orc.f32_to_bf16(ref_v))
    assert np.array_equal(k_out.cpu().numpy(), ref_k)
    assert np.array_equal(v_out.cpu().numpy(), ref_v)


def test_kv_gather_errors(gpu_ctx):
    """A length beyond the table's pages is Runtime before any launch (paged_kv.rs:303-308); a
    block id outside the pool gives zero rows and Runtime at the next fault check."""
    import torch

    from ferrisinfer_amd import DTYPE_F32, FerrisError

    nb, bs, hkv, d = 8, 16, 2, 32
    kc = torch.randn((nb, hkv, bs, d), device="cuda")
    vc = torch.randn((nb, hkv, bs, d), device="cuda")
    out_k = torch.zeros((40, hkv, d), device="cuda")
    out_v = torch.zeros_like(out_k)
    table = torch.tensor([3, 5], dtype=torch.int32, device="cuda")
    with pytest.raises(FerrisError) as e:
        gpu_ctx.kv_gather(kc, vc, DTYPE_F32, table, 33, nb, bs, hkv, d, out_k, out_v)
    assert e.value.kind == "Runtime" and "committed pages" in str(e.value)
    bad = torch.tensor([3, nb + 4, 1], dtype=torch.int32, device="cuda")
    gpu_ctx.kv_gather(kc, vc, DTYPE_F32, bad, 40, nb, bs, hkv, d, out_k, out_v)
    torch.cuda.synchronize()
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert e.value.kind == "Runtime"
    assert torch.equal(out_k[:16], kc[3].transpose(0, 1))
    assert not out_k[16:32].any() and not out_v[16:32].any()
    assert torch.equal(out_v[32:40], vc[1, :, :8].transpose(0, 1))


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", [
    # (num_seqs, min_len, max_len, hq, hkv, d, rotary_dims, splits, biases)
    (64, 1, 2300, 14, 2, 64, 64, 7, True),     # a C4 decode tick (Qwen2-0.5B heads, q/k/v biases)
    (6, 300, 3000, 32, 8, 128, 128, 3, False),  # C5 heads, no biases
    (9, 1, 700, 8, 2, 64, 32, 2, True),         # partial rotary (pass-through half), GQA 4
    (5, 1, 300, 8, 8, 32, 32, 1, True),         # MHA, D 32, one split
    (24, 1000, 3000, 8, 8, 32, 32, 2, True),    # 2304 workgroups: the two-kernel path
])
def test_decode_fused_qkv_matches_consumer_then_decode(gpu_ctx, kv_dtype, case):
    """fi_attn_decode_paged_qkv == fi_qkv_rope_append followed by fi_attn_decode_paged, bit for
    bit: the attention output and both pools (the new token's K/V rows appended at their
    slots).  The fused launch runs three times in a row: the appends write the same rows and
    the outputs repeat.  Launches of more than six workgroups a CU run the two kernels inside
    the entry point, with q_out between them (the last case)."""
    import torch

    import oracle
    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32
    from ferrisinfer_amd.workloads import paged_decode_c2

    n, lo, hi, hq, hkv, d, rot, splits, with_bias = case
    print(f"fused qkv decode case={case} dtype={kv_dtype}", flush=True)
    wl = paged_decode_c2(seed=41, num_seqs=n, min_len=lo, max_len=hi, num_q_heads=hq,
                         num_kv_heads=hkv, head_dim=d, num_blocks=12288 if d >= 64 else 4608)
    parts_n = -(-int(wl.max_context_len) // (256 if hkv * d < 512 else 512))
    two_kernel = n * hkv * parts_n > 6 * 256
    rng = np.random.default_rng(n * d + splits)
    width = (hq + 2 * hkv) * d
    parts = _dev(rng.standard_normal((splits, n, width), dtype=np.float32), torch)
    qw, kw = hq * d, hkv * d
    biases = None
    if with_bias:
        b = rng.standard_normal(width, dtype=np.float32)
        biases = (_dev(b[:qw], torch), _dev(b[qw:qw + kw], torch), _dev(b[qw + kw:], torch))
    ctxl = wl.context_lens.astype(np.int64)
    last = ctxl - 1  # the new token is each sequence's last key
    bs = wl.block_size
    slots = np.array([int(wl.block_tables[b, p // bs]) * bs + p % bs for b, p in enumerate(last)], np.int64)
    # RoPE positions: the last key's, except every third sequence (the kernel loads the table
    # rows at the last key's position first and again where the given position differs)
    pos = (last + np.where(np.arange(n) % 3 == 2, 5, 0)).astype(np.int32)
    max_pos = int(pos.max()) + 1
    cos_t = torch.empty((max_pos, max(rot // 2, 1)), device="cuda")
    sin_t = torch.empty_like(cos_t)
    gpu_ctx.rope_table(max_pos, d, rot, 1e6, cos_t, sin_t)
    if kv_dtype == "bf16":
        k0 = torch.from_numpy(oracle.f32_to_bf16(wl.k_pool).view(np.int16)).cuda()
        v0 = torch.from_numpy(oracle.f32_to_bf16(wl.v_pool).view(np.int16)).cuda()
        dt = DTYPE_BF16
    else:
        k0, v0, dt = _dev(wl.k_pool, torch), _dev(wl.v_pool, torch), DTYPE_F32
    bt, cl = _dev(wl.block_tables, torch), _dev(wl.context_lens, torch)
    dpos, dslots = _dev(pos, torch), _dev(slots, torch)
    # the two separate launches
    k1, v1 = k0.clone(), v0.clone()
    q1 = torch.empty((n, hq, d), device="cuda")
    gpu_ctx.qkv_rope_append(parts, splits, biases, dpos, cos_t, sin_t, rot, max_pos, dslots, k1, v1, dt,
                            wl.num_blocks, bs, hq, hkv, d, q1)
    out1 = torch.full((n, hq, d), float("nan"), device="cuda")
    gpu_ctx.attn_decode_paged(q1, k1, v1, dt, bt, cl, wl.max_context_len, hkv, bs, wl.num_blocks, wl.scale, out1)
    # the fused launch
    k2, v2 = k0.clone(), v0.clone()
    q2 = torch.full((n, hq, d), float("nan"), device="cuda")
    outs = [torch.full((n, hq, d), float("nan"), device="cuda") for _ in range(3)]
    for o in outs:
        gpu_ctx.attn_decode_paged_qkv(parts, splits, biases, dpos, cos_t, sin_t, rot, max_pos, dslots, k2, v2,
                                      dt, bt, cl, wl.max_context_len, hq, hkv, d, bs, wl.num_blocks, wl.scale, o,
                                      q_out=q2)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    assert not torch.equal(k1, k0)  # the appends happened
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    for o in outs:
        assert torch.equal(o, out1)
    if two_kernel:
        assert torch.equal(q2, q1)
    else:
        assert torch.isnan(q2).all()  # the fused kernel leaves q_out unwritten
