"""GPU parity of the packed-weight projection path against the CPU oracle:
weight pack + split-K MFMA GEMM (matmul_f32 / linear_f32_with_bias), the SwiGLU epilogue
(silu + mul of the up / gate projections), the greedy-head epilogue
(matmul_rhs_transposed_argmax_f32), the split-K consumer that adds bias and residual and
applies RMSNorm, and the QKV consumer that adds bias, applies RoPE and appends K/V to the
pool.  f32 tolerance 1e-5 normwise for products (only the summation order differs); RoPE
and the KV scatter are bit-exact against the standalone ops; greedy ids exact outside near
ties."""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


SHAPES = [  # (M, K, N, pack width): C4 decode / prefill shapes, C1 shapes, ragged tails
    (64, 896, 1152, 1), (64, 896, 896, 1), (64, 4864, 896, 1), (1, 896, 1152, 1),
    (37, 256, 688, 2), (64, 896, 4864, 2), (200, 896, 4864, 4), (1024, 896, 1152, 4),
    (5, 100, 50, 4), (17, 36, 20, 1), (3, 4, 1, 2), (64, 688, 256, 4),
    # pack width 32 (three-piece bf16 products on 32 x 32 tiles): the runtime's q|k|v, wo and
    # w2 at decode and prefill M, one- and two-slab workgroups, K and N tails
    (64, 896, 1152, 32), (64, 896, 896, 32), (64, 4864, 896, 32), (1, 896, 1152, 32),
    (1024, 896, 1152, 32), (1024, 896, 896, 32), (300, 4864, 896, 32), (33, 256, 688, 32),
    (5, 100, 50, 32), (17, 36, 20, 32), (3, 4, 1, 32),
]


def sum_splits(parts):
    """Split partials summed in split order, as the consumer kernels do."""
    acc = parts[0].copy()
    for z in range(1, parts.shape[0]):
        acc = acc + parts[z]
    return acc


@pytest.mark.parametrize("shape", SHAPES)
def test_packed_gemm_matches_linear(orc, gpu_ctx, shape):
    import torch

    m, k, n, pw = shape
    print(f"packed gemm shape={shape}", flush=True)
    rng = np.random.default_rng(m + 3 * k + 7 * n + pw)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float32)
    bp = gpu_ctx.weight_pack(dev(w), k, n, pw)
    splits = gpu_ctx.gemm_packed_splits(m, k, n, pw)
    # lda padded to a multiple of 4 as the kernel requires
    lda = (k + 3) // 4 * 4
    a_dev = torch.zeros((m, lda), device="cuda")
    a_dev[:, :k] = dev(a)
    out = torch.full((splits, m, n), float("nan"), device="cuda")
    gpu_ctx.gemm_packed(a_dev[:, :k], bp, k, n, pw, splits, out)
    torch.cuda.synchronize()
    got = sum_splits(out.cpu().numpy())
    ref = orc.linear_with_bias(a, w, None)
    assert normwise_error(got, ref) <= 1e-5, (shape, splits)


def test_packed_column_concatenation(orc, gpu_ctx):
    """The fused QKV pack (three [K, n_i] sources side by side) equals packing their
    concatenation."""
    import torch

    rng = np.random.default_rng(11)
    m, k = 40, 256
    parts = [(rng.standard_normal((k, n), dtype=np.float32) * 0.05).astype(np.float32)
             for n in (256, 64, 64)]
    for pw in (1, 2, 4, 32):
        bp = gpu_ctx.weight_pack_columns([dev(p) for p in parts], k, pw)
        ref_bp = gpu_ctx.weight_pack(dev(np.concatenate(parts, axis=1)), k, 384, pw)
        assert torch.equal(bp, ref_bp)
    a = rng.standard_normal((m, k), dtype=np.float32)
    ref = orc.linear_with_bias(a, np.concatenate(parts, axis=1), None)
    for pw in (1, 32):
        splits = gpu_ctx.gemm_packed_splits(m, k, 384, pw)
        out = torch.empty((splits, m, 384), device="cuda")
        bp = gpu_ctx.weight_pack_columns([dev(p) for p in parts], k, pw)
        gpu_ctx.gemm_packed(dev(a), bp, k, 384, pw, splits, out)
        torch.cuda.synchronize()
        assert normwise_error(sum_splits(out.cpu().numpy()), ref) <= 1e-5, pw


def test_packed_gemm_transposed_source_and_exact_integers(gpu_ctx):
    """Small integers make every product and partial sum exact, so the packed GEMM must equal
    numpy exactly (pins the fragment layout, the K tail and the [N, K] source path)."""
    import torch

    rng = np.random.default_rng(5)
    for m, k, n, pw in [(64, 64, 64, 4), (5, 20, 37, 2), (130, 96, 80, 1), (3, 1000, 68, 4),
                        (64, 64, 64, 32), (5, 20, 37, 32), (130, 96, 80, 32), (3, 1000, 68, 32),
                        (1024, 64, 512, 32)]:
        a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
        w = rng.integers(-4, 5, size=(k, n)).astype(np.float32)
        for layout, src in ((0, w), (1, np.ascontiguousarray(w.T))):
            bp = gpu_ctx.weight_pack(dev(src), k, n, pw, src_layout=layout)
            splits = gpu_ctx.gemm_packed_splits(m, k, n, pw)
            out = torch.empty((splits, m, n), device="cuda")
            gpu_ctx.gemm_packed(dev(a), bp, k, n, pw, splits, out)
            torch.cuda.synchronize()
            assert np.array_equal(sum_splits(out.cpu().numpy()), a @ w), (m, k, n, pw, layout)


@pytest.mark.parametrize("m,k,f,bias", [(64, 896, 4864, True), (7, 256, 688, False), (100, 64, 40, True),
                                         (9, 512, 1001, True)])
def test_packed_swiglu(orc, gpu_ctx, m, k, f, bias):
    """Even widths take the two-columns-a-thread split consumer, the odd one (split K, 4 splits)
    the one-column consumer."""
    import torch

    rng = np.random.default_rng(m + f)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w1 = (rng.standard_normal((k, f), dtype=np.float32) * 0.05).astype(np.float32)
    w3 = (rng.standard_normal((k, f), dtype=np.float32) * 0.05).astype(np.float32)
    b1 = rng.standard_normal(f, dtype=np.float32) if bias else None
    b3 = rng.standard_normal(f, dtype=np.float32) if bias else None
    bp = gpu_ctx.weight_pack_pair(dev(w1), dev(w3), k, f)
    out = torch.empty((m, f), device="cuda")
    gpu_ctx.gemm_packed_swiglu(dev(x), bp, k, f, out, dev(b1) if bias else None,
                               dev(b3) if bias else None)
    torch.cuda.synchronize()
    up = orc.linear_with_bias(x, w1, b1)
    gate = orc.linear_with_bias(x, w3, b3)
    ref = orc.mul(up, orc.silu(gate))
    assert normwise_error(out.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("m,h,v", [(1, 2, 3), (4, 256, 4096), (64, 896, 5000), (3, 64, 129), (64, 896, 151936)])
def test_packed_lm_head_argmax(orc, gpu_ctx, m, h, v):
    import torch

    print(f"packed lm_head m={m} h={h} v={v}", flush=True)
    rng = np.random.default_rng(h + v)
    hid = rng.standard_normal((m, h), dtype=np.float32)
    w = (rng.standard_normal((v, h), dtype=np.float32) * 0.05).astype(np.float32)
    lda = (h + 3) // 4 * 4
    hid_dev = torch.zeros((m, lda), device="cuda")
    hid_dev[:, :h] = dev(hid)
    bp = gpu_ctx.weight_pack(dev(w), h, v, 2, src_layout=1)
    tok = torch.empty(m, dtype=torch.int32, device="cuda")
    prob = torch.empty(m, device="cuda")
    gpu_ctx.lm_head_argmax_packed(hid_dev[:, :h], bp, v, tok, prob)
    torch.cuda.synchronize()
    logits = hid.astype(np.float64) @ w.T.astype(np.float64)
    for r in range(m):
        ridx, rprob = orc.matmul_rhs_transposed_argmax(hid[r:r + 1], w)
        top2 = np.sort(logits[r])[-2:] if v > 1 else None
        if top2 is not None and top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])):
            continue  # near tie: summation order may legitimately pick the other index
        assert int(tok[r]) == ridx, r
        assert abs(float(prob[r]) - rprob) <= 1e-4 * max(rprob, 1e-30) + 1e-7


def test_packed_lm_head_reference_vector_and_ties(gpu_ctx):
    """matmul.rs:745-758: lhs [1,2], rhs [[1,0],[0,1],[1,1]] -> (2, 0.66524094); equal logits
    across slabs and inside a lane vector keep the first index."""
    import torch

    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    prob = torch.empty(1, device="cuda")
    hid = torch.zeros((1, 4), device="cuda")
    hid[0, :2] = torch.tensor([1.0, 2.0])
    w = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    bp = gpu_ctx.weight_pack(dev(w), 2, 3, 2, src_layout=1)
    gpu_ctx.lm_head_argmax_packed(hid[:, :2], bp, 3, tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 2
    assert abs(float(prob[0]) - 0.66524094) <= 1e-6
    v, h = 300, 4
    w = np.zeros((v, h), np.float32)
    w[[70, 5, 200, 71, 6], 0] = 1.0  # max logit 1.0 at 5, 6, 70, 71, 200 -> first is 5
    bp = gpu_ctx.weight_pack(dev(w), h, v, 2, src_layout=1)
    hid = dev(np.array([[1, 0, 0, 0]], np.float32))
    gpu_ctx.lm_head_argmax_packed(hid, bp, v, tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 5


@pytest.mark.parametrize("rows,hidden,splits,bias", [(64, 896, 4, True), (3, 256, 1, False), (17, 4096, 3, True),
                                                     (5, 30, 2, True)])  # last: the scalar (hidden % 4) path
def test_splitk_residual_rms_norm(orc, gpu_ctx, rows, hidden, splits, bias):
    import torch

    rng = np.random.default_rng(rows + hidden)
    parts = rng.standard_normal((splits, rows, hidden), dtype=np.float32)
    b = rng.standard_normal(hidden, dtype=np.float32) if bias else None
    res = rng.standard_normal((rows, hidden), dtype=np.float32)
    w = rng.standard_normal(hidden, dtype=np.float32)
    s = torch.empty((rows, hidden), device="cuda")
    out = torch.empty((rows, hidden), device="cuda")
    gpu_ctx.splitk_residual_rms_norm(dev(parts), splits, dev(b) if bias else None, dev(res), s,
                                     dev(w), out, 1e-6)
    torch.cuda.synchronize()
    h = sum_splits(parts)
    if bias:
        h = h + b
    h = h + res
    assert np.array_equal(s.cpu().numpy(), h)  # same additions in the same order
    assert normwise_error(out.cpu().numpy(), orc.rms_norm(h, w, 1e-6)) <= 1e-5
    # bf16 output: the same sum, and exactly the nearest-even rounding of the f32 output
    s16 = torch.empty((rows, hidden), device="cuda")
    out16 = torch.empty((rows, hidden), dtype=torch.int16, device="cuda")
    gpu_ctx.splitk_residual_rms_norm(dev(parts), splits, dev(b) if bias else None, dev(res), s16,
                                     dev(w), out16, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(s16, s)
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), orc.f32_to_bf16(out.cpu().numpy()))


@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d,rot,splits", [(14, 2, 64, 64, 3), (8, 2, 32, 32, 1), (4, 2, 64, 32, 2),
                                                  (4, 2, 32, 6, 2)])  # last: scalar path (rot / 2 = 3)
def test_qkv_rope_append_matches_standalone_ops(gpu_ctx, kv, hq, hkv, d, rot, splits):
    """Fused consumer == split sum + bias, then fi_rope, then fi_kv_append, bit for bit."""
    import torch

    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    rng = np.random.default_rng(hq * d + splits)
    t, blocks, bs, max_pos = 37, 64, 16, 512
    width = (hq + 2 * hkv) * d
    parts = rng.standard_normal((splits, t, width), dtype=np.float32)
    bias = rng.standard_normal(width, dtype=np.float32)
    pos = rng.integers(0, max_pos, size=t).astype(np.int32)
    slots = rng.permutation(blocks * bs)[:t].astype(np.int64)
    slots[5] = -1  # skipped row
    cos_t = torch.empty((max_pos, rot // 2), device="cuda")
    sin_t = torch.empty((max_pos, rot // 2), device="cuda")
    gpu_ctx.rope_table(max_pos, d, rot, 1e6, cos_t, sin_t)
    dt = DTYPE_F32 if kv == "f32" else DTYPE_BF16
    tdt = torch.float32 if kv == "f32" else torch.int16
    pool = lambda: torch.zeros((blocks, hkv, bs, d), dtype=tdt, device="cuda")  # noqa: E731
    k1, v1, k2, v2 = pool(), pool(), pool(), pool()
    q1 = torch.empty((t, hq, d), device="cuda")
    qw, kw = hq * d, hkv * d
    biases = (dev(bias[:qw]), dev(bias[qw:qw + kw]), dev(bias[qw + kw:]))
    gpu_ctx.qkv_rope_append(dev(parts), splits, biases, dev(pos), cos_t, sin_t, rot, max_pos,
                            dev(slots), k1, v1, dt, blocks, bs, hq, hkv, d, q1)
    x = sum_splits(parts) + bias
    q2 = dev(x[:, :hq * d].reshape(t, hq, d))
    kk = dev(x[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d))
    vv = dev(x[:, (hq + hkv) * d:].reshape(t, hkv, d))
    gpu_ctx.rope(q2, kk, dev(pos), cos_t, sin_t, rot, max_pos)
    gpu_ctx.kv_append(kk, vv, dev(slots), k2, v2, dt, blocks, bs, hkv, d)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    assert torch.equal(q1, q2)
    assert torch.equal(k1, k2)
    assert torch.equal(v1, v2)
