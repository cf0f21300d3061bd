"""GPU parity of the bf16-weight projection path (bf16 configurations, e.g. C5 Llama-3-8B).

Two checks per op:
* tight: against the oracle's linear_f32_with_bias / SwiGLU / greedy head evaluated on the
  bf16-rounded operands (activations rounded to nearest even, weights widened exactly).  A
  product of two bf16 values is exact in f32, so only the summation order differs: 1e-5
  normwise.  This pins the packing, the MFMA fragment layout and the activation rounding;
* reference: against the reference semantics (f32 activations, weights widened from bf16 as
  io/safetensors.rs:540-542 loads them), within the bf16-storage tolerance 2e-2.
"""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def bf16_weights(rng, shape, scale=0.02):
    """Random weights as bf16 bits (RNE of N(0, scale))."""
    import oracle

    return oracle.f32_to_bf16((rng.standard_normal(shape, dtype=np.float32) * scale).astype(np.float32))


def round_bf16(orc, x):
    return orc.bf16_to_f32(orc.f32_to_bf16(x))


def sum_splits(parts):
    acc = parts[0].copy()
    for z in range(1, parts.shape[0]):
        acc = acc + parts[z]
    return acc


def padded(a):
    """Device copy of a [M, K] f32 array with rows padded to a multiple of 4 floats (NaN in the
    padding: the kernel must not read past K)."""
    import torch

    m, k = a.shape
    lda = (k + 3) // 4 * 4
    d = torch.full((m, lda), float("nan"), device="cuda")
    d[:, :k] = dev(a)
    return d[:, :k]


SHAPES = [  # (M, K, N): C5 decode / prefill tiles, C1 and C4 shapes, ragged tails; the C5 step's
    # M 2304 runs 128-row blocks over q|k|v's 24 column groups and 96-row blocks over 16 (K cut
    # short to keep the oracle quick)
    (256, 4096, 1024), (300, 512, 520), (64, 896, 1152), (8, 256, 688), (37, 96, 300),
    (1, 64, 40), (17, 100, 33), (130, 4096, 256), (5, 2, 3), (2304, 64, 6144), (2304, 96, 4096),
    (2300, 100, 4090),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_bf16_gemm_matches_linear(orc, gpu_ctx, shape):
    import torch

    m, k, n = shape
    print(f"bf16 gemm shape={shape}", flush=True)
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    wb = bf16_weights(rng, (k, n))
    w = orc.bf16_to_f32(wb)
    bp = gpu_ctx.weight_pack_bf16(dev(wb.view(np.int16)), k, n)
    tight = orc.linear_with_bias(round_bf16(orc, a), w, None)
    ref = orc.linear_with_bias(a, w, None)
    for splits in sorted({1, 2, gpu_ctx.gemm_bf16_splits(m, k, n)}):
        q = (k + 31) // 32
        per = (q + splits - 1) // splits
        if (q + per - 1) // per != splits:
            continue
        out = torch.full((splits, m, n), float("nan"), device="cuda")
        gpu_ctx.gemm_bf16(padded(a), bp, k, n, splits, out)
        torch.cuda.synchronize()
        got = sum_splits(out.cpu().numpy())
        assert normwise_error(got, tight) <= 1e-5, (shape, splits)
        assert normwise_error(got, ref) <= 2e-2, (shape, splits)


def test_bf16_pack_sources_agree(gpu_ctx):
    """Packing from f32 (rounded on the device) equals packing the RNE bf16 bits; the column
    concatenation pack equals packing the concatenated matrix; the [N, K] source layout equals
    the transposed [K, N] one."""
    import torch

    import oracle

    rng = np.random.default_rng(7)
    k = 96
    parts = [(rng.standard_normal((k, n), dtype=np.float32) * 0.05).astype(np.float32) for n in (64, 16, 48)]
    cat = np.concatenate(parts, axis=1)
    bits = oracle.f32_to_bf16(cat).view(np.int16)
    p_f32 = gpu_ctx.weight_pack_bf16(dev(cat), k, 128)
    p_bits = gpu_ctx.weight_pack_bf16(dev(bits), k, 128)
    assert torch.equal(p_f32, p_bits)
    p_cols = gpu_ctx.weight_pack_bf16_columns([dev(p) for p in parts], k)
    assert torch.equal(p_cols, p_bits)
    p_t = gpu_ctx.weight_pack_bf16(dev(np.ascontiguousarray(bits.T)), k, 128, src_layout=1)
    assert torch.equal(p_t, p_bits)


@pytest.mark.parametrize("m,k,f,bias", [(8, 4096, 1024, False), (300, 256, 688, True), (64, 896, 4864, False),
                                        (3, 64, 40, True)])
def test_bf16_swiglu(orc, gpu_ctx, m, k, f, bias):
    import torch

    print(f"bf16 swiglu m={m} k={k} f={f}", flush=True)
    rng = np.random.default_rng(m + k + f)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w1b, w3b = bf16_weights(rng, (k, f)), bf16_weights(rng, (k, f))
    w1, w3 = orc.bf16_to_f32(w1b), orc.bf16_to_f32(w3b)
    b1 = rng.standard_normal(f, dtype=np.float32) * 0.1 if bias else None
    b3 = rng.standard_normal(f, dtype=np.float32) * 0.1 if bias else None
    bp = gpu_ctx.weight_pack_bf16_pair(dev(w1b.view(np.int16)), dev(w3b.view(np.int16)), k, f)
    out = torch.full((m, f), float("nan"), device="cuda")
    gpu_ctx.gemm_bf16_swiglu(padded(a), bp, k, f, out, None if b1 is None else dev(b1),
                             None if b3 is None else dev(b3))
    torch.cuda.synchronize()
    got = out.cpu().numpy()

    def swiglu(x):
        up = orc.linear_with_bias(x, w1, b1)
        gate = orc.linear_with_bias(x, w3, b3)
        return orc.mul(up, orc.silu(gate))

    assert normwise_error(got, swiglu(round_bf16(orc, a))) <= 1e-5
    assert normwise_error(got, swiglu(a)) <= 2e-2


def logits_f64(hr, w, chunk=16384):
    """hr [M, H] times w [V, H]^T in f64, over vocabulary chunks (bounded host memory)."""
    out = np.empty((hr.shape[0], w.shape[0]), np.float64)
    h64 = hr.astype(np.float64)
    for v0 in range(0, w.shape[0], chunk):
        out[:, v0:v0 + chunk] = h64 @ w[v0:v0 + chunk].astype(np.float64).T
    return out


# (200, 256, 20000): 79 column groups over 96-row blocks (the third one partial), as the C5 head;
# (8, 4096, 128256): the C5 head itself (Llama-3-8B hidden and vocabulary)
@pytest.mark.parametrize("m,h,v", [(1, 64, 129), (4, 256, 4096), (257, 512, 3000), (8, 2048, 32000), (200, 256, 20000),
                                   (8, 4096, 128256)])
def test_bf16_lm_head_argmax(orc, gpu_ctx, m, h, v):
    import torch

    print(f"bf16 lm_head m={m} h={h} v={v}", flush=True)
    rng = np.random.default_rng(h + v)
    hid = rng.standard_normal((m, h), dtype=np.float32)
    wb = bf16_weights(rng, (v, h), 0.05)
    w = orc.bf16_to_f32(wb)
    bp = gpu_ctx.weight_pack_bf16(dev(wb.view(np.int16)), h, v, src_layout=1)
    del wb
    tok = torch.empty(m, dtype=torch.int32, device="cuda")
    prob = torch.empty(m, device="cuda")
    gpu_ctx.lm_head_argmax_bf16(padded(hid), bp, v, tok, prob)
    torch.cuda.synchronize()
    hr = round_bf16(orc, hid)
    logits = logits_f64(hr, w)
    rows = range(m) if m <= 64 else list(range(32)) + [m - 1]
    for r in rows:
        top2 = np.sort(logits[r])[-2:]
        if top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])):
            continue  # near tie: the summation order may pick the other index
        ridx, rprob = orc.matmul_rhs_transposed_argmax(hr[r:r + 1], w)
        assert int(tok[r]) == ridx, r
        assert abs(float(prob[r]) - rprob) <= 1e-4 * max(rprob, 1e-30) + 1e-7


def test_bf16_lm_head_reference_vector_and_ties(gpu_ctx):
    """matmul.rs:745-758: lhs [1,2], rhs [[1,0],[0,1],[1,1]] -> (2, 0.66524094) (all values
    exact in bf16); equal logits across slabs keep the first index."""
    import torch

    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    prob = torch.empty(1, device="cuda")
    hid = torch.zeros((1, 4), device="cuda")
    hid[0, :2] = torch.tensor([1.0, 2.0])
    w = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    bp = gpu_ctx.weight_pack_bf16(dev(w), 2, 3, src_layout=1)
    gpu_ctx.lm_head_argmax_bf16(hid[:, :2], bp, 3, tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 2
    assert abs(float(prob[0]) - 0.66524094) <= 1e-6
    v, h = 300, 4
    w = np.zeros((v, h), np.float32)
    w[[70, 5, 200, 71, 6], 0] = 1.0  # max logit 1.0 at 5, 6, 70, 71, 200 -> first is 5
    bp = gpu_ctx.weight_pack_bf16(dev(w), h, v, src_layout=1)
    gpu_ctx.lm_head_argmax_bf16(dev(np.array([[1, 0, 0, 0]], np.float32)), bp, v, tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 5


def padded16(bits):
    """Device copy of [M, K] bf16 bits (uint16) with rows padded to a multiple of 8 elements (NaN
    bits in the padding: the kernel must not read past K)."""
    import torch

    m, k = bits.shape
    lda = (k + 7) // 8 * 8
    d = torch.full((m, lda), 0x7fc0, dtype=torch.int16, device="cuda")
    d[:, :k] = dev(bits.view(np.int16))
    return d[:, :k]


@pytest.mark.parametrize("shape", SHAPES)
def test_bf16_gemm_bf16_activations_bit_identical(orc, gpu_ctx, shape):
    """A handed over as bf16 bits (RNE of the f32 activations) gives exactly the f32 call's
    partials: the kernel rounds f32 activations with the same rule."""
    import torch

    m, k, n = shape
    print(f"bf16-activation gemm shape={shape}", flush=True)
    rng = np.random.default_rng(5 * m + k + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    wb = bf16_weights(rng, (k, n))
    bp = gpu_ctx.weight_pack_bf16(dev(wb.view(np.int16)), k, n)
    splits = gpu_ctx.gemm_bf16_splits(m, k, n)
    ref = torch.full((splits, m, n), float("nan"), device="cuda")
    got = torch.full((splits, m, n), float("nan"), device="cuda")
    gpu_ctx.gemm_bf16(padded(a), bp, k, n, splits, ref)
    gpu_ctx.gemm_bf16(padded16(orc.f32_to_bf16(a)), bp, k, n, splits, got)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), shape


@pytest.mark.parametrize("m,k,f", [(300, 256, 688), (2304, 4096, 1024), (64, 896, 4864), (3, 100, 40)])
def test_bf16_swiglu_bf16_in_out(orc, gpu_ctx, m, k, f):
    """bf16 activations in: the same f32 output as the f32 call; bf16 output: exactly the RNE
    of the f32 output (direct epilogue and the split-sum path alike)."""
    import torch

    print(f"bf16 swiglu bf16 in/out m={m} k={k} f={f}", flush=True)
    rng = np.random.default_rng(m * 7 + k + f)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w1b, w3b = bf16_weights(rng, (k, f)), bf16_weights(rng, (k, f))
    bp = gpu_ctx.weight_pack_bf16_pair(dev(w1b.view(np.int16)), dev(w3b.view(np.int16)), k, f)
    b1 = dev(rng.standard_normal(f, dtype=np.float32) * 0.1)
    out32 = torch.full((m, f), float("nan"), device="cuda")
    gpu_ctx.gemm_bf16_swiglu(padded(a), bp, k, f, out32, b1, None)
    a16 = padded16(orc.f32_to_bf16(a))
    out32b = torch.full((m, f), float("nan"), device="cuda")
    gpu_ctx.gemm_bf16_swiglu(a16, bp, k, f, out32b, b1, None)
    out16 = torch.full((m, f), 0x7fc0, dtype=torch.int16, device="cuda")
    gpu_ctx.gemm_bf16_swiglu(a16, bp, k, f, out16, b1, None)
    torch.cuda.synchronize()
    assert torch.equal(out32b, out32)
    want = orc.f32_to_bf16(out32.cpu().numpy())
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("m,h,v", [(33, 200, 1000), (8, 4096, 128256)])
def test_bf16_head_bf16_activations(orc, gpu_ctx, m, h, v):
    """The greedy head over bf16 activations: the f32 call's tokens and probabilities exactly
    (also at the C5 head, 4096 -> 128256); at the C5 head the tokens also match the oracle's
    fused argmax over the bf16-rounded rows (matmul.rs:190-274) away from near ties."""
    import torch

    print(f"bf16 head bf16 activations m={m} h={h} v={v}", flush=True)
    rng = np.random.default_rng(21 + v)
    hid = rng.standard_normal((m, h), dtype=np.float32)
    wb = bf16_weights(rng, (v, h))
    bp = gpu_ctx.weight_pack_bf16(dev(wb.view(np.int16)), h, v, src_layout=1)
    tok = [torch.empty(m, dtype=torch.int32, device="cuda") for _ in range(2)]
    prob = [torch.empty(m, device="cuda") for _ in range(2)]
    gpu_ctx.lm_head_argmax_bf16(padded(hid), bp, v, tok[0], prob[0])
    gpu_ctx.lm_head_argmax_bf16(padded16(orc.f32_to_bf16(hid)), bp, v, tok[1], prob[1])
    torch.cuda.synchronize()
    assert torch.equal(tok[0], tok[1]) and torch.equal(prob[0], prob[1])
    if v < 100000:
        return
    w = orc.bf16_to_f32(wb)
    del wb
    hr = round_bf16(orc, hid)
    logits = logits_f64(hr, w)
    for r in range(m):
        top2 = np.sort(logits[r])[-2:]
        if top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])):
            continue
        ridx, rprob = orc.matmul_rhs_transposed_argmax(hr[r:r + 1], w)
        assert int(tok[1][r]) == ridx, r
        assert abs(float(prob[1][r]) - rprob) <= 1e-4 * max(rprob, 1e-30) + 1e-7


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4096 * 37 + 3, 0), (1000, 1), (1 << 20, 0)])
def test_convert_f32_to_bf16(orc, gpu_ctx, n, offset):
    """fi_convert_f32_to_bf16 against the oracle's nearest-even narrowing, with ties, the
    largest finite values, infinities, NaN, denormals and signed zeros; an offset start
    exercises the unaligned path."""
    import torch

    rng = np.random.default_rng(n)
    x = rng.standard_normal(n + offset, dtype=np.float32) * np.float32(100)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4028235e38, -3.4028235e38, 1e-40, -1e-41,
                        1.00390625, 1.01171875, -1.00390625], np.float32)  # ties: 1 + 2^-8, 1 + 3 * 2^-8
    x[offset:offset + min(n, special.size)] = special[:min(n, special.size)]
    src = dev(x)[offset:]
    out = torch.full((n + 1,), 0x1234, dtype=torch.int16, device="cuda")
    gpu_ctx.convert_f32_to_bf16(src, out[:n])
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = orc.f32_to_bf16(x[offset:])
    nan = np.isnan(x[offset:])
    assert np.array_equal(got[:n][~nan], want[~nan])
    assert np.all((got[:n][nan] & 0x7f80) == 0x7f80) and np.all((got[:n][nan] & 0x7f) != 0)
    assert got[n] == 0x1234  # nothing written past n
