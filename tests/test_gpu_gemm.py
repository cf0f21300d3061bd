"""GPU parity of the MFMA projection GEMM and the fused lm_head argmax against the CPU
oracle (matmul_f32 / linear_f32_with_bias / matmul_rhs_transposed_f32 /
matmul_rhs_transposed_argmax_f32).  f32 tolerance: 1e-4 normwise (only the summation order
differs); greedy token ids exact."""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu

SHAPES = [  # (M, K, N); M <= 64 with K, N multiples of 4 take the weight-streaming kernel
    (1, 7, 5), (3, 33, 65), (64, 896, 896), (64, 896, 128), (17, 4864, 896),
    (200, 256, 688), (64, 896, 4864), (130, 64, 70),
    (1, 4, 4), (5, 100, 1152), (33, 196, 260), (48, 388, 36), (64, 4864, 9728), (7, 2052, 12),
]


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemm_weight_layout(orc, gpu_ctx, shape, bias):
    import torch

    m, k, n = shape
    print(f"gemm [K,N] shape={shape} bias={bias}", flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float32)
    b = rng.standard_normal(n, dtype=np.float32) if bias else None
    out = torch.empty((m, n), device="cuda")
    gpu_ctx.gemm(dev(a), dev(w), out, bias=dev(b) if bias else None, b_layout=0)
    torch.cuda.synchronize()
    ref = orc.linear_with_bias(a, w, b)
    assert normwise_error(out.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("shape", SHAPES)
def test_gemm_transposed_layout(orc, gpu_ctx, shape):
    import torch

    m, k, n = shape
    print(f"gemm [N,K] shape={shape}", flush=True)
    rng = np.random.default_rng(m + 3 * k + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.standard_normal((n, k), dtype=np.float32)
    out = torch.empty((m, n), device="cuda")
    gpu_ctx.gemm(dev(a), dev(w), out, b_layout=1)
    torch.cuda.synchronize()
    assert normwise_error(out.cpu().numpy(), orc.matmul_rhs_transposed(a, w)) <= 1e-5


def test_gemm_exact_on_integers(gpu_ctx):
    """Small integers make every product and partial sum exact in f32, so the GEMM must
    equal numpy exactly whatever the summation order (pins the MFMA operand layout)."""
    import torch

    rng = np.random.default_rng(1)
    for m, k, n in [(64, 64, 64), (5, 20, 37), (128, 96, 80), (64, 384, 256), (3, 1000, 68)]:
        a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
        w = rng.integers(-4, 5, size=(k, n)).astype(np.float32)
        out = torch.empty((m, n), device="cuda")
        gpu_ctx.gemm(dev(a), dev(w), out, b_layout=0)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), a @ w)


@pytest.mark.parametrize("m,h,v", [(1, 2, 3), (4, 256, 4096), (64, 896, 5000), (3, 64, 129)])
def test_lm_head_argmax(orc, gpu_ctx, m, h, v):
    import torch

    print(f"lm_head argmax m={m} h={h} v={v}", flush=True)
    rng = np.random.default_rng(h + v)
    hid = rng.standard_normal((m, h), dtype=np.float32)
    w = rng.standard_normal((v, h), dtype=np.float32)
    tok = torch.empty(m, dtype=torch.int32, device="cuda")
    prob = torch.empty(m, device="cuda")
    gpu_ctx.lm_head_argmax(dev(hid), dev(w), tok, prob)
    torch.cuda.synchronize()
    logits = orc.matmul_rhs_transposed(hid, w)
    for r in range(m):
        ridx, rprob = orc.matmul_rhs_transposed_argmax(hid[r:r + 1], w)
        top2 = np.sort(logits[r])[-2:] if v > 1 else None
        if top2 is not None and top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])):
            continue  # near tie: summation order may legitimately pick the other index
        assert int(tok[r]) == ridx
        assert abs(float(prob[r]) - rprob) <= 1e-4 * max(rprob, 1e-30) + 1e-7


def test_lm_head_argmax_reference_vector(gpu_ctx):
    """matmul.rs:745-758: lhs [1,2], rhs [[1,0],[0,1],[1,1]] -> (2, 0.66524094)."""
    import torch

    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    prob = torch.empty(1, device="cuda")
    gpu_ctx.lm_head_argmax(dev(np.array([[1, 2]], np.float32)),
                           dev(np.array([[1, 0], [0, 1], [1, 1]], np.float32)), tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 2
    assert abs(float(prob[0]) - 0.66524094) <= 1e-6


def test_lm_head_argmax_first_max_on_ties(gpu_ctx):
    """Equal logits across tiles and inside a tile: the first index wins (strict > inside a
    chunk, left chunk wins on >=)."""
    import torch

    v, h = 300, 4
    w = np.zeros((v, h), np.float32)
    w[[70, 5, 200, 71], 0] = 1.0  # max logit 1.0 at 5, 70, 71, 200 -> first is 5
    hid = np.array([[1, 0, 0, 0]], np.float32)
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    prob = torch.empty(1, device="cuda")
    gpu_ctx.lm_head_argmax(dev(hid), dev(w), tok, prob)
    torch.cuda.synchronize()
    assert int(tok[0]) == 5
