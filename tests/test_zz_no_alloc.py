"""fi_attn_decode_paged_noalloc against fi_attn_decode_paged through the C ABI.

The no-allocation entry point runs the same kernels with the split-KV partials in the
library's fixed device array instead of the context workspace, so its outputs must be
bit-identical to the allocating entry point's.  Two calls in a row, the second on a smaller
batch, show that a call does not depend on what the previous one left in the shared array.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(x, torch):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _inputs(wl, kv_dtype, torch):
    import oracle
    from ferrisinfer_amd import DTYPE_BF16, DTYPE_F32

    if kv_dtype == "bf16":
        kp = torch.from_numpy(oracle.f32_to_bf16(wl.k_pool).view(np.int16)).cuda()
        vp = torch.from_numpy(oracle.f32_to_bf16(wl.v_pool).view(np.int16)).cuda()
        dt = DTYPE_BF16
    else:
        kp, vp, dt = _dev(wl.k_pool, torch), _dev(wl.v_pool, torch), DTYPE_F32
    return (_dev(wl.q, torch), kp, vp, dt, _dev(wl.block_tables, torch),
            _dev(wl.context_lens, torch))


def _both(ctx_ref, ctx_na, wl, kv_dtype, torch):
    q, kp, vp, dt, bt, cl = _inputs(wl, kv_dtype, torch)
    ref = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    args = (wl.max_context_len, wl.num_kv_heads, wl.block_size, wl.num_blocks, wl.scale)
    ctx_ref.attn_decode_paged(q, kp, vp, dt, bt, cl, *args, ref)
    torch.cuda.synchronize()
    ctx_ref.check_faults()
    free_before = torch.cuda.mem_get_info()[0]
    ctx_na.attn_decode_paged_noalloc(q, kp, vp, dt, bt, cl, *args, got)
    torch.cuda.synchronize()
    free_after = torch.cuda.mem_get_info()[0]
    ctx_na.check_faults()
    return ref, got, free_before, free_after


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_noalloc_decode_matches_allocating_entry_point(gpu_ctx, kv_dtype):
    import torch

    from ferrisinfer_amd import Context
    from ferrisinfer_amd.workloads import paged_decode_c2

    ctx_na = Context(0)  # a fresh context: it has never allocated a workspace
    try:
        # call 1: the C2 batch (64 ragged sequences, up to 4 partitions each)
        print(f"noalloc decode call 1: C2 full, {kv_dtype}", flush=True)
        wl = paged_decode_c2(seed=21)
        ref, got, fb, fa = _both(gpu_ctx, ctx_na, wl, kv_dtype, torch)
        assert torch.equal(ref, got)
        assert fa == fb, f"device free memory moved by {fb - fa} bytes"
        # call 2: a smaller batch of another shape (Qwen2-like GQA 7, up to 3 partitions)
        print(f"noalloc decode call 2: 9 seqs 14/2/64, {kv_dtype}", flush=True)
        wl2 = paged_decode_c2(seed=22, num_seqs=9, min_len=1, max_len=700, num_q_heads=14,
                              num_kv_heads=2, head_dim=64, num_blocks=1024)
        ref2, got2, fb2, fa2 = _both(gpu_ctx, ctx_na, wl2, kv_dtype, torch)
        assert torch.equal(ref2, got2)
        assert fa2 == fb2, f"device free memory moved by {fb2 - fa2} bytes"
        assert torch.isfinite(got2).all()
    finally:
        ctx_na.close()


def test_noalloc_decode_rejects_oversized_partials(gpu_ctx):
    """A launch whose partials exceed the fixed array is refused before anything is enqueued."""
    import torch

    from ferrisinfer_amd import DTYPE_F32, FerrisError

    b, hq, hkv, d, bs = 1024, 32, 8, 128, 16
    ctx_len = 4096  # 8 partitions: 1024 * 32 * 8 * 130 * 4 bytes > 96 MiB
    q = torch.zeros((b, hq, d), device="cuda")
    kc = torch.zeros((4, hkv, bs, d), device="cuda")
    bt = torch.zeros((b, ctx_len // bs), dtype=torch.int32, device="cuda")
    cl = torch.zeros((b,), dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(FerrisError) as e:
        gpu_ctx.attn_decode_paged_noalloc(q, kc, kc, DTYPE_F32, bt, cl, ctx_len, hkv, bs, 4,
                                          d ** -0.5, out)
    assert e.value.kind == "Runtime"
    assert "scratch" in str(e.value)
