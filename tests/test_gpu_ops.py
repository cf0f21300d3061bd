"""GPU parity of the decoder-block ops against the CPU oracle: embedding gather (exact),
RoPE (bit-exact: host cos/sin table built with the reference's loop), residual add (exact),
RMSNorm and SwiGLU (f32, within 1e-4 normwise; only summation order / libm expf differ)."""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def test_embedding_exact(orc, gpu_ctx):
    import torch

    rng = np.random.default_rng(0)
    table = rng.standard_normal((4096, 256), dtype=np.float32)
    ids = rng.integers(0, 4096, size=77).astype(np.int32)
    out = torch.empty((77, 256), device="cuda")
    gpu_ctx.embedding(dev(table), dev(ids), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), orc.embedding_gather(table, ids.astype(np.uint32)))


def test_embedding_out_of_vocab_reported(gpu_ctx):
    import torch

    from ferrisinfer_amd import FerrisError

    table = torch.ones((8, 32), device="cuda")
    ids = torch.tensor([1, 8], dtype=torch.int32, device="cuda")
    out = torch.empty((2, 32), device="cuda")
    gpu_ctx.embedding(table, ids, out)
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert e.value.kind == "Runtime"
    assert float(out[1].abs().sum()) == 0.0


@pytest.mark.parametrize("rows,hidden,eps", [(1, 256, 1e-6), (64, 896, 1e-6), (33, 4096, 1e-5), (3, 7, 1e-6)])
def test_rms_norm(orc, gpu_ctx, rows, hidden, eps):
    import torch

    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, hidden), dtype=np.float32)
    r = rng.standard_normal((rows, hidden), dtype=np.float32)
    w = rng.standard_normal(hidden, dtype=np.float32)
    out = torch.empty((rows, hidden), device="cuda")
    gpu_ctx.rms_norm(dev(x), dev(w), out, eps)
    s = torch.empty_like(out)
    out2 = torch.empty_like(out)
    gpu_ctx.add_rms_norm(dev(x), dev(r), s, dev(w), out2, eps)
    torch.cuda.synchronize()
    assert normwise_error(out.cpu().numpy(), orc.rms_norm(x, w, eps)) <= 1e-5
    summed = orc.add(x, r)
    assert np.array_equal(s.cpu().numpy(), summed)
    assert normwise_error(out2.cpu().numpy(), orc.rms_norm(summed, w, eps)) <= 1e-5


@pytest.mark.parametrize("hq,hkv,d,rot,theta", [
    (8, 2, 32, 32, 10000.0),      # C1 tiny
    (14, 2, 64, 64, 1000000.0),   # C4 Qwen2-0.5B
    (32, 8, 128, 128, 500000.0),  # C5 Llama-3-8B
    (4, 2, 64, 32, 10000.0),      # partial rotary
])
def test_rope_bit_exact_ragged_positions(orc, gpu_ctx, hq, hkv, d, rot, theta):
    """Three sequences packed in one token stream with their own position offsets."""
    import torch

    rng = np.random.default_rng(d)
    seqs = [(0, 17), (1000, 5), (8000, 30)]  # (position_offset, tokens)
    T = sum(n for _, n in seqs)
    q = rng.standard_normal((T, hq, d), dtype=np.float32)
    k = rng.standard_normal((T, hkv, d), dtype=np.float32)
    positions = np.concatenate([np.arange(o, o + n) for o, n in seqs]).astype(np.int32)
    max_pos = 8192
    cos_t = torch.empty((max_pos, rot // 2), device="cuda")
    sin_t = torch.empty_like(cos_t)
    gpu_ctx.rope_table(max_pos, d, rot, theta, cos_t, sin_t)
    qd, kd = dev(q), dev(k)
    gpu_ctx.rope(qd, kd, dev(positions), cos_t, sin_t, rot, max_pos)
    torch.cuda.synchronize()
    gpu_ctx.check_faults()
    start = 0
    for off, n in seqs:
        rq, rk = orc.rope(q[start:start + n], k[start:start + n], off, rot, theta)
        assert np.array_equal(qd[start:start + n].cpu().numpy(), rq)
        assert np.array_equal(kd[start:start + n].cpu().numpy(), rk)
        start += n


def test_rope_rejects_bad_config(gpu_ctx):
    import torch

    from ferrisinfer_amd import FerrisError

    t = torch.empty((16, 8), device="cuda")
    with pytest.raises(FerrisError) as e:
        gpu_ctx.rope_table(16, 32, 31, 10000.0, t, t)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(FerrisError) as e:
        gpu_ctx.rope_table(16, 32, 16, 0.0, t, t)
    assert e.value.kind == "InvalidConfig"


def test_silu_mul_and_add(orc, gpu_ctx):
    import torch

    rng = np.random.default_rng(9)
    up = rng.standard_normal((64, 4864), dtype=np.float32) * 3
    gate = rng.standard_normal((64, 4864), dtype=np.float32) * 3
    out = torch.empty((64, 4864), device="cuda")
    gpu_ctx.silu_mul(dev(up), dev(gate), out)
    s = torch.empty_like(out)
    gpu_ctx.add(dev(up), dev(gate), s)
    torch.cuda.synchronize()
    ref = orc.mul(up, orc.silu(gate))
    assert normwise_error(out.cpu().numpy(), ref) <= 1e-6
    assert np.array_equal(s.cpu().numpy(), orc.add(up, gate))


def test_rope_position_outside_table_reported(gpu_ctx):
    """A position beyond the RoPE table leaves its token unrotated and is reported as Runtime
    with the position message (not the token-id message)."""
    import torch

    from ferrisinfer_amd import FerrisError

    d, rot, npos = 32, 32, 16
    cos_t = torch.empty((npos, rot // 2), device="cuda")
    sin_t = torch.empty_like(cos_t)
    gpu_ctx.rope_table(npos, d, rot, 10000.0, cos_t, sin_t)
    q = torch.ones((2, 2, d), device="cuda")
    k = torch.ones((2, 1, d), device="cuda")
    pos = torch.tensor([3, npos + 5], dtype=torch.int32, device="cuda")
    gpu_ctx.rope(q, k, pos, cos_t, sin_t, rot, npos)
    torch.cuda.synchronize()
    with pytest.raises(FerrisError) as e:
        gpu_ctx.check_faults()
    assert "position outside the RoPE table" in str(e.value)
    assert "vocabulary" not in str(e.value)
    assert torch.equal(q[1], torch.ones_like(q[1]))
    gpu_ctx.check_faults()
