"""Checkpoint import on the GPU: fi_convert_to_f32 bit for bit against the numpy restatement
of the reference's conversion (every F16 / BF16 pattern, F32 NaN payloads, ragged and
transposed shapes), and HF Qwen2 checkpoints loaded by the runtime (fr_load_hf_weights)
generating the oracle's greedy tokens when the oracle is given the reference's conversion of
the same files (io/safetensors.rs, io/hf.rs)."""
import numpy as np
import pytest

from ferrisinfer_amd.workloads import write_qwen2_checkpoint
from oracle.checkpoint import bf16_bits_to_f32_bits, f16_bits_to_f32_bits, internal_weights

pytestmark = pytest.mark.gpu


def device_convert(ctx, bits: np.ndarray, dtype_code: int, transpose: bool) -> np.ndarray:
    import torch

    rows, cols = bits.shape
    tdt = torch.int32 if bits.dtype.itemsize == 4 else torch.int16
    src = torch.from_numpy(bits.view(np.int32 if bits.dtype.itemsize == 4 else np.int16).copy()).to("cuda", tdt)
    dst = torch.full((rows * cols,), -7.0, dtype=torch.float32, device="cuda")
    ctx.convert_to_f32(src, dtype_code, rows, cols, transpose, dst)
    torch.cuda.synchronize()
    out = dst.cpu().numpy().view(np.uint32)
    return out.reshape((cols, rows) if transpose else (rows, cols))


@pytest.mark.parametrize("transpose", [False, True])
def test_convert_every_16bit_pattern(gpu_ctx, transpose):
    from ferrisinfer_amd.kernel import DTYPE_BF16, DTYPE_F16

    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    for code, ref in ((DTYPE_F16, f16_bits_to_f32_bits), (DTYPE_BF16, bf16_bits_to_f32_bits)):
        want = ref(bits)
        got = device_convert(gpu_ctx, bits, code, transpose)
        assert np.array_equal(got, want.T if transpose else want), code


@pytest.mark.parametrize("shape", [(1, 1), (1, 1000), (33, 65), (300, 17), (64, 4864), (4864, 64)])
def test_convert_shapes_and_f32_payloads(gpu_ctx, shape):
    from ferrisinfer_amd.kernel import DTYPE_BF16, DTYPE_F16, DTYPE_F32

    rng = np.random.default_rng(sum(shape))
    b32 = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    b32.flat[:: max(1, b32.size // 7)] = 0x7FA00001  # signalling-NaN payloads stay untouched
    b16 = rng.integers(0, 2 ** 16, size=shape, dtype=np.uint32).astype(np.uint16)
    for transpose in (False, True):
        got = device_convert(gpu_ctx, b32, DTYPE_F32, transpose)
        assert np.array_equal(got, b32.T if transpose else b32)
        for code, ref in ((DTYPE_F16, f16_bits_to_f32_bits), (DTYPE_BF16, bf16_bits_to_f32_bits)):
            want = ref(b16)
            assert np.array_equal(device_convert(gpu_ctx, b16, code, transpose), want.T if transpose else want)


def test_convert_argument_errors(gpu_ctx):
    import torch

    from ferrisinfer_amd.kernel import DTYPE_F32, FerrisError

    x = torch.zeros(16, device="cuda")
    y = torch.zeros(16, device="cuda")
    gpu_ctx.convert_to_f32(x, DTYPE_F32, 0, 16, True, y)  # empty: no work
    with pytest.raises(FerrisError) as ei:
        gpu_ctx.convert_to_f32(x, 7, 4, 4, False, y)
    assert ei.value.kind == "Unsupported"
    with pytest.raises(FerrisError) as ei:
        gpu_ctx.convert_to_f32(x, DTYPE_F32, 4, 4, False, x)
    assert ei.value.kind == "InvalidConfig"
    with pytest.raises(FerrisError) as ei:
        gpu_ctx.convert_to_f32(x, DTYPE_F32, -1, 4, False, y)
    assert ei.value.kind == "InvalidShape"


CFG = {"hidden": 128, "intermediate": 320, "heads": 4, "kv_heads": 2, "layers": 2, "vocab": 384,
       "max_pos": 256, "eps": 1e-6, "theta": 10000.0}
REQUESTS_SEED = 11


def requests(vocab):
    rng = np.random.default_rng(REQUESTS_SEED)
    return [(rng.integers(0, vocab, size=n).astype(np.uint32), m) for n, m in ((9, 12), (23, 8), (40, 10))]


@pytest.mark.parametrize("dtype,shards,tie,biases", [
    ("BF16", 1, True, True), ("F16", 2, False, True), ("F32", 3, True, False)])
def test_hf_checkpoint_generates_oracle_tokens(orc, tmp_path, dtype, shards, tie, biases):
    from ferrisinfer_amd.runtime import Runtime, read_hf_config
    from test_gpu_model import compare

    cfg = dict(CFG, tie=tie)
    written = write_qwen2_checkpoint(tmp_path, cfg, dtype, seed=5, shards=shards, biases=biases)
    hf = read_hf_config(tmp_path)
    assert hf["rotary_dims"] == cfg["hidden"] // cfg["heads"] and hf["tie"] == tie
    weights = internal_weights(written, cfg)
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                      cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=tie)
    model.set_weights(weights)
    ref = orc.Scheduler(model, page_size=16)
    ref.attach_packer(256, 16)
    gpu = Runtime.from_hf(tmp_path, num_blocks=256, block_size=16)
    _, ties = compare(model, ref, gpu, requests(cfg["vocab"]))
    assert ties == 0
    gpu.close()


def test_hf_load_errors(tmp_path):
    import json
    import os

    from ferrisinfer_amd.kernel import FerrisError
    from ferrisinfer_amd.runtime import Runtime

    cfg = dict(CFG, tie=True)
    write_qwen2_checkpoint(tmp_path / "a", cfg, "BF16", shards=1)
    # shape mismatch: the config claims a wider MLP than the tensors hold
    c = json.loads((tmp_path / "a" / "config.json").read_text())
    c["intermediate_size"] = 384
    (tmp_path / "a" / "config.json").write_text(json.dumps(c))
    with pytest.raises(FerrisError) as ei:
        Runtime.from_hf(tmp_path / "a", num_blocks=64)
    assert ei.value.kind == "InvalidShape"
    # a required tensor absent from the index
    write_qwen2_checkpoint(tmp_path / "b", cfg, "F16", shards=2)
    idx = json.loads((tmp_path / "b" / "model.safetensors.index.json").read_text())
    del idx["weight_map"]["model.norm.weight"]
    (tmp_path / "b" / "model.safetensors.index.json").write_text(json.dumps(idx))
    with pytest.raises(FerrisError) as ei:
        Runtime.from_hf(tmp_path / "b", num_blocks=64)
    assert ei.value.kind == "MissingWeight"
    assert os.path.exists(tmp_path / "b" / "config.json")
