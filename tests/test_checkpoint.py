"""Checkpoint import, host side (no GPU): the numpy restatement of the reference's tensor
conversion pinned by the reference's own vectors and exhaustive closed forms; the runtime
library's safetensors repository (fr_safetensors_info / fr_safetensors_entry), HF config
reader (fr_hf_read_config) and inspection (fr_hf_inspect) against files written here and by
the canonical `safetensors` package, including the reference's error cases
(io/safetensors.rs, io/hf.rs)."""
import json
import os
import struct

import numpy as np
import pytest

from ferrisinfer_amd.workloads import encode, write_qwen2_checkpoint, write_safetensors
from oracle.checkpoint import (bf16_bits_to_f32_bits, convert_to_f32, f16_bits_to_f32_bits,
                               internal_weights, qwen2_plans)


def rt():
    from ferrisinfer_amd import runtime

    return runtime


def error_kind(excinfo):
    from ferrisinfer_amd.kernel import FerrisError

    assert isinstance(excinfo.value, FerrisError)
    return excinfo.value.kind


# ------------------------------------------------------------------ oracle pinning
def test_oracle_conversion_reference_vectors():
    # safetensors.rs tests: BF16 [3, 2] = 1..6 transposed -> [2, 3] = 1, 3, 5, 2, 4, 6
    raw = encode(np.arange(1, 7, dtype=np.float32), "BF16")
    out = convert_to_f32(raw, "BF16", [3, 2], True)
    assert out.shape == (2, 3)
    assert out.ravel().tolist() == [1.0, 3.0, 5.0, 2.0, 4.0, 6.0]
    # sharded test: F32 [10, 20], F16 [1.5, -2]
    assert convert_to_f32(encode(np.array([10, 20]), "F32"), "F32", [2], False).tolist() == [10.0, 20.0]
    assert convert_to_f32(encode(np.array([1.5, -2.0]), "F16"), "F16", [2], False).tolist() == [1.5, -2.0]


def test_oracle_f16_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = f16_bits_to_f32_bits(bits)
    exp = (bits >> 10) & 0x1F
    man = bits & 0x3FF
    nan = (exp == 0x1F) & (man != 0)
    # non-NaN: numpy's IEEE half -> single conversion is exact (zeros, subnormals, normals, inf)
    ref = bits[~nan].view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got[~nan], ref)
    # NaN: payload kept in the top mantissa bits, no quieting
    sign = (bits[nan].astype(np.uint32) & 0x8000) << 16
    assert np.array_equal(got[nan], sign | 0x7F800000 | (man[nan].astype(np.uint32) << 13))
    # spot values: smallest subnormal 2^-24, largest subnormal, smallest normal 2^-14
    f = lambda b: float(f16_bits_to_f32_bits(np.array([b], np.uint16)).view(np.float32)[0])
    assert f(0x0001) == 2.0 ** -24 and f(0x03FF) == 1023 * 2.0 ** -24 and f(0x0400) == 2.0 ** -14
    assert f(0x8000) == 0.0 and np.signbit(f(0x8000))


def test_oracle_bf16_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(bf16_bits_to_f32_bits(bits), bits.astype(np.uint32) << 16)


def test_oracle_plans_follow_reference_table():
    # hf.rs tests: hidden 4, 2 heads, 1 kv head -> wk [4, 2] after the transpose, wq.bias [4]
    cfg = {"hidden": 4, "intermediate": 8, "heads": 2, "kv_heads": 1, "layers": 1, "vocab": 16,
           "tie": True, "max_pos": 128, "eps": 1e-6, "theta": 1e6}
    plans = {p[1]: p for p in qwen2_plans(cfg)}
    assert plans["layers.0.attention.wk.weight"][2] == [2, 4] and plans["layers.0.attention.wk.weight"][3]
    assert plans["layers.0.attention.wq.bias"][2] == [4] and not plans["layers.0.attention.wq.bias"][4]
    assert "output.weight" not in plans
    assert plans["layers.0.feed_forward.w1.weight"][0].endswith("mlp.up_proj.weight")
    assert plans["layers.0.feed_forward.w3.weight"][0].endswith("mlp.gate_proj.weight")


# ------------------------------------------------------------------ repository
def read_raw(entry):
    with open(entry["path"], "rb") as f:
        f.seek(entry["offset"])
        return f.read(entry["byte_len"])


def test_single_file_transposes(tmp_path):
    write_safetensors(tmp_path / "model.safetensors",
                      [("tensor", "BF16", [3, 2], encode(np.arange(1, 7), "BF16"))])
    info = rt().safetensors_info(tmp_path)
    assert info == {"tensors": 1, "shards": 1, "total_data_bytes": 12}
    e = rt().safetensors_entry(tmp_path, "tensor")
    assert e["dtype"] == 1 and e["shape"] == [3, 2] and e["byte_len"] == 12
    assert convert_to_f32(read_raw(e), "BF16", e["shape"], True).ravel().tolist() == [1, 3, 5, 2, 4, 6]


def test_sharded_index(tmp_path):
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors",
                      [("first", "F32", [2], encode(np.array([10.0, 20.0]), "F32"))])
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors",
                      [("second", "F16", [2], encode(np.array([1.5, -2.0]), "F16"))])
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({
        "metadata": {"total_size": 12},
        "weight_map": {"first": "model-00001-of-00002.safetensors",
                       "second": "model-00002-of-00002.safetensors"}}))
    assert rt().safetensors_info(tmp_path) == {"tensors": 2, "shards": 2, "total_data_bytes": 12}
    e1, e2 = rt().safetensors_entry(tmp_path, "first"), rt().safetensors_entry(tmp_path, "second")
    assert convert_to_f32(read_raw(e1), "F32", [2], False).tolist() == [10.0, 20.0]
    assert e2["dtype"] == 2 and convert_to_f32(read_raw(e2), "F16", [2], False).tolist() == [1.5, -2.0]


def test_index_maps_only_listed_tensors(tmp_path):
    write_safetensors(tmp_path / "a.safetensors", [("x", "F32", [1], encode(np.ones(1), "F32")),
                                                   ("unlisted", "F32", [1], encode(np.ones(1), "F32"))])
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "a.safetensors"}}))
    assert rt().safetensors_info(tmp_path)["tensors"] == 1
    with pytest.raises(Exception) as ei:
        rt().safetensors_entry(tmp_path, "unlisted")
    assert error_kind(ei) == "MissingWeight"


def test_canonical_writer_files_parse(tmp_path):
    """Files from the `safetensors` package (the format's own writer): entries and payloads."""
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(0)
    tensors = {"a": torch.randn(5, 7, generator=g), "b": torch.randn(3, generator=g).half(),
               "c": torch.randn(4, 6, generator=g).bfloat16(), "scalar": torch.tensor(2.5)}
    st.save_file(tensors, str(tmp_path / "model.safetensors"), metadata={"format": "pt"})
    assert rt().safetensors_info(tmp_path)["tensors"] == 4
    for name, t in tensors.items():
        e = rt().safetensors_entry(tmp_path, name)
        assert e["shape"] == list(t.shape)
        dt = {torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16"}[t.dtype]
        got = convert_to_f32(read_raw(e), dt, e["shape"], False)
        assert np.array_equal(got.reshape(-1).view(np.uint32), t.float().reshape(-1).numpy().view(np.uint32))


def write_raw(path, header: bytes, body: bytes = b"", header_len=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if header_len is None else header_len))
        f.write(header)
        f.write(body)


def hdr(entries):
    return json.dumps(entries).encode()


@pytest.mark.parametrize("case,kind", [
    ("short", "Io"), ("truncated", "Parse"), ("utf8", "Parse"), ("json", "Parse"),
    ("dtype", "Unsupported"), ("no_dtype", "Parse"), ("no_shape", "Parse"), ("no_offsets", "Parse"),
    ("three_offsets", "Parse"), ("reversed", "Parse"), ("length", "InvalidType"), ("beyond", "Parse"),
    ("fraction", "Parse"),
])
def test_header_errors(tmp_path, case, kind):
    p = tmp_path / "model.safetensors"
    ok = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    body = b"\0" * 8
    if case == "short":
        p.write_bytes(b"\1\2\3")
    elif case == "truncated":
        write_raw(p, hdr({"t": ok}), body, header_len=1 << 20)
    elif case == "utf8":
        write_raw(p, b'{"t\xff": 1}', body)
    elif case == "json":
        write_raw(p, b'{"t": {"dtype": "F32",}', body)
    elif case == "dtype":
        write_raw(p, hdr({"t": dict(ok, dtype="I8")}), body)
    elif case in ("no_dtype", "no_shape", "no_offsets"):
        key = {"no_dtype": "dtype", "no_shape": "shape", "no_offsets": "data_offsets"}[case]
        write_raw(p, hdr({"t": {k: v for k, v in ok.items() if k != key}}), body)
    elif case == "three_offsets":
        write_raw(p, hdr({"t": dict(ok, data_offsets=[0, 4, 8])}), body)
    elif case == "reversed":
        write_raw(p, hdr({"t": dict(ok, data_offsets=[8, 0])}), body)
    elif case == "length":
        write_raw(p, hdr({"t": dict(ok, data_offsets=[0, 4])}), body)
    elif case == "beyond":
        write_raw(p, hdr({"t": ok}), b"\0" * 4)
    elif case == "fraction":
        write_raw(p, b'{"t": {"dtype": "F32", "shape": [2.0], "data_offsets": [0, 8]}}', body)
    with pytest.raises(Exception) as ei:
        rt().safetensors_info(tmp_path)
    assert error_kind(ei) == kind


def test_metadata_skipped_and_missing_files(tmp_path):
    write_safetensors(tmp_path / "model.safetensors", [("t", "F16", [2, 2], encode(np.ones(4), "F16"))],
                      metadata={"format": "pt", "note": "x"})
    assert rt().safetensors_info(tmp_path)["tensors"] == 1
    with pytest.raises(Exception) as ei:
        rt().safetensors_info(tmp_path / "absent")
    assert error_kind(ei) == "Io"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"t": "gone.safetensors"}}))
    with pytest.raises(Exception) as ei:
        rt().safetensors_info(tmp_path)
    assert error_kind(ei) == "Io"


def test_index_tensor_absent_from_shard(tmp_path):
    write_safetensors(tmp_path / "a.safetensors", [("x", "F32", [1], encode(np.ones(1), "F32"))])
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"y": "a.safetensors"}}))
    with pytest.raises(Exception) as ei:
        rt().safetensors_info(tmp_path)
    assert error_kind(ei) == "MissingWeight"


# ------------------------------------------------------------------ HF config / inspection
REF_CONFIG = {"architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2", "hidden_act": "silu",
              "hidden_size": 4, "intermediate_size": 8, "max_position_embeddings": 128,
              "num_attention_heads": 2, "num_hidden_layers": 1, "num_key_value_heads": 1,
              "rms_norm_eps": 0.000001, "rope_theta": 1000000.0, "tie_word_embeddings": True,
              "vocab_size": 16, "bos_token_id": 1, "eos_token_id": 2}


def write_config(d, **over):
    c = dict(REF_CONFIG)
    for k, v in over.items():
        if v is None:
            c.pop(k, None)
        else:
            c[k] = v
    (d / "config.json").write_text(json.dumps(c))


def test_hf_config_reference_case(tmp_path):
    write_config(tmp_path)
    c = rt().read_hf_config(tmp_path)
    assert (c["hidden"], c["intermediate"], c["layers"], c["heads"], c["kv_heads"], c["vocab"]) == (4, 8, 1, 2, 1, 16)
    assert c["max_pos"] == 128 and c["tie"] is True and c["rotary_dims"] == 2
    assert c["eps"] == np.float32(1e-6) and c["theta"] == 1e6


def test_hf_config_defaults_and_rotary(tmp_path):
    write_config(tmp_path, num_key_value_heads=None, rope_theta=None, tie_word_embeddings=None,
                 hidden_size=64, num_attention_heads=4, partial_rotary_factor=0.5, hidden_act="swish")
    c = rt().read_hf_config(tmp_path)
    assert c["kv_heads"] == 4 and c["theta"] == 10000.0 and c["tie"] is False and c["rotary_dims"] == 8
    # round(f32(16) * f32(0.55)) = round(8.8) = 9; round(16 * 0.53) = round(8.48) = 8
    write_config(tmp_path, hidden_size=64, num_attention_heads=4, partial_rotary_factor=0.55)
    assert rt().read_hf_config(tmp_path)["rotary_dims"] == 9
    write_config(tmp_path, hidden_size=64, num_attention_heads=4, partial_rotary_factor=0.53)
    assert rt().read_hf_config(tmp_path)["rotary_dims"] == 8


@pytest.mark.parametrize("over,kind", [
    ({"model_type": "llama"}, "Unsupported"), ({"hidden_act": "gelu"}, "Unsupported"),
    ({"hidden_act": "tanh"}, "Unsupported"), ({"hidden_size": 5}, "InvalidConfig"),
    ({"rms_norm_eps": None}, "Parse"), ({"hidden_size": 4.0}, "Parse"), ({"vocab_size": -3}, "Parse"),
    ({"tie_word_embeddings": 1}, "Parse"),
])
def test_hf_config_errors(tmp_path, over, kind):
    write_config(tmp_path, **over)
    with pytest.raises(Exception) as ei:
        rt().read_hf_config(tmp_path)
    assert error_kind(ei) == kind


def test_hf_inspect_counts(tmp_path):
    cfg = {"hidden": 8, "intermediate": 16, "heads": 2, "kv_heads": 1, "layers": 2, "vocab": 32,
           "tie": False, "max_pos": 64, "eps": 1e-6, "theta": 1e4}
    written = write_qwen2_checkpoint(tmp_path, cfg, "F16", biases=False, shards=2)
    r = rt().hf_inspect(tmp_path)
    assert r["shard_count"] == 2 and r["tensor_count"] == len(written)
    assert r["total_data_bytes"] == sum(len(raw) for *_, raw in written.values())
    assert r["mapped_required"] == 1 + 9 * 2 + 1 + 1 and r["mapped_optional"] == 0
    assert r["missing_optional"] == 3 * 2 and r["missing_required"] == 0 and r["compatible"]
    # the oracle mapping consumes exactly the written tensors
    assert len(internal_weights(written, cfg)) == len(written)


def test_hf_inspect_flags_shape_mismatch(tmp_path):
    cfg = {"hidden": 8, "intermediate": 16, "heads": 2, "kv_heads": 1, "layers": 1, "vocab": 32,
           "tie": True, "max_pos": 64, "eps": 1e-6, "theta": 1e4}
    write_qwen2_checkpoint(tmp_path, cfg, "F32")
    write_config(tmp_path, **{"hidden_size": 8, "intermediate_size": 24, "num_attention_heads": 2,
                              "num_hidden_layers": 1, "vocab_size": 32})
    r = rt().hf_inspect(tmp_path)
    assert r["shape_mismatches"] == 3 and not r["compatible"]  # up, down, gate
