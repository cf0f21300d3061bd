"""Checkpoint import restated in numpy — TEST INFRASTRUCTURE ONLY.

Restates the FerrisInfer reference's safetensors tensor conversion and Qwen2 weight mapping
(crates/ferrisinfer-io/src/safetensors.rs, hf.rs) so tests can check the device loader
(fr_load_hf_weights, fi_convert_to_f32) bit for bit.  Only tests/ may import this module.

Pinning (tests/test_checkpoint.py): the reference's own test vectors (safetensors.rs tests:
BF16 [3, 2] transposed, sharded F32 / F16 values), every one of the 65536 F16 bit patterns
against numpy's IEEE half -> single conversion (all non-NaN patterns) and the closed form
sign | 0x7f800000 | payload << 13 (NaN patterns), every BF16 pattern against bits << 16.
"""
from __future__ import annotations

import numpy as np

SIZES = {"F32": 4, "F16": 2, "BF16": 2}


def bf16_bits_to_f32_bits(bits: np.ndarray) -> np.ndarray:
    """safetensors.rs:538-540: the bf16 pattern is the high half of the f32 pattern."""
    return bits.astype(np.uint32) << np.uint32(16)


def f16_bits_to_f32_bits(bits: np.ndarray) -> np.ndarray:
    """safetensors.rs:542-567 f16_to_f32, vectorised: re-bias normal exponents, normalise
    subnormals (shift the mantissa until bit 10 is set, one exponent step per shift), keep
    the payload of infinities and NaNs."""
    h = bits.astype(np.uint32)
    sign = (h & 0x8000) << 16
    exp = (h >> 10) & 0x1F
    man = h & 0x3FF
    out = np.where(exp == 0x1F, sign | 0x7F800000 | (man << 13),
                   sign | ((exp + 112) << 23) | (man << 13)).astype(np.uint32)
    sub = (exp == 0) & (man != 0)
    if np.any(sub):
        m = man[sub].copy()
        e = np.full(m.shape, -14, np.int64)
        while True:  # the reference's normalisation loop, one step for every lane at once
            todo = (m & 0x400) == 0
            if not np.any(todo):
                break
            m[todo] <<= 1
            e[todo] -= 1
        out[sub] = sign[sub] | ((e + 127).astype(np.uint32) << 23) | ((m & 0x3FF) << 13)
    zero = (exp == 0) & (man == 0)
    out[zero] = sign[zero]
    return out


def convert_to_f32(raw: bytes, dtype: str, shape, transpose: bool) -> np.ndarray:
    """safetensors.rs:437-471 convert_to_f32_vec: little-endian payload -> f32 values in the
    source order, or the rank-2 transpose (output index col * rows + row)."""
    shape = [int(d) for d in shape]
    n = int(np.prod(shape)) if shape else 1
    if len(raw) != n * SIZES[dtype]:
        raise ValueError("byte length mismatch")
    if dtype == "F32":
        bits = np.frombuffer(raw, dtype="<u4").astype(np.uint32)
    elif dtype == "BF16":
        bits = bf16_bits_to_f32_bits(np.frombuffer(raw, dtype="<u2"))
    else:
        bits = f16_bits_to_f32_bits(np.frombuffer(raw, dtype="<u2"))
    vals = bits.view(np.float32)
    if transpose:
        if len(shape) != 2:
            raise ValueError("only rank-2 tensors can be transposed")
        return vals.reshape(shape).T.copy()
    return vals.reshape(shape) if shape else vals.reshape(())


def qwen2_plans(cfg: dict):
    """hf.rs:380-500 qwen2_tensor_plans: (external name, internal name, expected source shape,
    transpose, required) in the reference's order."""
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])
    plans = [("model.embed_tokens.weight", "tok_embeddings.weight", [v, h], False, True)]
    for layer in range(cfg["layers"]):
        s, d = f"model.layers.{layer}.", f"layers.{layer}."
        plans += [
            (s + "input_layernorm.weight", d + "attention_norm.weight", [h], False, True),
            (s + "self_attn.q_proj.weight", d + "attention.wq.weight", [h, h], True, True),
            (s + "self_attn.k_proj.weight", d + "attention.wk.weight", [kvw, h], True, True),
            (s + "self_attn.v_proj.weight", d + "attention.wv.weight", [kvw, h], True, True),
            (s + "self_attn.o_proj.weight", d + "attention.wo.weight", [h, h], True, True),
            (s + "post_attention_layernorm.weight", d + "ffn_norm.weight", [h], False, True),
            (s + "mlp.up_proj.weight", d + "feed_forward.w1.weight", [f, h], True, True),
            (s + "mlp.down_proj.weight", d + "feed_forward.w2.weight", [h, f], True, True),
            (s + "mlp.gate_proj.weight", d + "feed_forward.w3.weight", [f, h], True, True),
            (s + "self_attn.q_proj.bias", d + "attention.wq.bias", [h], False, False),
            (s + "self_attn.k_proj.bias", d + "attention.wk.bias", [kvw], False, False),
            (s + "self_attn.v_proj.bias", d + "attention.wv.bias", [kvw], False, False),
        ]
    plans.append(("model.norm.weight", "norm.weight", [h], False, True))
    if not cfg.get("tie", False):
        plans.append(("lm_head.weight", "output.weight", [v, h], False, True))
    return plans


def internal_weights(tensors: dict, cfg: dict) -> dict:
    """hf.rs:208-304 load_weights over {external name: (dtype, shape, raw bytes)}: the
    internal-name f32 weights the reference model receives (optional tensors skipped when
    absent)."""
    out = {}
    for ext, internal, shape, transpose, required in qwen2_plans(cfg):
        if ext not in tensors:
            if required:
                raise KeyError(ext)
            continue
        dtype, src_shape, raw = tensors[ext]
        if list(src_shape) != shape:
            raise ValueError(f"{ext}: shape {src_shape} != {shape}")
        out[internal] = convert_to_f32(raw, dtype, src_shape, transpose)
    return out
