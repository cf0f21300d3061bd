"""Seeded synthetic inputs for the BASELINE configurations (host numpy arrays).

C1-C4 draw from the reference's xorshift64* through ferrisinfer_amd.seeded (uniforms,
Box-Muller normals, integers, Fisher-Yates permutations, one tag per field), so any host can
regenerate them; the GPU path and the CPU oracle see bit-identical inputs.  The synthetic
checkpoints of the import tests keep numpy's PCG64.  Layouts follow
include/ferrisinfer_kernel.h.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import seeded
from .seeded import tag_of


@dataclass
class PagedDecodeWorkload:
    """Config C2: standalone paged decode attention over a shared block pool."""

    num_seqs: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    context_lens: np.ndarray   # int32 [B]
    block_tables: np.ndarray   # int32 [B, max_blocks]
    q: np.ndarray              # f32 [B, Hq, D]
    k_pool: np.ndarray         # f32 [num_blocks, Hkv, bs, D]  (device layout)
    v_pool: np.ndarray
    scale: float

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max())

    def pages_reference_layout(self, pool: np.ndarray) -> np.ndarray:
        """[num_blocks, Hkv, bs, D] -> the reference page layout [num_blocks, bs, Hkv, D]
        (runtime/paged_kv.rs:141-150)."""
        return np.ascontiguousarray(pool.transpose(0, 2, 1, 3))

    def algorithmic_bytes(self, kv_bytes: int = 4) -> int:
        """Bytes one launch must move: every context K/V row once, q in, out back, block
        table entries and context lengths."""
        L = self.context_lens.astype(np.int64)
        kv = int(L.sum()) * self.num_kv_heads * self.head_dim * 2 * kv_bytes
        qo = self.num_seqs * self.num_q_heads * self.head_dim * (4 + 4)
        bt = int(((L + self.block_size - 1) // self.block_size).sum()) * 4
        return kv + qo + bt + self.num_seqs * 4


def paged_decode_c2(seed: int = 0, num_seqs: int = 64, min_len: int = 128, max_len: int = 2048,
                    num_q_heads: int = 32, num_kv_heads: int = 8, head_dim: int = 128,
                    block_size: int = 16, num_blocks: int = 8192,
                    fill_unused_blocks: bool = False) -> PagedDecodeWorkload:
    """C2: lengths ~ U[min_len, max_len] (tag "c2.lens"); block ids are the first
    sum(ceil(L/bs)) entries of a permutation of the pool ("c2.perm"), handed to the sequences in
    order; Q ("c2.q") and the used blocks' K / V ("c2.k", "c2.v", in block-id order) ~ N(0, 1);
    scale 1/sqrt(D).  Unused pool blocks are zero unless ``fill_unused_blocks``."""
    lens = seeded.integers(seed, tag_of("c2.lens"), num_seqs, min_len, max_len).astype(np.int32)
    nblk = (lens + block_size - 1) // block_size
    total = int(nblk.sum())
    if total > num_blocks:
        raise ValueError(f"workload needs {total} blocks, pool has {num_blocks}")
    perm = seeded.permutation(seed, tag_of("c2.perm"), num_blocks)
    max_blocks = int(nblk.max())
    tables = np.zeros((num_seqs, max_blocks), np.int32)
    cursor = 0
    for i, n in enumerate(nblk):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    q = seeded.normals(seed, tag_of("c2.q"), (num_seqs, num_q_heads, head_dim))
    shape = (num_blocks, num_kv_heads, block_size, head_dim)
    k_pool = np.zeros(shape, np.float32)
    v_pool = np.zeros(shape, np.float32)
    used = np.sort(perm[:total] if not fill_unused_blocks else perm)
    k_pool[used] = seeded.normals(seed, tag_of("c2.k"), (used.size,) + shape[1:])
    v_pool[used] = seeded.normals(seed, tag_of("c2.v"), (used.size,) + shape[1:])
    return PagedDecodeWorkload(num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                               num_blocks, lens, tables, q, k_pool, v_pool,
                               float(1.0 / np.sqrt(np.float32(head_dim))))


@dataclass
class PrefillWorkload:
    """Config C3: ragged varlen causal prefill plus KV append with block-shared prefixes."""

    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    prompt_lens: np.ndarray    # int32 [B] total tokens per sequence
    shared_lens: np.ndarray    # int32 [B] prefix tokens shared by block id (0 = none)
    source_of: np.ndarray      # int32 [B] index of the sequence whose blocks are shared (-1)
    block_tables: np.ndarray   # int32 [B, max_blocks]
    cu_seqlens: np.ndarray     # int32 [B+1] over the new (computed) tokens
    context_lens: np.ndarray   # int32 [B] = prompt_lens
    slot_mapping: np.ndarray   # int64 [T_new]
    q: np.ndarray              # f32 [T_new, Hq, D]
    k_new: np.ndarray          # f32 [T_new, Hkv, D]
    v_new: np.ndarray
    scale: float

    @property
    def query_lens(self) -> np.ndarray:
        return np.diff(self.cu_seqlens)

    def full_kv(self, b: int):
        """K/V [L_b, Hkv, D] of sequence b's whole context (shared prefix + own rows)."""
        own_k = self.k_new[self.cu_seqlens[b]:self.cu_seqlens[b + 1]]
        own_v = self.v_new[self.cu_seqlens[b]:self.cu_seqlens[b + 1]]
        s = int(self.shared_lens[b])
        if s == 0:
            return own_k, own_v
        src = int(self.source_of[b])
        sk, sv = self.full_kv(src)
        return np.concatenate([sk[:s], own_k]), np.concatenate([sv[:s], own_v])

    def attention_flops(self) -> int:
        """4*Hq*D * sum over computed tokens of the keys each attends (causal, incl. self)."""
        total = 0
        for b, L in enumerate(self.context_lens):
            start = int(L) - int(self.query_lens[b])
            n = int(self.query_lens[b])
            total += n * start + n * (n + 1) // 2
        return 4 * self.num_q_heads * self.head_dim * total

    def append_bytes(self, kv_bytes: int = 4) -> int:
        t = int(self.cu_seqlens[-1])
        return t * self.num_kv_heads * self.head_dim * 2 * (4 + kv_bytes) + 8 * t


def prefill_c3(seed: int = 0, num_seqs: int = 16, min_len: int = 32, max_len: int = 1024,
               groups: int = 4, group_size: int = 4, shared_prefix: int = 512,
               num_q_heads: int = 32, num_kv_heads: int = 8, head_dim: int = 128,
               block_size: int = 16, num_blocks: int = 4096) -> PrefillWorkload:
    """C3: lengths ~ U[min_len, max_len]; groups of `group_size` consecutive sequences share
    a prefix through the same block ids.  The group's source is its longest member, padded
    to at least shared_prefix + 1 tokens; every other member shares
    min(shared_prefix, floor((L - 1) / block_size) * block_size) tokens (block aligned and
    never the whole prompt, as runtime/prefix_index.rs:98-109 keeps one token to compute)
    and computes only its suffix.  The source computes all its tokens in the same batch;
    KV append precedes attention, so members read the source's freshly written blocks.
    Seeded fields: "c3.lens", "c3.perm", "c3.q", "c3.k", "c3.v"."""
    lens = seeded.integers(seed, tag_of("c3.lens"), num_seqs, min_len, max_len).astype(np.int32)
    shared = np.zeros(num_seqs, np.int32)
    source = np.full(num_seqs, -1, np.int32)
    for g in range(min(groups, num_seqs // group_size)):
        idx = np.arange(g * group_size, (g + 1) * group_size)
        src = int(idx[np.argmax(lens[idx])])
        lens[src] = max(int(lens[src]), shared_prefix + 1)
        for b in idx:
            if b == src:
                continue
            shared[b] = min(shared_prefix, (int(lens[b]) - 1) // block_size * block_size)
            source[b] = src if shared[b] > 0 else -1
    nblk = (lens + block_size - 1) // block_size
    own_blocks = nblk - shared // block_size
    perm = seeded.permutation(seed, tag_of("c3.perm"), num_blocks)
    if int(own_blocks.sum()) > num_blocks:
        raise ValueError("pool too small")
    tables = np.zeros((num_seqs, int(nblk.max())), np.int32)
    cursor = 0
    order = sorted(range(num_seqs), key=lambda b: shared[b] > 0)  # sources first
    for b in order:
        k = int(shared[b]) // block_size
        if k:
            tables[b, :k] = tables[int(source[b]), :k]
        n = int(own_blocks[b])
        tables[b, k:k + n] = perm[cursor:cursor + n]
        cursor += n
    qlens = (lens - shared).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    T = int(cu[-1])
    slots = np.zeros(T, np.int64)
    for b in range(num_seqs):
        for i in range(int(qlens[b])):
            pos = int(shared[b]) + i
            slots[cu[b] + i] = int(tables[b, pos // block_size]) * block_size + pos % block_size
    q = seeded.normals(seed, tag_of("c3.q"), (T, num_q_heads, head_dim))
    k = seeded.normals(seed, tag_of("c3.k"), (T, num_kv_heads, head_dim))
    v = seeded.normals(seed, tag_of("c3.v"), (T, num_kv_heads, head_dim))
    return PrefillWorkload(num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, lens, shared,
                           source, tables, cu, lens.copy(), slots, q, k, v,
                           float(1.0 / np.sqrt(np.float32(head_dim))))


# ---------------------------------------------------------------------------------------
# Decoder configurations (C4, C5) and seeded random weights.

TINY_LLAMA_C1 = dict(hidden=256, intermediate=688, layers=4, heads=8, kv_heads=2, vocab=4096,
                     max_pos=4096, eps=1e-6, theta=10000.0, tie=False)
QWEN2_05B_C4 = dict(hidden=896, intermediate=4864, layers=24, heads=14, kv_heads=2, vocab=151936,
                    max_pos=32768, eps=1e-6, theta=1000000.0, tie=True)


def random_weights(cfg: dict, seed: int = 0, qkv_bias: bool = False, std: float = 0.02) -> dict:
    """Weights named as model/decoder.rs:30-52 in the reference's [in, out] layout.  Matrices,
    embeddings and (optional, Qwen2-style) q/k/v biases ~ N(0, std), each tensor seeded by its
    name (tag = CRC-32 of the name); RMSNorm weights = 1."""
    from concurrent.futures import ThreadPoolExecutor

    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])
    shapes = {"tok_embeddings.weight": (v, h)}
    for layer in range(cfg["layers"]):
        p = f"layers.{layer}."
        for name, shape in (("attention.wq.weight", (h, h)), ("attention.wk.weight", (h, kvw)),
                            ("attention.wv.weight", (h, kvw))):
            shapes[p + name] = shape
        if qkv_bias:
            for name, width in (("attention.wq.bias", h), ("attention.wk.bias", kvw), ("attention.wv.bias", kvw)):
                shapes[p + name] = (width,)
        shapes[p + "attention.wo.weight"] = (h, h)
        for name, shape in (("feed_forward.w1.weight", (h, f)), ("feed_forward.w2.weight", (f, h)),
                            ("feed_forward.w3.weight", (h, f))):
            shapes[p + name] = shape
    if not cfg.get("tie", False):
        shapes["output.weight"] = (v, h)
    # tensors are independent streams: generated on a thread pool (numpy's ufuncs release the
    # GIL), the values do not depend on it
    with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        drawn = dict(zip(shapes, ex.map(lambda k: seeded.normals(seed, tag_of(k), shapes[k], scale=std), shapes)))
    w = {"tok_embeddings.weight": drawn["tok_embeddings.weight"]}
    for layer in range(cfg["layers"]):
        p = f"layers.{layer}."
        w[p + "attention_norm.weight"] = np.ones(h, np.float32)
        for name in ("attention.wq.weight", "attention.wk.weight", "attention.wv.weight"):
            w[p + name] = drawn[p + name]
        if qkv_bias:
            for name in ("attention.wq.bias", "attention.wk.bias", "attention.wv.bias"):
                w[p + name] = drawn[p + name]
        w[p + "attention.wo.weight"] = drawn[p + "attention.wo.weight"]
        w[p + "ffn_norm.weight"] = np.ones(h, np.float32)
        for name in ("feed_forward.w1.weight", "feed_forward.w2.weight", "feed_forward.w3.weight"):
            w[p + name] = drawn[p + name]
    w["norm.weight"] = np.ones(h, np.float32)
    if not cfg.get("tie", False):
        w["output.weight"] = drawn["output.weight"]
    return w


def c1_requests(seed: int = 0, vocab: int = 4096):
    """C1: 4 prompts of 16/24/32/48 ids ~ U[0, vocab) (tags "c1.prompt.<i>"), 32 greedy tokens
    each."""
    return [(seeded.integers(seed, tag_of(f"c1.prompt.{i}"), n, 0, vocab - 1).astype(np.uint32), 32)
            for i, n in enumerate((16, 24, 32, 48))]


# ----------------------------------------------------------------------------- C4
C4_ARRIVAL_RATE = 8.0        # requests per second (Poisson)
C4_VIRTUAL_TICK_S = 0.05     # one scheduler tick stands for 50 ms of arrival time
C4_PROMPT_MEDIAN = 512
C4_PROMPT_SIGMA = 0.5        # lognormal shape (the config names the median only)
C4_MAX_PROMPT = 2048


def c4_requests(seed: int = 0, n: int = 128, vocab: int = 151936) -> list:
    """C4 workload: ``n`` requests, Poisson arrivals at 8/s mapped to integer ticks of a
    fixed 50 ms virtual duration (the reference's continuous-batching driver admits requests
    by integer arrival tick, cli/main.rs:1721-1741), prompt lengths lognormal (median 512,
    sigma 0.5) clipped to [1, 2048], ids ~ U[0, vocab), output lengths ~ U[64, 256].
    Seeded fields: gaps -ln(1 - u) / rate ("c4.gaps"), log-lengths from normals ("c4.lens"),
    outputs ("c4.outs"), the ids of request i ("c4.prompt.<i>"); f64 arithmetic."""
    u = seeded.uniforms(seed, tag_of("c4.gaps"), n).astype(np.float64)
    gaps = -np.log(1.0 - u) / C4_ARRIVAL_RATE
    arrival_s = np.cumsum(gaps) - gaps[0]
    ticks = np.floor(arrival_s / C4_VIRTUAL_TICK_S).astype(np.int64)
    z = seeded.normals(seed, tag_of("c4.lens"), (n,)).astype(np.float64)
    lens = np.exp(np.log(C4_PROMPT_MEDIAN) + C4_PROMPT_SIGMA * z)
    lens = np.clip(np.rint(lens), 1, C4_MAX_PROMPT).astype(np.int64)
    outs = seeded.integers(seed, tag_of("c4.outs"), n, 64, 256)
    return [dict(prompt=seeded.integers(seed, tag_of(f"c4.prompt.{i}"), int(L), 0, vocab - 1).astype(np.uint32),
                 max_new_tokens=int(o), arrival_tick=int(t))
            for i, (L, o, t) in enumerate(zip(lens, outs, ticks))]


def run_continuous(sched, requests: list, max_ticks: int | None = None, run_ahead: bool = False) -> dict:
    """Drives a scheduler (the GPU Runtime or the oracle's ReferenceScheduler) the way the
    reference's continuous-batching profile does (cli/main.rs:1716-1834): requests arriving
    at the current tick are submitted before it runs, an idle scheduler jumps to the next
    arrival, and each tick's wall time is the scheduler's own ``execute_next_tick``.  Returns
    the tick log and per-request generated tokens; ``decode_tok_s`` is generated tokens over
    the summed decode-tick time (cli/main.rs:1502-1512, 1619-1622).

    run_ahead (GPU Runtime only): a tick followed by no arrival is executed with run_ahead, so
    the next decode tick is already on the device when the driver comes back."""
    ticks, seq_of = [], []
    nxt, tick_index = 0, 0
    while nxt < len(requests) or sched.has_pending():
        if max_ticks is not None and len(ticks) >= max_ticks:
            break
        while (nxt < len(requests) and requests[nxt]["arrival_tick"] < tick_index
               and not sched.has_pending()):
            tick_index = requests[nxt]["arrival_tick"]
        while nxt < len(requests) and requests[nxt]["arrival_tick"] == tick_index:
            r = requests[nxt]
            seq_of.append(sched.submit(r["prompt"], max_new_tokens=r["max_new_tokens"]))
            nxt += 1
        if run_ahead:
            quiet = nxt >= len(requests) or requests[nxt]["arrival_tick"] > tick_index + 1
            rep = sched.execute_next_tick(run_ahead=quiet)
        else:
            rep = sched.execute_next_tick()
        if rep is None:
            if nxt < len(requests):
                tick_index = requests[nxt]["arrival_tick"]
                continue
            break
        kind, updates = rep
        ticks.append(dict(tick=tick_index, kind=kind, batch=len(updates),
                          generated=sum(u["token"] is not None for u in updates),
                          appended=sum(u["appended"] for u in updates),
                          reused=sum(u["reused"] for u in updates),
                          seconds=sched.last_tick_seconds))
        if hasattr(sched, "last_tick_profile"):
            ticks[-1]["profile"] = sched.last_tick_profile()
        if hasattr(sched, "last_batch_context_sum"):
            ticks[-1]["ctx_sum"] = sched.last_batch_context_sum()
        tick_index += 1
    dec = [t for t in ticks if t["kind"] == 1]
    pre = [t for t in ticks if t["kind"] == 0]
    gen = sum(t["generated"] for t in ticks)
    dec_s = sum(t["seconds"] for t in dec)
    pre_s = sum(t["seconds"] for t in pre)
    return dict(ticks=ticks, sequence_ids=seq_of, generated_tokens=gen,
                decode_ticks=len(dec), prefill_ticks=len(pre), decode_seconds=dec_s,
                prefill_seconds=pre_s,
                decode_tok_s=gen / dec_s if dec_s > 0 else 0.0,
                prefill_tok_s=sum(t["appended"] for t in pre) / pre_s if pre_s > 0 else 0.0,
                avg_decode_batch=(sum(t["batch"] for t in dec) / len(dec)) if dec else 0.0,
                max_decode_batch=max((t["batch"] for t in dec), default=0))

# ----------------------------------------------------------------------------- checkpoints
# Synthetic HF checkpoints for the checkpoint-import tests and bench leg.  Safetensors format:
# 8-byte little-endian header length, JSON header {name: {dtype, shape, data_offsets}}, then
# the packed little-endian payloads.


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (finite inputs)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def encode(values: np.ndarray, dtype: str) -> bytes:
    v = np.asarray(values, np.float32)
    if dtype == "F32":
        return v.astype("<f4").tobytes()
    if dtype == "F16":
        return v.astype("<f2").tobytes()
    return f32_to_bf16_bits(v).astype("<u2").tobytes()


def write_safetensors(path, tensors, metadata=None, header_override=None):
    """tensors: list of (name, dtype, shape, raw bytes).  header_override (dict) replaces the
    generated header, for malformed-file tests."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = json.dumps(header_override if header_override is not None else header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def qwen2_config(cfg: dict, **extra) -> dict:
    c = {
        "architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2", "hidden_act": "silu",
        "hidden_size": cfg["hidden"], "intermediate_size": cfg["intermediate"],
        "max_position_embeddings": cfg["max_pos"], "num_attention_heads": cfg["heads"],
        "num_hidden_layers": cfg["layers"], "num_key_value_heads": cfg["kv_heads"],
        "rms_norm_eps": cfg["eps"], "rope_theta": cfg["theta"],
        "tie_word_embeddings": cfg["tie"], "vocab_size": cfg["vocab"],
    }
    c.update(extra)
    return c


def write_qwen2_checkpoint(model_dir, cfg: dict, dtype: str = "BF16", seed: int = 0, shards: int = 1,
                           biases: bool = True, std: float = 0.05, config_extra=None):
    """A random Qwen2 checkpoint in HF naming ([out, in] projections).  Returns {external
    name: (dtype, shape, raw bytes)} of everything written."""
    os.makedirs(model_dir, exist_ok=True)
    rng = np.random.default_rng(seed)
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])

    def t(name, *shape, ones=False):
        vals = (1.0 + 0.1 * rng.standard_normal(shape)) if ones else rng.standard_normal(shape) * std
        return (name, dtype, list(shape), encode(vals.astype(np.float32), dtype))

    tensors = [t("model.embed_tokens.weight", v, h)]
    for layer in range(cfg["layers"]):
        p = f"model.layers.{layer}."
        tensors += [t(p + "input_layernorm.weight", h, ones=True),
                    t(p + "self_attn.q_proj.weight", h, h), t(p + "self_attn.k_proj.weight", kvw, h),
                    t(p + "self_attn.v_proj.weight", kvw, h), t(p + "self_attn.o_proj.weight", h, h),
                    t(p + "post_attention_layernorm.weight", h, ones=True),
                    t(p + "mlp.gate_proj.weight", f, h), t(p + "mlp.up_proj.weight", f, h),
                    t(p + "mlp.down_proj.weight", h, f)]
        if biases:
            tensors += [t(p + "self_attn.q_proj.bias", h), t(p + "self_attn.k_proj.bias", kvw),
                        t(p + "self_attn.v_proj.bias", kvw)]
    tensors.append(t("model.norm.weight", h, ones=True))
    if not cfg["tie"]:
        tensors.append(t("lm_head.weight", v, h))
    with open(os.path.join(model_dir, "config.json"), "w") as fh:
        json.dump(qwen2_config(cfg, **(config_extra or {})), fh)
    if shards == 1:
        write_safetensors(os.path.join(model_dir, "model.safetensors"), tensors, metadata={"format": "pt"})
    else:
        weight_map = {}
        for s in range(shards):
            part = tensors[s::shards]
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(os.path.join(model_dir, fname), part, metadata={"format": "pt"})
            weight_map.update({name: fname for name, *_ in part})
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as fh:
            json.dump({"metadata": {"total_size": sum(len(r) for *_, r in tensors)}, "weight_map": weight_map}, fh)
    return {name: (dt, shape, raw) for name, dt, shape, raw in tensors}
