"""A decoder forward step over bf16-stored weights, composed from the kernel C ABI: the path of
the bf16 configurations (BASELINE C5: a Llama-3-8B-shaped decoder with bf16 weights and a bf16
KV pool, one step = the batch's decode tokens plus a chunk of prefill tokens).

Per layer, in the order of the reference decoder block (runtime/reference.rs:163-370):

    attention_norm -> q|k|v projection (fi_gemm_bf16, split-K partials)
    -> fi_qkv_rope_append (split sum, RoPE, K/V appended to the layer's bf16 pool by slot)
    -> paged attention: fi_attn_decode_paged over the decode rows, fi_attn_prefill_paged_bf16
       (bf16 MFMA) over the prefill chunk (the reference's decode / cached-prefixed attention
       per sequence, kernel/cpu/attention.rs:332-686)
    -> wo projection -> fi_splitk_residual_rms_norm (residual add + ffn_norm)
    -> fi_gemm_bf16_swiglu (w1, w3, silu * mul) -> w2 projection
    -> fi_splitk_residual_rms_norm (residual add + the next layer's attention_norm, or the
       final norm after the last layer)

then each sequence's last row goes through the fused greedy head (fi_lm_head_argmax_bf16,
matmul_rhs_transposed_argmax_f32, kernel/cpu/matmul.rs:190-274).

The reference loads bf16 weights by exact widening (io/safetensors.rs:540-542) and runs f32
math; the projections here multiply bf16-rounded activations by the bf16 weights with f32
accumulation; the prefill chunk's attention multiplies bf16-rounded queries and probabilities
by the bf16 K/V; the rest (norms, RoPE, decode attention, softmax, SwiGLU) stays f32.

With `bf16_activations` (the default) the projections' inputs are handed over as bf16 bits,
rounded to nearest even where they are produced: the residual norms write them directly
(fi_splitk_residual_rms_norm_bf16), the SwiGLU epilogue stores them, and the attention output
and the first norm are narrowed by fi_convert_f32_to_bf16.  The GEMMs round f32 activations
the same way, so the step's results are bit-identical either way; bf16 inputs halve the bytes
the projections stage per K step.
"""
from __future__ import annotations

from dataclasses import dataclass

from .kernel import DTYPE_BF16, FerrisError

LLAMA3_8B_C5 = dict(hidden=4096, intermediate=14336, layers=32, heads=32, kv_heads=8, vocab=128256,
                    max_pos=8192 + 2048, eps=1e-6, theta=500000.0, tie=False)


@dataclass
class StepBatch:
    """Device metadata of one mixed step: rows [0, num_decode) are one decode token per
    sequence, rows [num_decode, T) the prefill chunks packed by cu_seqlens."""
    positions: object          # int32 [T]
    slot_mapping: object       # int64 [T]
    num_decode: int
    dec_block_tables: object   # int32 [Bd, max_blocks]
    dec_context_lens: object   # int32 [Bd] (including the new token)
    dec_max_context: int
    pf_block_tables: object    # int32 [Bp, max_blocks]
    pf_cu_seqlens: object      # int32 [Bp + 1] (relative to row num_decode)
    pf_context_lens: object    # int32 [Bp]
    pf_max_query: int
    last_rows: object          # int32 [R]: the rows that feed the greedy head


class Bf16Decoder:
    """Packed bf16 weights, per-layer bf16 K/V pools and the step buffers for up to
    `max_tokens` rows."""

    def __init__(self, ctx, cfg: dict, num_blocks: int, block_size: int, max_tokens: int,
                 max_last_rows: int, bf16_activations: bool = True):
        import torch

        self.ctx, self.cfg = ctx, cfg
        self.bf16_activations = bool(bf16_activations)
        self.h, self.f, self.v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
        self.hq, self.hkv = cfg["heads"], cfg["kv_heads"]
        self.d = self.h // self.hq
        self.nqkv = (self.hq + 2 * self.hkv) * self.d
        self.num_blocks, self.block_size = num_blocks, block_size
        self.layers: list[dict] = []
        self.final_norm = None
        self.lm_head = None
        dev = "cuda"
        pool = (num_blocks, self.hkv, block_size, self.d)
        self.k_pools = [torch.empty(pool, dtype=torch.int16, device=dev) for _ in range(cfg["layers"])]
        self.v_pools = [torch.empty(pool, dtype=torch.int16, device=dev) for _ in range(cfg["layers"])]
        t = max_tokens
        self.hidden = [torch.empty(t, self.h, device=dev), torch.empty(t, self.h, device=dev)]
        self.normed = torch.empty(t, self.h, device=dev)
        self.q = torch.empty(t, self.hq, self.d, device=dev)
        self.attn = torch.empty(t, self.hq, self.d, device=dev)
        if self.bf16_activations:  # bf16 bits (int16) of the projections' inputs
            self.normed16 = torch.empty(t, self.h, dtype=torch.int16, device=dev)
            self.attn16 = torch.empty(t, self.h, dtype=torch.int16, device=dev)
            self.act = torch.empty(t, self.f, dtype=torch.int16, device=dev)
        else:
            self.act = torch.empty(t, self.f, device=dev)
        self.max_tokens = t
        self.last = torch.empty(max_last_rows, self.h, device=dev)
        if self.bf16_activations:
            self.last16 = torch.empty(max_last_rows, self.h, dtype=torch.int16, device=dev)
        self.tok = torch.empty(max_last_rows, dtype=torch.int32, device=dev)
        self.prob = torch.empty(max_last_rows, device=dev)
        self.max_pos = cfg["max_pos"]
        self.cos = torch.empty(self.max_pos, self.d // 2, device=dev)
        self.sin = torch.empty(self.max_pos, self.d // 2, device=dev)
        ctx.rope_table(self.max_pos, self.d, self.d, cfg["theta"], self.cos, self.sin)
        self.parts = None

    # ---- weights ----
    def set_layer(self, wq, wk, wv, wo, w1, w2, w3, attention_norm, ffn_norm):
        """Packs one layer's [in, out] weights (bf16 bits as int16 / torch.bfloat16, or f32)."""
        c = self.ctx
        self.layers.append(dict(
            qkv=c.weight_pack_bf16_columns([wq, wk, wv], self.h),
            wo=c.weight_pack_bf16(wo, self.h, self.h),
            w13=c.weight_pack_bf16_pair(w1, w3, self.h, self.f),
            w2=c.weight_pack_bf16(w2, self.f, self.h),
            attention_norm=attention_norm, ffn_norm=ffn_norm))

    def set_head(self, final_norm, output_weight):
        """Final norm [H] and the [vocab, hidden] output weight."""
        self.final_norm = final_norm
        self.lm_head = self.ctx.weight_pack_bf16(output_weight, self.h, self.v, src_layout=1)

    def _parts(self, rows: int, n: int, splits: int):
        import torch

        need = splits * rows * n
        if self.parts is None or self.parts.numel() < need:
            self.parts = torch.empty(need, device="cuda")
        return self.parts[:need].view(splits, rows, n)

    # ---- one step ----
    def step(self, x, b: StepBatch, layers: int | None = None, head: bool = True):
        """Runs the step on input rows x [T, H] (f32 embeddings); returns (tokens, probs) of
        the last rows (device tensors) when `head`, else the final hidden state."""
        c, cfg = self.ctx, self.cfg
        t = int(x.shape[0])
        if t > self.max_tokens:
            raise FerrisError(3, f"step of {t} rows exceeds the decoder's {self.max_tokens}")
        nl = len(self.layers) if layers is None else layers
        if nl == 0 or nl > len(self.layers):
            raise FerrisError(7, "decoder layers are not set")
        h, f, eps, nd = self.h, self.f, cfg["eps"], b.num_decode
        scale = 1.0 / float(self.d) ** 0.5
        res, other = self.hidden[0][:t], self.hidden[1][:t]
        res.copy_(x)
        normed, q, attn, act = self.normed[:t], self.q[:t], self.attn[:t], self.act[:t]
        c.rms_norm(res, self.layers[0]["attention_norm"], normed, eps)
        b16 = self.bf16_activations
        # the projections' inputs: bf16 bits of the normed rows and the attention output
        xin = self.normed16[:t] if b16 else normed
        ain = self.attn16[:t] if b16 else attn.view(t, h)
        if b16:
            c.convert_f32_to_bf16(normed, xin)
        s_qkv = c.gemm_bf16_splits(t, h, self.nqkv)
        s_o = c.gemm_bf16_splits(t, h, h)
        s_w2 = c.gemm_bf16_splits(t, f, h)
        for li in range(nl):
            w = self.layers[li]
            parts = self._parts(t, self.nqkv, s_qkv)
            c.gemm_bf16(xin, w["qkv"], h, self.nqkv, s_qkv, parts)
            c.qkv_rope_append(parts, s_qkv, None, b.positions, self.cos, self.sin, self.d, self.max_pos,
                              b.slot_mapping, self.k_pools[li], self.v_pools[li], DTYPE_BF16,
                              self.num_blocks, self.block_size, self.hq, self.hkv, self.d, q)
            if nd > 0:
                c.attn_decode_paged(q[:nd], self.k_pools[li], self.v_pools[li], DTYPE_BF16,
                                    b.dec_block_tables, b.dec_context_lens, b.dec_max_context, self.hkv,
                                    self.block_size, self.num_blocks, scale, attn[:nd])
            if t > nd:
                c.attn_prefill_paged_bf16(q[nd:], self.k_pools[li], self.v_pools[li], b.pf_block_tables,
                                          b.pf_cu_seqlens, b.pf_context_lens, b.pf_max_query, self.hkv,
                                          self.block_size, self.num_blocks, scale, attn[nd:])
            if b16:
                c.convert_f32_to_bf16(attn, ain)
            parts = self._parts(t, h, s_o)
            c.gemm_bf16(ain, w["wo"], h, h, s_o, parts)
            c.splitk_residual_rms_norm(parts, s_o, None, res, other, w["ffn_norm"], xin, eps)
            c.gemm_bf16_swiglu(xin, w["w13"], h, f, act)
            parts = self._parts(t, h, s_w2)
            c.gemm_bf16(act, w["w2"], f, h, s_w2, parts)
            nxt = self.layers[li + 1]["attention_norm"] if li + 1 < nl else self.final_norm
            # the final norm stays f32: its last rows feed the head
            c.splitk_residual_rms_norm(parts, s_w2, None, other, res, nxt, xin if li + 1 < nl else normed, eps)
        if not head:
            return res
        r = int(b.last_rows.numel())
        last = self.last[:r]
        c.embedding(normed, b.last_rows, last)
        if b16:  # the head's input as bf16 bits (the kernel rounds f32 the same way)
            c.convert_f32_to_bf16(last, self.last16[:r])
            last = self.last16[:r]
        c.lm_head_argmax_bf16(last, self.lm_head, self.v, self.tok[:r], self.prob[:r])
        return self.tok[:r], self.prob[:r]


def build_step_batch(decode_ctx, prefill, block_size: int, num_blocks: int, seed: int = 0):
    """Host metadata of a mixed step -> (StepBatch on the device, per-sequence block tables).

    decode_ctx: context length (including the new token) of each decode sequence;
    prefill: list of (cached_prefix_len, new_tokens) chunks.
    Block ids: the first sum(ceil(len / block_size)) entries of a permutation of the pool
    (ferrisinfer_amd.seeded, tag "c5.block_ids"), assigned to the sequences in order (decode
    sequences first)."""
    import numpy as np
    import torch

    from . import seeded

    lens = [int(c) for c in decode_ctx] + [int(p + n) for p, n in prefill]
    need = [(n + block_size - 1) // block_size for n in lens]
    if sum(need) > num_blocks:
        raise FerrisError(6, f"step needs {sum(need)} blocks, pool has {num_blocks}")
    perm = seeded.permutation(seed, seeded.tag_of("c5.block_ids"), num_blocks)
    tables, off = [], 0
    for k in need:
        tables.append(perm[off:off + k])
        off += k
    maxb = max(need)

    def table(rows):
        out = np.zeros((max(len(rows), 1), maxb), np.int32)
        for i, r in enumerate(rows):
            out[i, :len(r)] = r
        return out

    nd = len(decode_ctx)
    pos, slot = [], []
    for i, ctx in enumerate(decode_ctx):
        p = int(ctx) - 1
        pos.append(p)
        slot.append(int(tables[i][p // block_size]) * block_size + p % block_size)
    cu = [0]
    for j, (pre, n) in enumerate(prefill):
        for p in range(pre, pre + n):
            pos.append(p)
            slot.append(int(tables[nd + j][p // block_size]) * block_size + p % block_size)
        cu.append(cu[-1] + n)
    last = list(range(nd)) + [nd + cu[j + 1] - 1 for j in range(len(prefill))]
    d = lambda a, dt: torch.from_numpy(np.ascontiguousarray(np.asarray(a, dt))).cuda()  # noqa: E731
    batch = StepBatch(
        positions=d(pos, np.int32), slot_mapping=d(slot, np.int64), num_decode=nd,
        dec_block_tables=d(table(tables[:nd]), np.int32), dec_context_lens=d(list(decode_ctx) or [0], np.int32),
        dec_max_context=max([int(c) for c in decode_ctx] or [1]),
        pf_block_tables=d(table(tables[nd:]), np.int32), pf_cu_seqlens=d(cu, np.int32),
        pf_context_lens=d([p + n for p, n in prefill] or [0], np.int32),
        pf_max_query=max([n for _, n in prefill] or [1]),
        last_rows=d(last, np.int32))
    return batch, tables


def c5_step_shape(seed: int = 0, num_decode: int = 256, min_ctx: int = 512, max_ctx: int = 8192,
                  chunk: int = 2048, chunk_prefix: int = 2048):
    """BASELINE C5's step: 256 decode sequences with context U[min_ctx, max_ctx]
    (ferrisinfer_amd.seeded, tag "c5.context_lens") and one 2048-token prefill chunk (the
    second chunk of a 4096-token prompt: 2048 tokens cached)."""
    from . import seeded

    decode_ctx = seeded.integers(seed, seeded.tag_of("c5.context_lens"), num_decode, min_ctx, max_ctx).tolist()
    return decode_ctx, [(chunk_prefix, chunk)]
