"""ctypes binding of the CPU oracle (oracle/liboracle.so) — TEST INFRASTRUCTURE ONLY.

The oracle is a C++ restatement of the FerrisInfer reference CPU path (Rust sources under
crates/ferrisinfer-{kernel,runtime,model}); each C++ function cites the reference
file:line it follows.  Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the timed CPU
baseline.  The product path (ferrisinfer_amd) never imports it.

Parity pinning: tests/test_oracle_golden.py (the reference's known-answer vectors),
tests/test_oracle_reference_units.py (the reference's own unit tests of the scheduler, prefix
index, prefix block manager, sequence state, session and KV cache, run against this
restatement) and tests/test_oracle_invariants.py (closed forms and f64 brute force: RoPE
angles, norms and pairing, attention, softmax, RMSNorm, SwiGLU, the greedy head).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import time

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

ERROR_KINDS = ["Io", "Parse", "InvalidShape", "InvalidLayout", "InvalidType", "InvalidConfig",
               "MissingWeight", "Unsupported", "Runtime"]


class OracleError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.kind = ERROR_KINDS[status - 1] if 0 < status <= len(ERROR_KINDS) else f"status{status}"
        super().__init__(f"{self.kind}: {message}")


def build(force: bool = False) -> str:
    """Compiles liboracle.so with the committed Makefile (g++, -ffp-contract=off)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s"] + (["-B"] if force else []), cwd=_HERE, check=True)
    return LIB_PATH


_lib = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
I64P = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
I64 = C.c_int64
VP = C.c_void_p

_SIGS = {
    "orc_embedding_gather_f32": [F32P, I64, I64, U32P, I64, F32P],
    "orc_rms_norm_f32": [F32P, F32P, I64, I64, C.c_float, F32P],
    "orc_matmul_f32": [F32P, F32P, I64, I64, I64, F32P],
    "orc_linear_f32_with_bias": [F32P, F32P, VP, I64, I64, I64, F32P],
    "orc_matmul_rhs_transposed_f32": [F32P, F32P, I64, I64, I64, F32P],
    "orc_matmul_rhs_transposed_argmax_f32": [F32P, F32P, I64, I64, C.POINTER(C.c_uint32),
                                             C.POINTER(C.c_float)],
    "orc_argmax_last_token": [F32P, I64, I64, C.POINTER(C.c_uint32), C.POINTER(C.c_float)],
    "orc_sample_last_token": [F32P, I64, I64, C.c_float, I64, C.c_float, C.POINTER(C.c_uint64),
                              C.POINTER(C.c_uint32), C.POINTER(C.c_float)],
    "orc_rope_f32": [F32P, F32P, I64, I64, I64, I64, I64, I64, C.c_float],
    "orc_prefixed_causal_attention_f32": [F32P, F32P, F32P, I64, I64, I64, I64, I64, F32P],
    "orc_cached_prefixed_causal_attention_f32": [F32P, F32P, F32P, I64, F32P, F32P, I64, I64,
                                                 I64, I64, F32P],
    "orc_decode_causal_attention_f32": [F32P, F32P, F32P, I64, F32P, F32P, I64, I64, I64, F32P],
    "orc_silu_f32_in_place": [F32P, I64],
    "orc_mul_f32_in_place": [F32P, F32P, I64],
    "orc_add_f32_in_place": [F32P, F32P, I64],
    "orc_paged_decode_gather_attention": [F32P, F32P, F32P, I32P, I64, I32P, I64, I64, I64, I64,
                                          I64, F32P],
    "orc_paged_kv_write_sequence": [VP, I64, I64, I64, F32P, F32P],
    "orc_paged_kv_write_slot": [VP, I64, I64, F32P, F32P],
    "orc_paged_kv_read_prefix": [VP, I64, I64, F32P, F32P],
    "orc_paged_kv_block_table": [VP, I64, I64, I64P, I64, C.POINTER(I64)],
    "orc_paged_kv_page_infos": [VP, I64, I64P, I64, C.POINTER(I64)],
    "orc_paged_kv_import_prefix": [VP, VP, I64],
    "orc_model_set_weight": [VP, C.c_char_p, F32P, I64],
    "orc_model_forward_logits": [VP, U32P, I64, F32P],
    "orc_session_prefill": [VP, U32P, I64],
    "orc_session_step": [VP, C.POINTER(C.c_uint32), C.POINTER(C.c_float)],
    "orc_session_last_sample": [VP, C.POINTER(C.c_uint32), C.POINTER(C.c_float)],
    "orc_session_last_hidden": [VP, F32P],
    "orc_session_copy_prefix": [VP, VP, I64],
    "orc_session_read_prefix": [VP, I64, I64, F32P, F32P],
    "orc_scheduler_submit": [VP, U32P, I64, I64, I64, C.POINTER(C.c_uint64)],
    "orc_scheduler_execute_next_tick": [VP, C.POINTER(C.c_int32)],
    "orc_scheduler_last_report": [VP, C.POINTER(C.c_int32), I64P, F32P, I64, C.POINTER(I64)],
    "orc_scheduler_last_released": [VP, I64, I64P, I64, C.POINTER(I64)],
    "orc_scheduler_generated": [VP, C.c_uint64, U32P, I64, C.POINTER(I64)],
    "orc_scheduler_block_ref_count": [VP, C.c_uint64, I64, I64, C.POINTER(I64)],
    "orc_scheduler_attach_packer": [VP, I64, I64],
    "orc_scheduler_packed_sizes": [VP, I64P],
    "orc_scheduler_packed": [VP, I32P, I64P, I32P, I32P, I32P, I64, I32P, I32P, I32P,
                             np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")],
    "orc_scheduler_packer_free": [VP, C.POINTER(I64)],
    "orc_scheduler_packer_pages": [VP, C.c_uint64, I32P, I64, C.POINTER(I64)],
    "orc_scheduler_session_blocks": [VP, C.c_uint64, I64, I64, I64P, I64, C.POINTER(I64)],
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int32
        L.orc_last_error.restype = C.c_char_p
        L.orc_runtime_last_error.restype = C.c_char_p
        L.orc_sampler_state_new.argtypes = [C.c_uint64]
        L.orc_sampler_state_new.restype = C.c_uint64
        L.orc_sampler_next_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_sampler_next_f32.restype = C.c_float
        L.orc_set_threads.argtypes = [I64]
        L.orc_set_threads.restype = None
        L.orc_threads.restype = I64
        L.orc_f32_to_bf16_rne.argtypes = [F32P, U16P, I64]
        L.orc_f32_to_bf16_rne.restype = None
        L.orc_bf16_to_f32.argtypes = [U16P, F32P, I64]
        L.orc_bf16_to_f32.restype = None
        L.orc_paged_kv_create.argtypes = [I64] * 5
        L.orc_paged_kv_create.restype = VP
        L.orc_paged_kv_destroy.argtypes = [VP]
        L.orc_paged_kv_destroy.restype = None
        L.orc_paged_kv_reset.argtypes = [VP]
        L.orc_paged_kv_reset.restype = None
        L.orc_paged_kv_allocated_pages.argtypes = [VP, I64]
        L.orc_paged_kv_allocated_pages.restype = I64
        L.orc_paged_kv_free_pages.argtypes = [VP, I64]
        L.orc_paged_kv_free_pages.restype = I64
        L.orc_model_create.argtypes = [I64] * 7 + [C.c_float, C.c_float, I64, C.c_int32]
        L.orc_model_create.restype = VP
        L.orc_model_destroy.argtypes = [VP]
        L.orc_model_destroy.restype = None
        L.orc_session_create.argtypes = [VP, I64, I64, I64]
        L.orc_session_create.restype = VP
        L.orc_session_destroy.argtypes = [VP]
        L.orc_session_destroy.restype = None
        L.orc_session_position.argtypes = [VP]
        L.orc_session_position.restype = I64
        L.orc_scheduler_create.argtypes = [VP] + [I64] * 8
        L.orc_scheduler_create.restype = VP
        L.orc_scheduler_destroy.argtypes = [VP]
        L.orc_scheduler_destroy.restype = None
        L.orc_scheduler_has_pending.argtypes = [VP]
        L.orc_scheduler_has_pending.restype = C.c_int32
        for name in ("orc_session_set_sampler", "orc_scheduler_set_sampler"):
            getattr(L, name).argtypes = [VP, C.c_float, I64, C.c_float, C.c_uint64]
            getattr(L, name).restype = C.c_int32
        L.orc_session_sampler_state.argtypes = [VP, C.POINTER(C.c_uint64)]
        L.orc_session_sampler_state.restype = C.c_int32
        _lib = L
    return _lib


def _check(status: int, runtime: bool = False):
    if status != 0:
        L = lib()
        msg = (L.orc_runtime_last_error() if runtime else L.orc_last_error()) or b""
        raise OracleError(status, msg.decode())


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return int(lib().orc_threads())


# ----------------------------------------------------------------- kernels
def embedding_gather(embedding, ids):
    e = f32(embedding)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.zeros((ids.size, e.shape[1]), np.float32)
    _check(lib().orc_embedding_gather_f32(e, e.shape[0], e.shape[1], ids, ids.size, out))
    return out


def rms_norm(x, w, eps):
    x = f32(x)
    w = f32(w)
    out = np.zeros_like(x)
    hidden = x.shape[-1]
    _check(lib().orc_rms_norm_f32(x, w, x.size // hidden, hidden, eps, out))
    return out


def matmul(a, b):
    a, b = f32(a), f32(b)
    out = np.zeros((a.shape[0], b.shape[1]), np.float32)
    _check(lib().orc_matmul_f32(a, b, a.shape[0], a.shape[1], b.shape[1], out))
    return out


def linear_with_bias(x, w, bias=None):
    x, w = f32(x), f32(w)
    out = np.zeros((x.shape[0], w.shape[1]), np.float32)
    bias_arr = f32(bias) if bias is not None else None
    ptr = bias_arr.ctypes.data_as(C.c_void_p) if bias_arr is not None else None
    _check(lib().orc_linear_f32_with_bias(x, w, ptr, x.shape[0], x.shape[1], w.shape[1], out))
    return out


def matmul_rhs_transposed(a, b):
    a, b = f32(a), f32(b)
    out = np.zeros((a.shape[0], b.shape[0]), np.float32)
    _check(lib().orc_matmul_rhs_transposed_f32(a, b, a.shape[0], a.shape[1], b.shape[0], out))
    return out


def matmul_rhs_transposed_argmax(h, w):
    h, w = f32(h), f32(w)
    idx = C.c_uint32()
    prob = C.c_float()
    _check(lib().orc_matmul_rhs_transposed_argmax_f32(h, w, w.shape[1], w.shape[0],
                                                      C.byref(idx), C.byref(prob)))
    return int(idx.value), float(prob.value)


def sampler_state_new(seed: int) -> int:
    """SamplerState::new (runtime/sampler.rs:55-63)."""
    return int(lib().orc_sampler_state_new(C.c_uint64(seed)))


def sampler_next_f32(state: int):
    """SamplerState::next_f32 (runtime/sampler.rs:65-74): returns (value, new_state)."""
    st = C.c_uint64(state)
    v = lib().orc_sampler_next_f32(C.byref(st))
    return float(v), int(st.value)


def sample_last_token(logits, temperature, top_k, top_p, state):
    """sample_last_token (runtime/sampler.rs:121-241) on the last row of logits [seq, vocab]:
    returns (token, probability, new_state)."""
    logits = f32(logits)
    if logits.ndim == 1:
        logits = logits[None, :]
    st = C.c_uint64(state)
    idx = C.c_uint32()
    prob = C.c_float()
    _check(lib().orc_sample_last_token(logits, logits.shape[0], logits.shape[1], float(temperature), int(top_k),
                                       float(top_p), C.byref(st), C.byref(idx), C.byref(prob)))
    return int(idx.value), float(prob.value), int(st.value)


def argmax_last_token(logits):
    logits = f32(logits)
    if logits.ndim == 1:
        logits = logits[None, :]
    idx = C.c_uint32()
    prob = C.c_float()
    _check(lib().orc_argmax_last_token(logits, logits.shape[0], logits.shape[1], C.byref(idx),
                                       C.byref(prob)))
    return int(idx.value), float(prob.value)


def rope(q, k, position_offset, rotary_dims, theta):
    """q [T,Hq,D], k [T,Hkv,D]; returns rotated copies."""
    q, k = f32(q).copy(), f32(k).copy()
    _check(lib().orc_rope_f32(q, k, q.shape[0], q.shape[1], k.shape[1], q.shape[2],
                              position_offset, rotary_dims, theta))
    return q, k


def prefixed_causal_attention(q, k, v, cache_len):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros_like(q)
    _check(lib().orc_prefixed_causal_attention_f32(q, k, v, q.shape[0], cache_len, q.shape[1],
                                                   k.shape[1], q.shape[2], out))
    return out


def causal_self_attention(q, k, v):
    return prefixed_causal_attention(q, k, v, 0)


def cached_prefixed_causal_attention(q, ck, cv, cache_len, ks, vs):
    q, ck, cv, ks, vs = (f32(x) for x in (q, ck, cv, ks, vs))
    out = np.zeros_like(q)
    _check(lib().orc_cached_prefixed_causal_attention_f32(q, ck, cv, cache_len, ks, vs,
                                                          q.shape[0], q.shape[1], ks.shape[1],
                                                          q.shape[2], out))
    return out


def decode_causal_attention(q, ck, cv, cache_len, kslot, vslot):
    q, ck, cv, kslot, vslot = (f32(x) for x in (q, ck, cv, kslot, vslot))
    out = np.zeros_like(q)
    _check(lib().orc_decode_causal_attention_f32(q, ck, cv, cache_len, kslot, vslot, q.shape[1],
                                                 kslot.shape[0], q.shape[2], out))
    return out


def silu(x):
    x = f32(x).copy()
    _check(lib().orc_silu_f32_in_place(x, x.size))
    return x


def mul(a, b):
    a = f32(a).copy()
    _check(lib().orc_mul_f32_in_place(a, f32(b), a.size))
    return a


def add(a, b):
    a = f32(a).copy()
    _check(lib().orc_add_f32_in_place(a, f32(b), a.size))
    return a


def f32_to_bf16(x) -> np.ndarray:
    x = f32(x)
    out = np.zeros(x.shape, np.uint16)
    lib().orc_f32_to_bf16_rne(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.zeros(x.shape, np.float32)
    lib().orc_bf16_to_f32(x.reshape(-1), out.reshape(-1), x.size)
    return out


def paged_decode_gather_attention(q, k_pages, v_pages, block_tables, context_lens, page_size):
    """Reference paged decode (gather + cached-prefixed attention) over pages laid out
    [num_blocks, page_size, Hkv, D]; q [B, Hq, D]."""
    q, kp, vp = f32(q), f32(k_pages), f32(v_pages)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    out = np.zeros_like(q)
    _check(lib().orc_paged_decode_gather_attention(q, kp, vp, bt, bt.shape[1], cl, q.shape[0],
                                                   q.shape[1], kp.shape[2], q.shape[2],
                                                   page_size, out), runtime=True)
    return out


# ----------------------------------------------------------------- paged KV storage
class PagedKvStorage:
    """runtime/paged_kv.rs PagedKvCacheStorage restated (per-layer pages, LIFO free list)."""

    def __init__(self, layers, kv_heads, head_dim, max_seq, page_size):
        self.h = lib().orc_paged_kv_create(layers, kv_heads, head_dim, max_seq, page_size)
        if not self.h:
            raise OracleError(6, lib().orc_runtime_last_error().decode())
        self.kv_heads, self.head_dim, self.page_size, self.max_seq = kv_heads, head_dim, page_size, max_seq

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_paged_kv_destroy(self.h)
            self.h = None

    def write_sequence(self, layer, start, k, v):
        k, v = f32(k), f32(v)
        _check(lib().orc_paged_kv_write_sequence(self.h, layer, start, k.shape[0], k, v), True)

    def write_slot(self, layer, pos, k, v):
        _check(lib().orc_paged_kv_write_slot(self.h, layer, pos, f32(k), f32(v)), True)

    def read_prefix(self, layer, length):
        k = np.zeros((length, self.kv_heads, self.head_dim), np.float32)
        v = np.zeros_like(k)
        _check(lib().orc_paged_kv_read_prefix(self.h, layer, length, k, v), True)
        return k, v

    def block_table(self, layer, tokens):
        cap = tokens // self.page_size + 2
        e = np.zeros((cap, 4), np.int64)
        n = I64()
        _check(lib().orc_paged_kv_block_table(self.h, layer, tokens, e, cap, C.byref(n)), True)
        return [tuple(int(x) for x in row) for row in e[: n.value]]

    def page_infos(self, layer):
        cap = self.max_seq // self.page_size + 2
        e = np.zeros((cap, 3), np.int64)
        n = I64()
        _check(lib().orc_paged_kv_page_infos(self.h, layer, e, cap, C.byref(n)), True)
        return [tuple(int(x) for x in row) for row in e[: n.value]]

    def allocated_pages(self, layer):
        return int(lib().orc_paged_kv_allocated_pages(self.h, layer))

    def free_pages(self, layer):
        return int(lib().orc_paged_kv_free_pages(self.h, layer))

    def reset(self):
        lib().orc_paged_kv_reset(self.h)

    def import_prefix_from(self, source: "PagedKvStorage", tokens: int):
        _check(lib().orc_paged_kv_import_prefix(self.h, source.h, tokens), True)


# ----------------------------------------------------------------- model / session / scheduler
class Model:
    """Decoder-only model (model/config.rs, model/decoder.rs); weights [in, out] like the
    reference's internal layout."""

    def __init__(self, hidden, intermediate, layers, heads, kv_heads, vocab, max_pos=4096,
                 eps=1e-6, theta=10000.0, rotary_dims=None, tie=False):
        head_dim = hidden // heads
        rotary = head_dim if rotary_dims is None else rotary_dims
        self.h = lib().orc_model_create(hidden, intermediate, layers, heads, kv_heads, vocab,
                                        max_pos, eps, theta, rotary, 1 if tie else 0)
        if not self.h:
            raise OracleError(6, lib().orc_runtime_last_error().decode())
        self.vocab, self.hidden = vocab, hidden

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_destroy(self.h)
            self.h = None

    def set_weight(self, name, array):
        a = f32(array).reshape(-1)
        _check(lib().orc_model_set_weight(self.h, name.encode(), a, a.size), True)

    def set_weights(self, weights: dict):
        for k, v in weights.items():
            self.set_weight(k, v)

    def forward_logits(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros((ids.size, self.vocab), np.float32)
        _check(lib().orc_model_forward_logits(self.h, ids, ids.size, out), True)
        return out


class Session:
    def __init__(self, model: Model, max_seq=4096, max_gen=512, page_size=0):
        self.model = model
        self.h = lib().orc_session_create(model.h, max_seq, max_gen, page_size)
        if not self.h:
            raise OracleError(6, lib().orc_runtime_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_session_destroy(self.h)
            self.h = None

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        _check(lib().orc_session_prefill(self.h, ids, ids.size), True)

    def step(self):
        t, p = C.c_uint32(), C.c_float()
        _check(lib().orc_session_step(self.h, C.byref(t), C.byref(p)), True)
        return int(t.value), float(p.value)

    def last_sample(self):
        t, p = C.c_uint32(), C.c_float()
        _check(lib().orc_session_last_sample(self.h, C.byref(t), C.byref(p)), True)
        return int(t.value), float(p.value)

    def last_hidden(self):
        out = np.zeros(self.model.hidden, np.float32)
        _check(lib().orc_session_last_hidden(self.h, out), True)
        return out

    @property
    def position(self):
        return int(lib().orc_session_position(self.h))

    def copy_prefix_from(self, source: "Session", tokens: int):
        _check(lib().orc_session_copy_prefix(self.h, source.h, tokens), True)

    def set_sampler(self, temperature=0.0, top_k=1, top_p=1.0, seed=0):
        """SamplerConfig (runtime/sampler.rs:3-43); restarts the sampler state."""
        _check(lib().orc_session_set_sampler(self.h, temperature, top_k, top_p, seed), True)

    @property
    def sampler_state(self) -> int:
        out = C.c_uint64()
        _check(lib().orc_session_sampler_state(self.h, C.byref(out)), True)
        return int(out.value)


class Scheduler:
    def __init__(self, model: Model, max_seq=4096, max_gen=512, page_size=16, max_batch=16,
                 max_chunk=256, max_batch_tokens=1024, max_consecutive_prefill=2, min_share=64,
                 sampler=None):
        """sampler: None (greedy) or (temperature, top_k, top_p, seed), the SessionConfig
        sampler of every submitted request."""
        self.model = model
        self.h = lib().orc_scheduler_create(model.h, max_seq, max_gen, page_size, max_batch,
                                            max_chunk, max_batch_tokens, max_consecutive_prefill,
                                            min_share)
        if not self.h:
            raise OracleError(6, lib().orc_runtime_last_error().decode())
        if sampler is not None:
            _check(lib().orc_scheduler_set_sampler(self.h, *sampler), True)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_scheduler_destroy(self.h)
            self.h = None

    def submit(self, ids, max_new_tokens=128, stop_token=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = C.c_uint64()
        _check(lib().orc_scheduler_submit(self.h, ids, ids.size, max_new_tokens,
                                          -1 if stop_token is None else stop_token,
                                          C.byref(out)), True)
        return int(out.value)

    def execute_next_tick(self):
        """Returns None or (kind, [update dicts]); the native call's wall time is kept in
        ``last_tick_seconds``."""
        ex = C.c_int32()
        t0 = time.perf_counter()
        status = lib().orc_scheduler_execute_next_tick(self.h, C.byref(ex))
        self.last_tick_seconds = time.perf_counter() - t0
        _check(status, True)
        if not ex.value:
            return None
        cap = 4096
        rows = np.zeros((cap, 9), np.int64)
        probs = np.zeros(cap, np.float32)
        kind = C.c_int32()
        n = I64()
        _check(lib().orc_scheduler_last_report(self.h, C.byref(kind), rows, probs, cap,
                                               C.byref(n)), True)
        updates = []
        for i in range(n.value):
            r = rows[i]
            rel = np.zeros((max(int(r[8]), 1), 3), np.int64)
            nr = I64()
            _check(lib().orc_scheduler_last_released(self.h, i, rel, rel.shape[0], C.byref(nr)),
                   True)
            updates.append(dict(sequence_id=int(r[0]), batch_kind=int(r[1]), reused=int(r[2]),
                                appended=int(r[3]), token=(int(r[5]) if r[4] else None),
                                probability=float(probs[i]), phase=int(r[6]),
                                finish_reason=int(r[7]),
                                released=[tuple(int(x) for x in row) for row in rel[: nr.value]]))
        return int(kind.value), updates

    def has_pending(self):
        return bool(lib().orc_scheduler_has_pending(self.h))

    def attach_packer(self, num_pages, page_size):
        """Packs every following tick over a global page pool (GlobalPagePacker)."""
        _check(lib().orc_scheduler_attach_packer(self.h, num_pages, page_size), True)

    def packed(self) -> dict:
        sizes = np.zeros(5, np.int64)
        _check(lib().orc_scheduler_packed_sizes(self.h, sizes), True)
        T, B, mb, nc, kind = (int(x) for x in sizes)
        out = dict(positions=np.zeros(T, np.int32), slot_mapping=np.zeros(T, np.int64),
                   cu_seqlens=np.zeros(B + 1, np.int32), context_lens=np.zeros(B, np.int32),
                   block_tables=np.zeros((B, mb), np.int32), copy_src=np.zeros(nc, np.int32),
                   copy_dst=np.zeros(nc, np.int32), copy_count=np.zeros(nc, np.int32),
                   sequence_ids=np.zeros(B, np.uint64))
        _check(lib().orc_scheduler_packed(self.h, out["positions"], out["slot_mapping"],
                                          out["cu_seqlens"], out["context_lens"],
                                          out["block_tables"], mb, out["copy_src"],
                                          out["copy_dst"], out["copy_count"],
                                          out["sequence_ids"]), True)
        out["kind"] = kind
        return out

    def session_blocks(self, seq, layer, tokens):
        """Page ids of a live sequence's own paged storage (None once it was released)."""
        out = np.zeros(tokens + 1, np.int64)
        n = I64()
        _check(lib().orc_scheduler_session_blocks(self.h, seq, layer, tokens, out, out.size,
                                                  C.byref(n)), True)
        return [int(x) for x in out[: n.value]] if n.value else None

    def packer_pages(self, seq):
        """Pages the packer holds for a sequence (empty once it finished)."""
        out = np.zeros(1 << 16, np.int32)
        n = I64()
        _check(lib().orc_scheduler_packer_pages(self.h, seq, out, out.size, C.byref(n)), True)
        return [int(x) for x in out[: n.value]]

    def packer_free_pages(self):
        n = I64()
        _check(lib().orc_scheduler_packer_free(self.h, C.byref(n)), True)
        return int(n.value)

    def generated(self, seq):
        out = np.zeros(65536, np.uint32)
        n = I64()
        _check(lib().orc_scheduler_generated(self.h, seq, out, out.size, C.byref(n)), True)
        return [int(x) for x in out[: n.value]]

    def block_ref_count(self, owner, layer, block):
        out = I64()
        _check(lib().orc_scheduler_block_ref_count(self.h, owner, layer, block, C.byref(out)),
               True)
        return int(out.value)


# ----------------------------------------------------------------- runtime units, one at a time
# (oracle_units_capi.cpp): the prefix index, prefix block manager, sequence state and KV cache
# on their own, so the reference's unit tests run against the restatement directly.
_UNITS_READY = False

FINISH_REASONS = {-1: None, 0: "StopToken", 1: "MaxNewTokens", 2: "SessionLimit", 3: "SequenceLength",
                  4: "Cancelled"}
PHASES = {0: "Prefill", 1: "Decode", 2: "Finished"}
BATCH_KINDS = {0: "Prefill", 1: "Decode"}


def _units():
    global _UNITS_READY
    L = lib()
    if _UNITS_READY:
        return L
    U32 = C.c_uint32
    P = C.POINTER
    sigs = {
        "orc_units_last_error": ([], C.c_char_p),
        "orc_prefix_index_create": ([I64], VP),
        "orc_prefix_index_destroy": ([VP], None),
        "orc_prefix_index_upsert": ([VP, C.c_uint64, U32P, I64, I64, I64], C.c_int32),
        "orc_prefix_index_best_match": ([VP, C.c_uint64, U32P, I64, P(C.c_int32), P(C.c_uint64), P(I64)],
                                        C.c_int32),
        "orc_block_manager_create": ([], VP),
        "orc_block_manager_destroy": ([VP], None),
        "orc_block_manager_update_owned": ([VP, C.c_uint64, C.c_int32, I64, I64, I64, I64P, I64P, I64P, I64,
                                            P(I64)], C.c_int32),
        "orc_block_manager_update_shared": ([VP, C.c_uint64, C.c_int32, C.c_uint64, I64, I64, I64, I64P, I64P,
                                             I64P, I64, P(I64)], C.c_int32),
        "orc_block_manager_remove": ([VP, C.c_uint64, I64P, I64, P(I64)], C.c_int32),
        "orc_block_manager_ref_count": ([VP, C.c_uint64, I64, I64], I64),
        "orc_block_manager_tracked": ([VP], I64),
        "orc_block_manager_prefixes": ([VP, C.c_uint64, P(C.c_int32), P(C.c_uint64)], C.c_int32),
        "orc_sequence_create": ([C.c_uint64, C.c_uint64, U32P, I64, I64, I64, I64], VP),
        "orc_sequence_destroy": ([VP], None),
        "orc_sequence_record_prefill": ([VP, I64], None),
        "orc_sequence_record_generated": ([VP, U32], None),
        "orc_sequence_finish": ([VP, C.c_int32], None),
        "orc_sequence_query": ([VP, I64P], None),
        "orc_sequence_generated": ([VP, U32P, I64], I64),
        "orc_sequence_next_chunk": ([VP, I64, U32P, I64], I64),
        "orc_kvcache_create": ([I64] * 5, VP),
        "orc_kvcache_destroy": ([VP], None),
        "orc_kvcache_reserve_slot": ([VP, P(I64)], C.c_int32),
        "orc_kvcache_advance": ([VP, I64], C.c_int32),
        "orc_kvcache_write": ([VP, I64, I64, F32P, F32P], C.c_int32),
        "orc_kvcache_write_uncommitted": ([VP, I64, I64, F32P, F32P], C.c_int32),
        "orc_kvcache_write_sequence_uncommitted": ([VP, I64, I64, I64, F32P, F32P], C.c_int32),
        "orc_kvcache_read_prefix": ([VP, I64, I64, F32P, F32P], C.c_int32),
        "orc_kvcache_counts": ([VP, I64P], None),
        "orc_kvcache_reset": ([VP], None),
        "orc_kvcache_prefix_handle": ([VP, I64, P(C.c_int32), I64P, I64P, I64, I64P, I64], C.c_int32),
        "orc_kvcache_copy_prefix_from": ([VP, VP, I64], C.c_int32),
        "orc_session_history": ([VP, U32P, I64, P(I64)], C.c_int32),
        "orc_session_kv_counts": ([VP, I64P], None),
        "orc_session_prefix_handle": ([VP, I64, P(C.c_int32), I64P, I64P, I64, I64P, I64], C.c_int32),
        "orc_session_generate": ([VP, U32P, I64, I64, I64, U32P, F32P, I64, P(I64), P(C.c_int32)], C.c_int32),
        "orc_scheduler_plan": ([VP, P(C.c_int32), P(C.c_int32), np.ctypeslib.ndpointer(np.uint64), I64, P(I64)],
                               C.c_int32),
        "orc_scheduler_sequence": ([VP, C.c_uint64, I64P], C.c_int32),
        "orc_scheduler_resident_sessions": ([VP], I64),
        "orc_scheduler_shared_prefix": ([VP, C.c_uint64, P(C.c_int32), P(C.c_uint64)], C.c_int32),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _UNITS_READY = True
    return L


def _ucheck(status: int):
    if status != 0:
        raise OracleError(status, (_units().orc_units_last_error() or b"").decode())


def _ids(tokens) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))


def _flatten_handle(handle: dict):
    """handle = {token_count, page_size, layers: [[(logical, block_id, start, count), ...], ...]}"""
    layers = handle["layers"]
    counts = np.array([len(l) for l in layers] or [0], np.int64)
    rows = [e for l in layers for e in l]
    entries = np.array(rows or [(0, 0, 0, 0)], np.int64).reshape(-1, 4)
    return handle["token_count"], handle["page_size"], len(layers), counts, np.ascontiguousarray(entries)


def _read_handle(fn, *args):
    has = C.c_int32()
    header = np.zeros(3, np.int64)
    counts = np.zeros(256, np.int64)
    entries = np.zeros((1 << 14, 4), np.int64)
    _ucheck(fn(*args, C.byref(has), header, counts, counts.size, entries, entries.shape[0]))
    if not has.value:
        return None
    layers, k = [], 0
    for l in range(int(header[2])):
        n = int(counts[l])
        layers.append([tuple(int(x) for x in entries[k + i]) for i in range(n)])
        k += n
    return {"token_count": int(header[0]), "page_size": int(header[1]), "layers": layers}


def _released(buf, n):
    return [tuple(int(x) for x in buf[i]) for i in range(n)]


class PrefixIndex:
    """runtime/prefix_index.rs:24-113."""

    def __init__(self, min_prefix_share_tokens: int):
        self.h = _units().orc_prefix_index_create(min_prefix_share_tokens)

    def __del__(self):
        if getattr(self, "h", None):
            _units().orc_prefix_index_destroy(self.h)
            self.h = None

    def upsert(self, sequence_id, prompt_tokens, cached_prompt_tokens, session_position):
        t = _ids(prompt_tokens)
        _ucheck(_units().orc_prefix_index_upsert(self.h, sequence_id, t, t.size, cached_prompt_tokens,
                                                 session_position))

    def best_match(self, target_sequence_id, target_prompt_tokens):
        """(sequence_id, shared_prefix_tokens) or None."""
        t = _ids(target_prompt_tokens)
        found, seq, shared = C.c_int32(), C.c_uint64(), I64()
        _ucheck(_units().orc_prefix_index_best_match(self.h, target_sequence_id, t, t.size, C.byref(found),
                                                     C.byref(seq), C.byref(shared)))
        return (int(seq.value), int(shared.value)) if found.value else None


class PrefixBlockManager:
    """runtime/block_manager.rs:58-172; released blocks are (owner, layer, block_id)."""

    def __init__(self):
        self.h = _units().orc_block_manager_create()
        self._buf = np.zeros((1 << 14, 3), np.int64)

    def __del__(self):
        if getattr(self, "h", None):
            _units().orc_block_manager_destroy(self.h)
            self.h = None

    def update_owned_prefix(self, sequence_id, handle):
        n = I64()
        if handle is None:
            z = np.zeros(1, np.int64)
            _ucheck(_units().orc_block_manager_update_owned(self.h, sequence_id, 0, 0, 0, 0, z,
                                                            np.zeros((1, 4), np.int64), self._buf,
                                                            self._buf.shape[0], C.byref(n)))
        else:
            tc, ps, nl, counts, entries = _flatten_handle(handle)
            _ucheck(_units().orc_block_manager_update_owned(self.h, sequence_id, 1, tc, ps, nl, counts, entries,
                                                            self._buf, self._buf.shape[0], C.byref(n)))
        return _released(self._buf, n.value)

    def update_shared_prefix(self, sequence_id, assignment):
        """assignment = None or (source_sequence_id, handle)."""
        n = I64()
        if assignment is None:
            _ucheck(_units().orc_block_manager_update_shared(self.h, sequence_id, 0, 0, 0, 0, 0,
                                                             np.zeros(1, np.int64), np.zeros((1, 4), np.int64),
                                                             self._buf, self._buf.shape[0], C.byref(n)))
        else:
            source, handle = assignment
            tc, ps, nl, counts, entries = _flatten_handle(handle)
            _ucheck(_units().orc_block_manager_update_shared(self.h, sequence_id, 1, source, tc, ps, nl, counts,
                                                             entries, self._buf, self._buf.shape[0], C.byref(n)))
        return _released(self._buf, n.value)

    def remove_sequence(self, sequence_id):
        n = I64()
        _ucheck(_units().orc_block_manager_remove(self.h, sequence_id, self._buf, self._buf.shape[0], C.byref(n)))
        return _released(self._buf, n.value)

    def block_ref_count(self, owner, layer, block_id):
        return int(_units().orc_block_manager_ref_count(self.h, owner, layer, block_id))

    def tracked_block_count(self):
        return int(_units().orc_block_manager_tracked(self.h))

    def prefixes(self, sequence_id):
        """(has owned prefix, shared prefix source or None)."""
        flags, source = C.c_int32(), C.c_uint64()
        _ucheck(_units().orc_block_manager_prefixes(self.h, sequence_id, C.byref(flags), C.byref(source)))
        return bool(flags.value & 1), (int(source.value) if flags.value & 2 else None)


class SequenceState:
    """runtime/sequence.rs:43-205 (new / with_generation_budget)."""

    _FIELDS = ("request_id", "sequence_id", "prompt_len", "generated_len", "cached_tokens",
               "cached_prompt_tokens", "pending_prompt_tokens", "requested_max_new_tokens", "max_new_tokens",
               "stop_token_id", "phase", "finish_reason", "is_finished", "generation_budget_reached",
               "generation_budget_finish_reason", "total_tokens")

    def __init__(self, request_id, sequence_id, prompt_tokens, max_new_tokens, stop_token_id=None,
                 generation_budget=None):
        t = _ids(prompt_tokens)
        budget = max_new_tokens if generation_budget is None else generation_budget
        self.h = _units().orc_sequence_create(request_id, sequence_id, t, t.size, max_new_tokens, budget,
                                              -1 if stop_token_id is None else stop_token_id)

    def __del__(self):
        if getattr(self, "h", None):
            _units().orc_sequence_destroy(self.h)
            self.h = None

    def state(self) -> dict:
        f = np.zeros(16, np.int64)
        _units().orc_sequence_query(self.h, f)
        d = dict(zip(self._FIELDS, (int(x) for x in f)))
        d["stop_token_id"] = None if d["stop_token_id"] < 0 else d["stop_token_id"]
        d["phase"] = PHASES[d["phase"]]
        d["finish_reason"] = FINISH_REASONS[d["finish_reason"]]
        d["generation_budget_finish_reason"] = FINISH_REASONS[d["generation_budget_finish_reason"]]
        d["is_finished"] = bool(d["is_finished"])
        d["generation_budget_reached"] = bool(d["generation_budget_reached"])
        return d

    def generated_tokens(self):
        out = np.zeros(1 << 12, np.uint32)
        n = _units().orc_sequence_generated(self.h, out, out.size)
        return [int(x) for x in out[:n]]

    def next_prefill_chunk(self, max_chunk_tokens):
        out = np.zeros(max(max_chunk_tokens, 1), np.uint32)
        n = _units().orc_sequence_next_chunk(self.h, max_chunk_tokens, out, out.size)
        return [int(x) for x in out[:n]]

    def record_prefill(self, appended):
        _units().orc_sequence_record_prefill(self.h, appended)

    def record_generated_token(self, token):
        _units().orc_sequence_record_generated(self.h, token)

    def finish(self, reason: str):
        code = {v: k for k, v in FINISH_REASONS.items()}[reason]
        _units().orc_sequence_finish(self.h, code)


class KvCache:
    """runtime/kv_cache.rs:359-597: contiguous (page_size 0) or paged storage."""

    def __init__(self, layers, kv_heads, head_dim, max_seq, page_size=0):
        self.h = _units().orc_kvcache_create(layers, kv_heads, head_dim, max_seq, page_size)
        if not self.h:
            raise OracleError(6, (_units().orc_units_last_error() or b"").decode())
        self.kv_heads, self.head_dim = kv_heads, head_dim

    def __del__(self):
        if getattr(self, "h", None):
            _units().orc_kvcache_destroy(self.h)
            self.h = None

    def counts(self) -> dict:
        c = np.zeros(5, np.int64)
        _units().orc_kvcache_counts(self.h, c)
        return dict(used_tokens=int(c[0]), remaining_tokens=int(c[1]), paged=bool(c[2]), layers=int(c[3]),
                    layer_elements=int(c[4]))

    def reserve_slot(self):
        pos = I64()
        _ucheck(_units().orc_kvcache_reserve_slot(self.h, C.byref(pos)))
        return int(pos.value)

    def advance(self, n):
        _ucheck(_units().orc_kvcache_advance(self.h, n))

    def reset(self):
        _units().orc_kvcache_reset(self.h)

    def write(self, layer, position, key, value):
        _ucheck(_units().orc_kvcache_write(self.h, layer, position, f32(key).reshape(-1), f32(value).reshape(-1)))

    def write_uncommitted(self, layer, position, key, value):
        _ucheck(_units().orc_kvcache_write_uncommitted(self.h, layer, position, f32(key).reshape(-1),
                                                       f32(value).reshape(-1)))

    def write_sequence_uncommitted(self, layer, start, keys, values):
        k, v = f32(keys), f32(values)
        n = k.size // (self.kv_heads * self.head_dim)
        _ucheck(_units().orc_kvcache_write_sequence_uncommitted(self.h, layer, start, n, k.reshape(-1),
                                                                v.reshape(-1)))

    def read_prefix(self, layer, length):
        k = np.zeros((length, self.kv_heads, self.head_dim), np.float32)
        v = np.zeros_like(k)
        _ucheck(_units().orc_kvcache_read_prefix(self.h, layer, length, k.reshape(-1), v.reshape(-1)))
        return k, v

    def prefix_handle(self, token_count):
        return _read_handle(_units().orc_kvcache_prefix_handle, self.h, token_count)

    def copy_prefix_from(self, source: "KvCache", token_count):
        _ucheck(_units().orc_kvcache_copy_prefix_from(self.h, source.h, token_count))


def session_token_history(session: Session):
    out = np.zeros(1 << 16, np.uint32)
    n = I64()
    _ucheck(_units().orc_session_history(session.h, out, out.size, C.byref(n)))
    return [int(x) for x in out[: n.value]]


def session_kv_used_tokens(session: Session) -> int:
    c = np.zeros(2, np.int64)
    _units().orc_session_kv_counts(session.h, c)
    return int(c[0])


def session_kv_is_paged(session: Session) -> bool:
    c = np.zeros(2, np.int64)
    _units().orc_session_kv_counts(session.h, c)
    return bool(c[1])


def session_prefix_handle(session: Session, token_count: int):
    return _read_handle(_units().orc_session_prefix_handle, session.h, token_count)


def session_generate_from_tokens(session: Session, prompt, max_new_tokens, stop_token_id=None):
    """Session::generate_reference_from_tokens (session.rs:276-331): ([(token, prob)], finish)."""
    t = _ids(prompt)
    cap = max(int(max_new_tokens), 1)
    toks = np.zeros(cap, np.uint32)
    probs = np.zeros(cap, np.float32)
    n, finish = I64(), C.c_int32()
    _ucheck(_units().orc_session_generate(session.h, t, t.size, max_new_tokens,
                                          -1 if stop_token_id is None else stop_token_id, toks, probs, cap,
                                          C.byref(n), C.byref(finish)))
    return [(int(toks[i]), float(probs[i])) for i in range(n.value)], FINISH_REASONS[finish.value]


def scheduler_plan_next_tick(sched: Scheduler):
    """ReferenceScheduler::plan_next_tick: None or (batch kind, [sequence ids])."""
    has, kind, n = C.c_int32(), C.c_int32(), I64()
    ids = np.zeros(4096, np.uint64)
    _ucheck(_units().orc_scheduler_plan(sched.h, C.byref(has), C.byref(kind), ids, ids.size, C.byref(n)))
    if not has.value:
        return None
    return BATCH_KINDS[kind.value], [int(x) for x in ids[: n.value]]


def scheduler_sequence_state(sched: Scheduler, seq: int) -> dict:
    out = np.zeros(5, np.int64)
    _ucheck(_units().orc_scheduler_sequence(sched.h, seq, out))
    return dict(phase=PHASES[int(out[0])], finish_reason=FINISH_REASONS[int(out[1])], cached_tokens=int(out[2]),
                generated_len=int(out[3]), has_session=bool(out[4]))


def scheduler_resident_session_count(sched: Scheduler) -> int:
    return int(_units().orc_scheduler_resident_sessions(sched.h))


def scheduler_shared_prefix_source(sched: Scheduler, seq: int):
    has, source = C.c_int32(), C.c_uint64()
    _ucheck(_units().orc_scheduler_shared_prefix(sched.h, seq, C.byref(has), C.byref(source)))
    return int(source.value) if has.value else None
