"""ctypes binding of libferrisinfer_runtime.so (include/ferrisinfer_runtime.h): the host
runtime that keeps the reference's ReferenceScheduler API and runs each tick as one packed
ragged batch on the HIP backend."""
from __future__ import annotations

import ctypes as C
import os
import time

import numpy as np

from .kernel import DTYPE_BF16, DTYPE_F16, DTYPE_F32, FerrisError, PKG_DIR, load as load_kernel

LIB_PATH = os.path.join(PKG_DIR, "libferrisinfer_runtime.so")


class ModelConfig(C.Structure):
    _fields_ = [("hidden_size", C.c_int32), ("intermediate_size", C.c_int32),
                ("num_layers", C.c_int32), ("num_attention_heads", C.c_int32),
                ("num_key_value_heads", C.c_int32), ("vocab_size", C.c_int32),
                ("max_position_embeddings", C.c_int32), ("rms_norm_eps", C.c_float),
                ("rope_theta", C.c_float), ("rotary_dims", C.c_int32),
                ("tie_word_embeddings", C.c_int32)]


class RuntimeConfig(C.Structure):
    _fields_ = [("max_sequence_length", C.c_int64), ("max_generated_tokens", C.c_int64),
                ("max_batch_size", C.c_int64), ("max_prefill_chunk_tokens", C.c_int64),
                ("max_prefill_batch_tokens", C.c_int64),
                ("max_consecutive_prefill_ticks", C.c_int64),
                ("min_prefix_share_tokens", C.c_int64), ("num_blocks", C.c_int32),
                ("block_size", C.c_int32), ("kv_dtype", C.c_int32),
                ("temperature", C.c_float), ("top_k", C.c_int64), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64),
                ("weight_dtype", C.c_int32), ("graph_decode", C.c_int32)]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        load_kernel()  # raises when the HIP backend is missing
        if not os.path.exists(LIB_PATH):
            raise FerrisError(8, f"host runtime {LIB_PATH} is not built; run "
                                 "`python -m ferrisinfer_amd.build`")
        L = C.CDLL(LIB_PATH)
        sig = {
            "fr_create": [_I32, C.POINTER(ModelConfig), C.POINTER(RuntimeConfig), C.POINTER(_P)],
            "fr_destroy": [_P],
            "fr_set_weight": [_P, C.c_char_p, _P, _I64],
            "fr_set_weight_device": [_P, C.c_char_p, _P, _I32, _I64],
            "fr_submit": [_P, _P, _I64, _I64, _I64, C.POINTER(C.c_uint64)],
            "fr_execute_next_tick": [_P, C.POINTER(_I32)],
            "fr_execute_next_tick_ex": [_P, _I32, C.POINTER(_I32)],
            "fr_run_ahead_counters": [_P, _P],
            "fr_has_pending": [_P],
            "fr_last_report": [_P, C.POINTER(_I32), _P, _P, _I64, C.POINTER(_I64)],
            "fr_last_released": [_P, _I64, _P, _I64, C.POINTER(_I64)],
            "fr_generated": [_P, C.c_uint64, _P, _I64, C.POINTER(_I64)],
            "fr_sequence_blocks": [_P, C.c_uint64, _P, _I64, C.POINTER(_I64)],
            "fr_pool_free_count": [_P, C.POINTER(_I64)],
            "fr_graph_counters": [_P, _P],
            "fr_last_batch_sizes": [_P, _P],
            "fr_last_logits": [_P, _P, _I64, C.POINTER(_I64)],
            "fr_last_batch": [_P] + [_P] * 10,
            "fr_last_tick_profile": [_P, _P],
            "fr_hf_read_config": [C.c_char_p, C.POINTER(ModelConfig)],
            "fr_hf_inspect": [C.c_char_p, _P],
            "fr_safetensors_info": [C.c_char_p, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64)],
            "fr_safetensors_entry": [C.c_char_p, C.c_char_p, C.POINTER(_I32), _P, _I32, C.POINTER(_I32),
                                     C.c_char_p, _I64, C.POINTER(_I64), C.POINTER(_I64)],
            "fr_load_hf_weights": [_P, C.c_char_p, C.POINTER(_I64)],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _I32
        L.fr_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def _check(status):
    if status != 0:
        raise FerrisError(int(status), (load().fr_last_error() or b"").decode(errors="replace"))


def _addr(a: np.ndarray) -> int:
    return a.ctypes.data


def _path(p) -> bytes:
    return os.fsencode(os.fspath(p))


def read_hf_config(model_dir) -> dict:
    """config.json of a Qwen2 checkpoint as Runtime keyword arguments (io/hf.rs:306-369)."""
    mc = ModelConfig()
    _check(load().fr_hf_read_config(_path(model_dir), C.byref(mc)))
    return {"hidden": mc.hidden_size, "intermediate": mc.intermediate_size, "layers": mc.num_layers,
            "heads": mc.num_attention_heads, "kv_heads": mc.num_key_value_heads, "vocab": mc.vocab_size,
            "max_pos": mc.max_position_embeddings, "eps": mc.rms_norm_eps, "theta": mc.rope_theta,
            "rotary_dims": mc.rotary_dims, "tie": bool(mc.tie_word_embeddings)}


def hf_inspect(model_dir) -> dict:
    """io/hf.rs:66-118 HfSource::inspect counts (the tokenizer is not read)."""
    c = np.zeros(8, np.int64)
    _check(load().fr_hf_inspect(_path(model_dir), _addr(c)))
    keys = ("shard_count", "tensor_count", "total_data_bytes", "mapped_required", "mapped_optional",
            "missing_required", "missing_optional", "shape_mismatches")
    out = {k: int(v) for k, v in zip(keys, c)}
    out["compatible"] = out["missing_required"] == 0 and out["shape_mismatches"] == 0
    return out


def safetensors_info(model_dir) -> dict:
    """io/safetensors.rs SafeTensorsRepository::open + tensor_count / shard_count / total_data_bytes."""
    t, s, b = _I64(), _I64(), _I64()
    _check(load().fr_safetensors_info(_path(model_dir), C.byref(t), C.byref(s), C.byref(b)))
    return {"tensors": t.value, "shards": s.value, "total_data_bytes": b.value}


def safetensors_entry(model_dir, name) -> dict:
    """One tensor's entry: dtype code, shape, shard path, absolute data offset and length."""
    dtype, rank = _I32(), _I32()
    shape = np.zeros(16, np.int64)
    path = C.create_string_buffer(4096)
    off, n = _I64(), _I64()
    _check(load().fr_safetensors_entry(_path(model_dir), name.encode(), C.byref(dtype), _addr(shape), 16,
                                       C.byref(rank), path, 4096, C.byref(off), C.byref(n)))
    return {"dtype": dtype.value, "shape": [int(x) for x in shape[:rank.value]],
            "path": os.fsdecode(path.value), "offset": off.value, "byte_len": n.value}


class Runtime:
    """A model, a KV block pool and a ReferenceScheduler-compatible scheduler on one GPU."""

    def __init__(self, hidden, intermediate, layers, heads, kv_heads, vocab, max_pos=4096,
                 eps=1e-6, theta=10000.0, rotary_dims=None, tie=False, max_seq=4096,
                 max_gen=512, max_batch=16, max_chunk=256, max_batch_tokens=1024,
                 max_consecutive_prefill=2, min_share=64, num_blocks=4096, block_size=16,
                 kv_dtype="f32", ordinal=0, sampler=None, weight_dtype="f32", graph_decode=False):
        """sampler: None (greedy) or (temperature, top_k, top_p, seed), the SamplerConfig of
        every session (runtime/sampler.rs:3-43).  weight_dtype "f32" or "bf16": storage of the
        packed projections and head.  graph_decode: replay decode ticks from HIP graphs."""
        L = load()
        temperature, top_k, top_p, seed = (0.0, 1, 1.0, 0) if sampler is None else sampler
        head_dim = hidden // heads
        mc = ModelConfig(hidden, intermediate, layers, heads, kv_heads, vocab, max_pos, eps, theta,
                         head_dim if rotary_dims is None else rotary_dims, 1 if tie else 0)
        rc = RuntimeConfig(max_seq, max_gen, max_batch, max_chunk, max_batch_tokens,
                           max_consecutive_prefill, min_share, num_blocks, block_size,
                           DTYPE_F32 if kv_dtype == "f32" else DTYPE_BF16,
                           temperature, top_k, top_p, 1.0, seed,
                           DTYPE_F32 if weight_dtype == "f32" else DTYPE_BF16,
                           1 if graph_decode else 0)
        h = _P()
        _check(L.fr_create(ordinal, C.byref(mc), C.byref(rc), C.byref(h)))
        self.h = h
        self._ahead_used = False  # a call asked to run ahead: later ticks may have started early
        self._last_return = None  # perf_counter when the last execute call returned
        self.vocab = vocab

    def close(self):
        if getattr(self, "h", None):
            _check(load().fr_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run_ahead_counters(self) -> dict:
        """Ticks enqueued ahead, kept, dropped; whether the last tick was one enqueued ahead."""
        out = np.zeros(4, np.uint64)
        _check(load().fr_run_ahead_counters(self.h, _addr(out)))
        return dict(launched=int(out[0]), kept=int(out[1]), dropped=int(out[2]), last_ahead=bool(out[3]))

    def graph_counters(self) -> dict:
        """Decode ticks replayed from graphs, graphs captured, graphs dropped."""
        out = np.zeros(3, np.uint64)
        _check(load().fr_graph_counters(self.h, _addr(out)))
        return dict(replays=int(out[0]), captures=int(out[1]), drops=int(out[2]))

    def set_weight(self, name, array):
        a = np.ascontiguousarray(np.asarray(array, dtype=np.float32)).reshape(-1)
        _check(load().fr_set_weight(self.h, name.encode(), _addr(a), a.size))

    def set_weight_device(self, name, tensor):
        """set_weight from a contiguous torch tensor on this runtime's GPU (float32, bfloat16 or
        float16), widened to f32 on the device."""
        import torch

        dtypes = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}
        if not tensor.is_cuda or not tensor.is_contiguous() or tensor.dtype not in dtypes:
            raise FerrisError(6, "set_weight_device takes a contiguous f32 / bf16 / f16 device tensor")
        _check(load().fr_set_weight_device(self.h, name.encode(), tensor.data_ptr(), dtypes[tensor.dtype],
                                           tensor.numel()))

    @classmethod
    def from_hf(cls, model_dir, **kwargs):
        """A runtime for the Qwen2 checkpoint under model_dir: config.json gives the model
        shape, every planned tensor is loaded on the device (fr_load_hf_weights); kwargs are
        the runtime options of __init__."""
        cfg = read_hf_config(model_dir)
        cfg["max_pos"] = kwargs.pop("max_pos", cfg["max_pos"])
        rt = cls(**cfg, **kwargs)
        rt.load_hf_weights(model_dir)
        return rt

    def load_hf_weights(self, model_dir) -> int:
        """Every planned tensor of the checkpoint into this runtime's model; returns the count."""
        n = _I64()
        _check(load().fr_load_hf_weights(self.h, _path(model_dir), C.byref(n)))
        return n.value

    def set_weights(self, weights: dict):
        for k, v in weights.items():
            self.set_weight(k, v)

    def submit(self, ids, max_new_tokens=128, stop_token=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = C.c_uint64()
        _check(load().fr_submit(self.h, _addr(ids), ids.size, max_new_tokens,
                                -1 if stop_token is None else stop_token, C.byref(out)))
        return int(out.value)

    def execute_next_tick(self, run_ahead=False):
        """Returns None or (kind, [update dicts]) in the oracle Scheduler's format.  The wall
        time of the native tick (host scheduling, the batched forward, the sample download) is
        kept in ``last_tick_seconds``.

        run_ahead (FR_TICK_RUN_AHEAD): also enqueue the next tick when it will be a decode tick,
        so the device runs it while this call returns; the results are those of calls
        without it.  A tick that ran ahead started on the device during the previous call, so
        its ``last_tick_seconds`` is the time since the previous call returned (the caller's
        time in between included), not the call's own duration."""
        L = load()
        ex = C.c_int32()
        t0 = time.perf_counter()
        if run_ahead or self._ahead_used:
            self._ahead_used = True
            status = L.fr_execute_next_tick_ex(self.h, 1 if run_ahead else 0, C.byref(ex))
        else:
            status = L.fr_execute_next_tick(self.h, C.byref(ex))
        t1 = time.perf_counter()
        self.last_tick_seconds = t1 - t0
        _check(status)
        if self._ahead_used and self._last_return is not None and self.run_ahead_counters()["last_ahead"]:
            self.last_tick_seconds = t1 - self._last_return
        self._last_return = t1
        if not ex.value:
            return None
        cap = 4096
        rows = np.zeros((cap, 9), np.int64)
        probs = np.zeros(cap, np.float32)
        kind = C.c_int32()
        n = _I64()
        _check(L.fr_last_report(self.h, C.byref(kind), _addr(rows), _addr(probs), cap, C.byref(n)))
        updates = []
        for i in range(n.value):
            r = rows[i]
            rel = np.zeros((max(int(r[8]), 1), 3), np.int64)
            nr = _I64()
            _check(L.fr_last_released(self.h, i, _addr(rel), rel.shape[0], C.byref(nr)))
            updates.append(dict(sequence_id=int(r[0]), batch_kind=int(r[1]), reused=int(r[2]),
                                appended=int(r[3]), token=(int(r[5]) if r[4] else None),
                                probability=float(probs[i]), phase=int(r[6]),
                                finish_reason=int(r[7]),
                                released=[tuple(int(x) for x in row) for row in rel[: nr.value]]))
        return int(kind.value), updates

    def has_pending(self):
        return bool(load().fr_has_pending(self.h))

    def generated(self, seq):
        out = np.zeros(65536, np.uint32)
        n = _I64()
        _check(load().fr_generated(self.h, seq, _addr(out), out.size, C.byref(n)))
        return [int(x) for x in out[: n.value]]

    def sequence_blocks(self, seq):
        out = np.zeros(65536, np.int32)
        n = _I64()
        _check(load().fr_sequence_blocks(self.h, seq, _addr(out), out.size, C.byref(n)))
        return [int(x) for x in out[: n.value]]

    def pool_free_count(self):
        n = _I64()
        _check(load().fr_pool_free_count(self.h, C.byref(n)))
        return int(n.value)

    def last_tick_profile(self) -> dict:
        """Host seconds of the last tick: scheduling, enqueue, wait, total."""
        out = np.zeros(4, np.float64)
        _check(load().fr_last_tick_profile(self.h, _addr(out)))
        return dict(schedule=float(out[0]), enqueue=float(out[1]), wait=float(out[2]),
                    total=float(out[3]))

    def last_batch_context_sum(self) -> int:
        """Sum of the context lengths of the last tick's packed batch (its KV tokens read)."""
        return int(self.last_batch()["context_lens"].sum())

    def last_logits(self) -> np.ndarray:
        """The logits rows the last tick sampled from ([B, vocab] f32, the batch's sequence
        order); empty after a greedy tick."""
        B = int(self.last_batch()["sequence_ids"].size)
        out = np.zeros((B, self.vocab), np.float32)
        rows = _I64()
        _check(load().fr_last_logits(self.h, _addr(out), out.size, C.byref(rows)))
        return out[: rows.value]

    def last_batch(self) -> dict:
        L = load()
        sizes = np.zeros(7, np.int64)
        _check(L.fr_last_batch_sizes(self.h, _addr(sizes)))
        T, B, mb, nc, kind, mq, mctx = (int(x) for x in sizes)
        arr = dict(token_ids=np.zeros(T, np.int32), positions=np.zeros(T, np.int32),
                   slot_mapping=np.zeros(T, np.int64), cu_seqlens=np.zeros(B + 1, np.int32),
                   context_lens=np.zeros(B, np.int32), block_tables=np.zeros((B, mb), np.int32),
                   copy_src=np.zeros(nc, np.int32), copy_dst=np.zeros(nc, np.int32),
                   copy_count=np.zeros(nc, np.int32), sequence_ids=np.zeros(B, np.uint64))
        order = ["token_ids", "positions", "slot_mapping", "cu_seqlens", "context_lens",
                 "block_tables", "copy_src", "copy_dst", "copy_count", "sequence_ids"]
        _check(L.fr_last_batch(self.h, *[_addr(arr[k]) for k in order]))
        arr.update(kind=kind, max_query_len=mq, max_context_len=mctx)
        return arr
