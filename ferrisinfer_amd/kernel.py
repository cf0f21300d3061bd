"""ctypes binding of libferrisinfer_kernel.so (the C ABI in include/ferrisinfer_kernel.h).

The shared library is the product: every op here calls straight into the HIP backend and
raises :class:`FerrisError` with the reference's error kinds (core/error.rs:5-16) when it
fails.  There is no fallback path: if the library is missing, importing ops raises.

torch is used only as plumbing for device memory and streams: tensors are passed by
``data_ptr()`` and the context enqueues on torch's current stream.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libferrisinfer_kernel.so")

ERROR_KINDS = ["Io", "Parse", "InvalidShape", "InvalidLayout", "InvalidType", "InvalidConfig",
               "MissingWeight", "Unsupported", "Runtime"]

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2


class FerrisError(RuntimeError):
    """FerrisError{kind, message} (core/error.rs:18-48) raised from a non-zero status."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = ERROR_KINDS[status - 1] if 0 < status <= len(ERROR_KINDS) else f"status{status}"
        self.message = message
        super().__init__(f"{self.kind}: {message}")


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_F32 = C.c_float
_SZ = C.c_size_t

# name -> argtypes; every function returns int32 status unless listed in _RESTYPES.
_SIGNATURES = {
    "fi_ctx_create": [_I32, C.POINTER(_P)],
    "fi_convert_to_f32": [_P, _P, _I32, _I64, _I64, _I32, _P],
    "fi_ctx_destroy": [_P],
    "fi_ctx_sync": [_P],
    "fi_ctx_set_stream": [_P, _P],
    "fi_ctx_stream": [_P],
    "fi_ctx_check_faults": [_P],
    "fi_device_info": [_P, C.c_char_p, _SZ, C.c_char_p, _SZ, C.POINTER(C.c_uint64), C.POINTER(_I32)],
    "fi_buf_alloc": [_P, _SZ, C.POINTER(_P)],
    "fi_buf_free": [_P, _P],
    "fi_buf_upload": [_P, _P, _SZ, _P, _SZ],
    "fi_buf_download": [_P, _P, _SZ, _P, _SZ],
    "fi_buf_zero": [_P, _P, _SZ],
    "fi_host_alloc": [_P, _SZ, C.POINTER(_P)],
    "fi_host_free": [_P, _P],
    "fi_buf_upload_async": [_P, _P, _SZ, _P, _SZ],
    "fi_buf_download_async": [_P, _P, _SZ, _P, _SZ],
    "fi_ctx_faults_async": [_P, _P],
    "fi_event_create": [_P, C.POINTER(_P)],
    "fi_event_record": [_P, _P],
    "fi_event_wait": [_P],
    "fi_event_destroy": [_P],
    "fi_token_feed": [_P, _P, _I32, _P, _I32, _P],
    "fi_kv_append": [_P, _P, _P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32],
    "fi_kv_copy_blocks": [_P, _P, _P, _I32, _P, _P, _P, _I32, _I32, _I32, _I32, _I32],
    "fi_kv_gather": [_P, _P, _P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P],
    "fi_attn_decode_paged": [_P, _P, _P, _P, _I32, _P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _I32,
                             _I32, _F32, _P],
    "fi_attn_decode_paged_qkv": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _I32, _P, _I32,
                                 _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _P],
    "fi_attn_decode_paged_noalloc": [_P, _P, _P, _P, _I32, _P, _I32, _P, _I32, _I32, _I32, _I32, _I32,
                                     _I32, _I32, _F32, _P],
    "fi_attn_prefill_paged": [_P, _P, _P, _P, _I32, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32,
                              _I32, _I32, _F32, _P],
    "fi_rms_norm": [_P, _P, _P, _P, _I32, _I32, _F32],
    "fi_add_rms_norm": [_P, _P, _P, _P, _P, _P, _I32, _I32, _F32],
    "fi_rope": [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32],
    "fi_rope_table": [_P, _I32, _I32, _I32, _F32, _P, _P],
    "fi_embedding": [_P, _P, _I32, _I32, _P, _I32, _P],
    "fi_silu_mul": [_P, _P, _P, _I64],
    "fi_add": [_P, _P, _P, _I64],
    "fi_gemm": [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32],
    "fi_lm_head_argmax": [_P, _P, _P, _I32, _I32, _I32, _P, _P],
    "fi_weight_packed_floats": [_I32, _I32, _I32, C.POINTER(_SZ)],
    "fi_weight_pack": [_P, _P, _I32, _I32, _I32, _I32, _P],
    "fi_weight_pack_pair": [_P, _P, _P, _I32, _I32, _P],
    "fi_gemm_packed_splits": [_P, _I32, _I32, _I32, _I32, C.POINTER(_I32)],
    "fi_gemm_packed": [_P, _P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _P],
    "fi_gemm_packed_swiglu": [_P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P],
    "fi_lm_head_argmax_packed": [_P, _P, _I32, _P, _I32, _I32, _I32, _P, _P],
    "fi_splitk_residual_rms_norm": [_P, _P, _I32, _P, _P, _P, _P, _P, _I32, _I32, _F32],
    "fi_qkv_rope_append": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _I32, _I32,
                           _I32, _I32, _I32, _I32, _I32, _P],
    "fi_weight_pack_columns": [_P, C.POINTER(_P), C.POINTER(_I32), _I32, _I32, _I32, _P],
    "fi_attn_prefill_paged_bf16": [_P, _P, _P, _P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32,
                                   _I32, _F32, _P],
    "fi_weight_packed_bf16_elems": [_I32, _I32, _I32, C.POINTER(_SZ)],
    "fi_weight_pack_bf16": [_P, _P, _I32, _I32, _I32, _I32, _P],
    "fi_weight_pack_bf16_columns": [_P, C.POINTER(_P), C.POINTER(_I32), _I32, _I32, _I32, _P],
    "fi_weight_pack_bf16_pair": [_P, _P, _P, _I32, _I32, _I32, _P],
    "fi_gemm_bf16_splits": [_P, _I32, _I32, _I32, C.POINTER(_I32)],
    "fi_gemm_bf16": [_P, _P, _I32, _I32, _P, _I32, _I32, _I32, _I32, _P],
    "fi_gemm_bf16_swiglu": [_P, _P, _I32, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _I32],
    "fi_lm_head_argmax_bf16": [_P, _P, _I32, _I32, _P, _I32, _I32, _I32, _P, _P],
    "fi_splitk_residual_rms_norm_bf16": [_P, _P, _I32, _P, _P, _P, _P, _P, _I32, _I32, _F32],
    "fi_convert_f32_to_bf16": [_P, _P, C.c_int64, _P],
    "fi_sample_tokens": [_P, _P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P],
    "fi_sample_reserve": [_P, _I32, _I32],
}
_RESTYPES = {"fi_ctx_stream": _P, "fi_last_error": C.c_char_p}

_lib = None
_lib_lock = threading.Lock()


def library_path() -> str:
    return LIB_PATH


def load() -> C.CDLL:
    """Loads the HIP backend; raises if it has not been built (no fallback exists)."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise FerrisError(8, f"HIP backend {LIB_PATH} is not built; run "
                                 "`python -m ferrisinfer_amd.build` (or __graft_entry__.build())")
        # torch bundles its own libamdhip64 (soname libamdhip64.so.7) and binds its libraries to
        # it by path.  Loaded first, it also satisfies this library's libamdhip64.so.7
        # dependency, so the process holds a single HIP runtime; loaded after this library, it
        # would bring a second one, whose initialisation fails.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = C.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _I32)
        lib.fi_last_error.restype = C.c_char_p
        lib.fi_last_error.argtypes = []
        _lib = lib
        return lib


def exported_symbols() -> list:
    lib = load()
    return [n for n in _SIGNATURES if getattr(lib, n, None) is not None]


def check(status: int) -> None:
    if status != 0:
        msg = load().fi_last_error() or b""
        raise FerrisError(int(status), msg.decode(errors="replace"))


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor / int / None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


class Context:
    """fi_context: one device, one stream (kernel/gpu/nvidia.rs:214-262 lifecycle)."""

    def __init__(self, ordinal: int = 0, use_torch_stream: bool = True):
        lib = load()
        h = _P()
        check(lib.fi_ctx_create(ordinal, C.byref(h)))
        self.handle = h
        self.lib = lib
        self.ordinal = ordinal
        if use_torch_stream:
            self.follow_torch_stream()

    def follow_torch_stream(self) -> None:
        import torch

        s = torch.cuda.current_stream(self.ordinal)
        check(self.lib.fi_ctx_set_stream(self.handle, s.cuda_stream))

    def set_stream(self, stream_ptr) -> None:
        check(self.lib.fi_ctx_set_stream(self.handle, stream_ptr))

    @property
    def stream(self) -> int:
        return int(self.lib.fi_ctx_stream(self.handle) or 0)

    def sync(self) -> None:
        check(self.lib.fi_ctx_sync(self.handle))

    def check_faults(self) -> None:
        check(self.lib.fi_ctx_check_faults(self.handle))

    def device_info(self) -> dict:
        name = C.create_string_buffer(256)
        arch = C.create_string_buffer(64)
        hbm = C.c_uint64()
        cus = _I32()
        check(self.lib.fi_device_info(self.handle, name, 256, arch, 64, C.byref(hbm), C.byref(cus)))
        return {"name": name.value.decode(), "arch": arch.value.decode(), "hbm_bytes": hbm.value,
                "compute_units": cus.value}

    def close(self) -> None:
        if getattr(self, "handle", None):
            check(self.lib.fi_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------ ops
    def kv_append(self, key, value, slot_mapping, k_cache, v_cache, kv_dtype, num_blocks,
                  block_size, num_kv_heads, head_dim):
        check(self.lib.fi_kv_append(self.handle, ptr(key), ptr(value), ptr(slot_mapping),
                                    int(slot_mapping.numel()), ptr(k_cache), ptr(v_cache), kv_dtype,
                                    num_blocks, block_size, num_kv_heads, head_dim))

    def kv_copy_blocks(self, k_cache, v_cache, kv_dtype, src_blocks, dst_blocks, token_counts,
                       num_blocks, block_size, num_kv_heads, head_dim):
        check(self.lib.fi_kv_copy_blocks(self.handle, ptr(k_cache), ptr(v_cache), kv_dtype,
                                         ptr(src_blocks), ptr(dst_blocks), ptr(token_counts),
                                         int(src_blocks.numel()), num_blocks, block_size,
                                         num_kv_heads, head_dim))

    def kv_gather(self, k_cache, v_cache, kv_dtype, block_table, length, num_blocks, block_size,
                  num_kv_heads, head_dim, k_out, v_out):
        """read_prefix_f32 of one sequence: its first `length` rows as f32 [length, Hkv, D]."""
        check(self.lib.fi_kv_gather(self.handle, ptr(k_cache), ptr(v_cache), kv_dtype, ptr(block_table),
                                    int(block_table.numel()), int(length), num_blocks, block_size,
                                    num_kv_heads, head_dim, ptr(k_out), ptr(v_out)))

    def attn_decode_paged(self, q, k_cache, v_cache, kv_dtype, block_tables, context_lens,
                          max_context_len, num_kv_heads, block_size, num_blocks, scale, out):
        num_seqs, num_q_heads, head_dim = q.shape
        check(self.lib.fi_attn_decode_paged(self.handle, ptr(q), ptr(k_cache), ptr(v_cache),
                                            kv_dtype, ptr(block_tables), int(block_tables.shape[1]),
                                            ptr(context_lens), num_seqs, int(max_context_len),
                                            num_q_heads, num_kv_heads, head_dim, block_size,
                                            num_blocks, float(scale), ptr(out)))

    def attn_decode_paged_qkv(self, parts, splits, biases, positions, cos_t, sin_t, rotary_dims,
                              max_positions, slot_mapping, k_cache, v_cache, kv_dtype, block_tables,
                              context_lens, max_context_len, num_q_heads, num_kv_heads, head_dim,
                              block_size, num_blocks, scale, out, q_out=None):
        """qkv_rope_append + attn_decode_paged in one launch (one new token per sequence);
        large launches run the two kernels with q_out [num_seqs, Hq, D] between them."""
        bq, bk, bv = biases if biases is not None else (None, None, None)
        check(self.lib.fi_attn_decode_paged_qkv(self.handle, ptr(parts), int(splits), ptr(bq), ptr(bk),
                                                ptr(bv), ptr(positions), ptr(cos_t), ptr(sin_t),
                                                int(rotary_dims), int(max_positions), ptr(slot_mapping),
                                                ptr(k_cache), ptr(v_cache), int(kv_dtype), ptr(block_tables),
                                                int(block_tables.shape[1]), ptr(context_lens),
                                                int(context_lens.numel()), int(max_context_len),
                                                int(num_q_heads), int(num_kv_heads), int(head_dim),
                                                int(block_size), int(num_blocks), float(scale), ptr(q_out),
                                                ptr(out)))

    def attn_decode_paged_noalloc(self, q, k_cache, v_cache, kv_dtype, block_tables, context_lens,
                                  max_context_len, num_kv_heads, block_size, num_blocks, scale, out):
        """attn_decode_paged with the partials in the library's fixed scratch (no allocation)."""
        num_seqs, num_q_heads, head_dim = q.shape
        check(self.lib.fi_attn_decode_paged_noalloc(self.handle, ptr(q), ptr(k_cache), ptr(v_cache),
                                                    kv_dtype, ptr(block_tables),
                                                    int(block_tables.shape[1]), ptr(context_lens),
                                                    num_seqs, int(max_context_len), num_q_heads,
                                                    num_kv_heads, head_dim, block_size, num_blocks,
                                                    float(scale), ptr(out)))

    def embedding(self, table, ids, out):
        check(self.lib.fi_embedding(self.handle, ptr(table), int(table.shape[0]),
                                    int(table.shape[1]), ptr(ids), int(ids.numel()), ptr(out)))

    def rms_norm(self, x, weight, out, eps):
        hidden = int(x.shape[-1])
        check(self.lib.fi_rms_norm(self.handle, ptr(x), ptr(weight), ptr(out),
                                   int(x.numel() // hidden), hidden, float(eps)))

    def add_rms_norm(self, a, residual, sum_out, weight, out, eps):
        hidden = int(a.shape[-1])
        check(self.lib.fi_add_rms_norm(self.handle, ptr(a), ptr(residual), ptr(sum_out),
                                       ptr(weight), ptr(out), int(a.numel() // hidden), hidden,
                                       float(eps)))

    def rope_table(self, max_positions, head_dim, rotary_dims, theta, cos_out, sin_out):
        check(self.lib.fi_rope_table(self.handle, int(max_positions), int(head_dim),
                                     int(rotary_dims), float(theta), ptr(cos_out), ptr(sin_out)))

    def rope(self, q, k, positions, cos_t, sin_t, rotary_dims, max_positions):
        t, hq, d = q.shape
        check(self.lib.fi_rope(self.handle, ptr(q), ptr(k), ptr(positions), ptr(cos_t),
                               ptr(sin_t), int(t), int(hq), int(k.shape[1]), int(d),
                               int(rotary_dims), int(max_positions)))

    def silu_mul(self, up, gate, out):
        check(self.lib.fi_silu_mul(self.handle, ptr(up), ptr(gate), ptr(out), int(up.numel())))

    def add(self, a, b, out):
        check(self.lib.fi_add(self.handle, ptr(a), ptr(b), ptr(out), int(a.numel())))

    def gemm(self, a, b, out, bias=None, b_layout=0):
        """out[M,N] = a[M,K] * b (+ bias); b is [K,N] (layout 0) or [N,K] (layout 1)."""
        m, k = a.shape
        n = b.shape[1] if b_layout == 0 else b.shape[0]
        check(self.lib.fi_gemm(self.handle, ptr(a), ptr(b), ptr(bias), ptr(out), int(m), int(k),
                               int(n), int(b_layout)))

    def lm_head_argmax(self, hidden, weight, token_out, prob_out):
        m, h = hidden.shape
        check(self.lib.fi_lm_head_argmax(self.handle, ptr(hidden), ptr(weight), int(m), int(h),
                                         int(weight.shape[0]), ptr(token_out), ptr(prob_out)))

    def attn_prefill_paged(self, q, k_cache, v_cache, kv_dtype, block_tables, cu_seqlens,
                           context_lens, max_query_len, num_kv_heads, block_size, num_blocks,
                           scale, out):
        t, num_q_heads, head_dim = q.shape
        check(self.lib.fi_attn_prefill_paged(self.handle, ptr(q), ptr(k_cache), ptr(v_cache),
                                             kv_dtype, ptr(block_tables),
                                             int(block_tables.shape[1]), ptr(cu_seqlens),
                                             ptr(context_lens), int(context_lens.numel()),
                                             int(max_query_len), num_q_heads, num_kv_heads,
                                             head_dim, block_size, num_blocks, float(scale),
                                             ptr(out)))

    def attn_prefill_paged_bf16(self, q, k_cache, v_cache, block_tables, cu_seqlens, context_lens,
                                max_query_len, num_kv_heads, block_size, num_blocks, scale, out):
        """fi_attn_prefill_paged over a bf16 pool on bf16 MFMA (Q and P rounded to bf16)."""
        t, num_q_heads, head_dim = q.shape
        check(self.lib.fi_attn_prefill_paged_bf16(self.handle, ptr(q), ptr(k_cache), ptr(v_cache),
                                                  ptr(block_tables), int(block_tables.shape[1]),
                                                  ptr(cu_seqlens), ptr(context_lens),
                                                  int(context_lens.numel()), int(max_query_len),
                                                  num_q_heads, num_kv_heads, head_dim, block_size,
                                                  num_blocks, float(scale), ptr(out)))

    # ---------------------------------------------------------- packed-weight GEMMs
    def weight_packed_floats(self, k, n, pack_width):
        out = _SZ()
        check(self.lib.fi_weight_packed_floats(int(k), int(n), int(pack_width), C.byref(out)))
        return int(out.value)

    def weight_pack(self, src, k, n, pack_width, src_layout=0):
        """Packs a device weight [K, N] (src_layout 0) or [N, K] (1) for fi_gemm_packed."""
        import torch

        dst = torch.empty(self.weight_packed_floats(k, n, pack_width), dtype=torch.float32,
                          device=src.device)
        check(self.lib.fi_weight_pack(self.handle, ptr(src), int(src_layout), int(k), int(n),
                                      int(pack_width), ptr(dst)))
        return dst

    def weight_pack_pair(self, first, second, k, n):
        """SwiGLU pair pack of two [K, N] weights (up = first, gate = second)."""
        import torch

        dst = torch.empty(self.weight_packed_floats(k, 2 * n, 2), dtype=torch.float32,
                          device=first.device)
        check(self.lib.fi_weight_pack_pair(self.handle, ptr(first), ptr(second), int(k), int(n),
                                           ptr(dst)))
        return dst

    def gemm_packed_splits(self, m, k, n, pack_width):
        out = _I32()
        check(self.lib.fi_gemm_packed_splits(self.handle, int(m), int(k), int(n), int(pack_width),
                                             C.byref(out)))
        return int(out.value)

    def gemm_packed(self, a, bp, k, n, pack_width, splits, out):
        """out [splits, M, N] = split-K partial products of a [M, K] and the packed weight."""
        check(self.lib.fi_gemm_packed(self.handle, ptr(a), int(a.stride(0)), ptr(bp), int(k), int(n),
                                      int(pack_width), int(a.shape[0]), int(splits), ptr(out)))

    def gemm_packed_swiglu(self, a, bp_pair, k, n, out, bias_up=None, bias_gate=None):
        check(self.lib.fi_gemm_packed_swiglu(self.handle, ptr(a), int(a.stride(0)), ptr(bp_pair),
                                             int(k), int(n), int(a.shape[0]), ptr(bias_up),
                                             ptr(bias_gate), ptr(out)))

    def lm_head_argmax_packed(self, hidden, bp, vocab, token_out, prob_out):
        """Greedy head over a weight packed from [vocab, hidden] at pack width 2."""
        m, h = hidden.shape
        check(self.lib.fi_lm_head_argmax_packed(self.handle, ptr(hidden), int(hidden.stride(0)),
                                                ptr(bp), int(m), int(h), int(vocab),
                                                ptr(token_out), ptr(prob_out)))

    def splitk_residual_rms_norm(self, parts, splits, bias, residual, sum_out, weight, out, eps):
        """out = rms_norm(sum) * weight with sum = split sum (+ bias) + residual stored to sum_out;
        a 2-byte `out` (bf16 or int16) receives the normalised row as bf16 bits."""
        rows, hidden = residual.shape
        fn = (self.lib.fi_splitk_residual_rms_norm_bf16 if self._act_dtype(out) == DTYPE_BF16
              else self.lib.fi_splitk_residual_rms_norm)
        check(fn(self.handle, ptr(parts), int(splits), ptr(bias), ptr(residual), ptr(sum_out), ptr(weight),
                 ptr(out), int(rows), int(hidden), float(eps)))

    def convert_f32_to_bf16(self, src, out):
        """out (bf16 or int16, same element count) = src (f32) rounded to nearest even."""
        if src.numel() != out.numel():
            raise FerrisError(3, "convert_f32_to_bf16: element counts differ")
        check(self.lib.fi_convert_f32_to_bf16(self.handle, ptr(src), int(src.numel()), ptr(out)))

    def weight_pack_columns(self, srcs, k, pack_width):
        """Packs the column concatenation of up to three device weights [K, n_i]."""
        import torch

        ns = [int(s.shape[1]) for s in srcs]
        dst = torch.empty(self.weight_packed_floats(k, sum(ns), pack_width), dtype=torch.float32,
                          device=srcs[0].device)
        arr = (_P * len(srcs))(*[ptr(s) for s in srcs])
        nar = (_I32 * len(srcs))(*ns)
        check(self.lib.fi_weight_pack_columns(self.handle, arr, nar, len(srcs), int(k),
                                              int(pack_width), ptr(dst)))
        return dst

    # ---- bf16-stored weights ----

    @staticmethod
    def _src_dtype(t):
        import torch

        if t.dtype == torch.float32:
            return DTYPE_F32
        if t.dtype in (torch.bfloat16, torch.int16):
            return DTYPE_BF16
        raise FerrisError(5, f"bf16 weight pack: unsupported source dtype {t.dtype}")

    def weight_packed_bf16_elems(self, k, n, pair=False):
        out = _SZ()
        check(self.lib.fi_weight_packed_bf16_elems(int(k), int(n), int(bool(pair)), C.byref(out)))
        return int(out.value)

    def weight_pack_bf16(self, src, k, n, src_layout=0):
        """Packs a device weight (f32, bf16 or raw bf16 bits as int16), [K, N] (src_layout 0) or
        [N, K] (1), for fi_gemm_bf16; returns the packed bf16 bits as int16."""
        import torch

        dst = torch.empty(self.weight_packed_bf16_elems(k, n), dtype=torch.int16, device=src.device)
        check(self.lib.fi_weight_pack_bf16(self.handle, ptr(src), self._src_dtype(src),
                                           int(src_layout), int(k), int(n), ptr(dst)))
        return dst

    def weight_pack_bf16_columns(self, srcs, k):
        import torch

        ns = [int(t.shape[1]) for t in srcs]
        dst = torch.empty(self.weight_packed_bf16_elems(k, sum(ns)), dtype=torch.int16,
                          device=srcs[0].device)
        arr = (_P * len(srcs))(*[ptr(t) for t in srcs])
        nar = (_I32 * len(srcs))(*ns)
        check(self.lib.fi_weight_pack_bf16_columns(self.handle, arr, nar, len(srcs),
                                                   self._src_dtype(srcs[0]), int(k), ptr(dst)))
        return dst

    def weight_pack_bf16_pair(self, up, gate, k, n):
        import torch

        dst = torch.empty(self.weight_packed_bf16_elems(k, n, pair=True), dtype=torch.int16,
                          device=up.device)
        check(self.lib.fi_weight_pack_bf16_pair(self.handle, ptr(up), ptr(gate), self._src_dtype(up),
                                                int(k), int(n), ptr(dst)))
        return dst

    def gemm_bf16_splits(self, m, k, n):
        out = _I32()
        check(self.lib.fi_gemm_bf16_splits(self.handle, int(m), int(k), int(n), C.byref(out)))
        return int(out.value)

    @staticmethod
    def _act_dtype(t):
        """Activation dtype of a tensor: f32, or bf16 bits in any 2-byte dtype."""
        import torch

        if t.dtype == torch.float32:
            return DTYPE_F32
        if t.element_size() == 2 and t.dtype != torch.float16:
            return DTYPE_BF16
        raise FerrisError(5, f"activation dtype {t.dtype} is neither f32 nor bf16")

    def gemm_bf16(self, a, bp, k, n, splits, out):
        """out [splits, M, N] = split-K partial products of a [M, K] (f32, or bf16 bits) and the
        packed bf16 weight."""
        check(self.lib.fi_gemm_bf16(self.handle, ptr(a), self._act_dtype(a), int(a.stride(0)), ptr(bp),
                                    int(k), int(n), int(a.shape[0]), int(splits), ptr(out)))

    def gemm_bf16_swiglu(self, a, bp_pair, k, n, out, bias_up=None, bias_gate=None):
        """out [M, N] (f32, or bf16 bits when out is a 2-byte tensor) = SwiGLU of the pair."""
        check(self.lib.fi_gemm_bf16_swiglu(self.handle, ptr(a), self._act_dtype(a), int(a.stride(0)),
                                           ptr(bp_pair), int(k), int(n), int(a.shape[0]), ptr(bias_up),
                                           ptr(bias_gate), ptr(out), self._act_dtype(out)))

    def lm_head_argmax_bf16(self, hidden, bp, vocab, token_out, prob_out):
        m, h = hidden.shape
        check(self.lib.fi_lm_head_argmax_bf16(self.handle, ptr(hidden), self._act_dtype(hidden),
                                              int(hidden.stride(0)), ptr(bp), int(m), int(h), int(vocab),
                                              ptr(token_out), ptr(prob_out)))

    def sample_tokens(self, logits, temperature, top_k, top_p, rng_state, token_out, prob_out):
        """One token per row of logits [rows, vocab] (f32, row stride logits.stride(0)) under the
        per-row configuration (temperature f32, top_k int32, top_p f32) and xorshift64* states
        (uint64 stored as int64, advanced in place for sampled rows)."""
        rows, vocab = logits.shape
        check(self.lib.fi_sample_tokens(self.handle, ptr(logits), int(logits.stride(0)), int(rows),
                                        int(vocab), ptr(temperature), ptr(top_k), ptr(top_p),
                                        ptr(rng_state), ptr(token_out), ptr(prob_out)))

    def sample_reserve(self, rows, vocab):
        """Room for sample_tokens to serve top_k above 1024 (up to the vocabulary) in calls of
        up to `rows` rows of `vocab` logits."""
        check(self.lib.fi_sample_reserve(self.handle, int(rows), int(vocab)))

    def convert_to_f32(self, src, src_dtype, rows, cols, transpose, dst):
        """dst (f32) = the widening of src, a [rows, cols] row-major tensor of src_dtype
        (DTYPE_F32 / DTYPE_BF16 / DTYPE_F16 raw bits in any torch dtype of that width), or its
        [cols, rows] transpose when transpose is true."""
        check(self.lib.fi_convert_to_f32(self.handle, ptr(src), int(src_dtype), int(rows), int(cols),
                                         1 if transpose else 0, ptr(dst)))

    def qkv_rope_append(self, parts, splits, biases, positions, cos_t, sin_t, rotary_dims,
                        max_positions, slot_mapping, k_cache, v_cache, kv_dtype, num_blocks,
                        block_size, num_q_heads, num_kv_heads, head_dim, q_out):
        bq, bk, bv = biases if biases is not None else (None, None, None)
        check(self.lib.fi_qkv_rope_append(self.handle, ptr(parts), int(splits), ptr(bq), ptr(bk),
                                          ptr(bv),
                                          ptr(positions), ptr(cos_t), ptr(sin_t), int(rotary_dims),
                                          int(max_positions), ptr(slot_mapping), ptr(k_cache),
                                          ptr(v_cache), int(kv_dtype), int(num_blocks),
                                          int(block_size), int(positions.numel()),
                                          int(num_q_heads), int(num_kv_heads), int(head_dim),
                                          ptr(q_out)))
