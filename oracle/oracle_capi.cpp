// C entry points of the oracle library (liboracle.so) — TEST INFRASTRUCTURE ONLY.
// Loaded by tests/ (ctypes), __graft_entry__.smoke() and bench.py's cpu_baseline leg.
// Each wrapper returns 0 or ErrorKind+1 and keeps the message for orc_last_error().
#include <cstring>
#include <string>

#include "oracle.h"

using orc::ErrorKind;
using orc::OracleError;

static thread_local std::string g_last_error;

template <typename F>
static int32_t guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const OracleError& e) {
    g_last_error = e.message;
    return static_cast<int32_t>(e.kind) + 1;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return static_cast<int32_t>(ErrorKind::Runtime) + 1;
  }
}

extern "C" {

const char* orc_last_error(void) { return g_last_error.c_str(); }

void orc_set_threads(int64_t threads) { orc::set_available_parallelism(static_cast<size_t>(threads)); }
int64_t orc_threads(void) { return static_cast<int64_t>(orc::available_parallelism()); }

int32_t orc_embedding_gather_f32(const float* embedding, int64_t vocab, int64_t hidden,
                                 const uint32_t* ids, int64_t rows, float* out) {
  return guard([&] { orc::embedding_gather_f32(embedding, vocab, hidden, ids, rows, out); });
}

int32_t orc_rms_norm_f32(const float* x, const float* w, int64_t rows, int64_t hidden, float eps,
                         float* out) {
  return guard([&] { orc::rms_norm_f32(x, w, rows, hidden, eps, out); });
}

int32_t orc_matmul_f32(const float* lhs, const float* rhs, int64_t m, int64_t k, int64_t n,
                       float* out) {
  return guard([&] { orc::matmul_f32(lhs, rhs, m, k, n, out); });
}

int32_t orc_linear_f32_with_bias(const float* x, const float* w, const float* bias, int64_t m,
                                 int64_t k, int64_t n, float* out) {
  return guard([&] { orc::linear_f32_with_bias(x, w, bias, m, k, n, out); });
}

int32_t orc_matmul_rhs_transposed_f32(const float* lhs, const float* rhs, int64_t m, int64_t k,
                                      int64_t n, float* out) {
  return guard([&] { orc::matmul_rhs_transposed_f32(lhs, rhs, m, k, n, out); });
}

int32_t orc_matmul_rhs_transposed_argmax_f32(const float* lhs, const float* rhs, int64_t k,
                                             int64_t n, uint32_t* best, float* prob) {
  return guard([&] { orc::matmul_rhs_transposed_argmax_f32(lhs, rhs, k, n, best, prob); });
}

int32_t orc_argmax_last_token(const float* logits, int64_t seq_len, int64_t vocab, uint32_t* id,
                              float* prob) {
  return guard([&] { orc::argmax_last_token(logits, seq_len, vocab, id, prob); });
}

uint64_t orc_sampler_state_new(uint64_t seed) { return orc::sampler_state_new(seed); }

float orc_sampler_next_f32(uint64_t* state) { return orc::sampler_next_f32(state); }

int32_t orc_sample_last_token(const float* logits, int64_t seq_len, int64_t vocab, float temperature, int64_t top_k,
                              float top_p, uint64_t* state, uint32_t* id, float* prob) {
  return guard([&] {
    orc::sample_last_token(logits, seq_len, vocab, temperature, static_cast<size_t>(top_k < 0 ? 0 : top_k), top_p,
                           state, id, prob);
  });
}

int32_t orc_rope_f32(float* q, float* k, int64_t seq_len, int64_t hq, int64_t hkv, int64_t d,
                     int64_t position_offset, int64_t rotary_dims, float theta) {
  return guard([&] { orc::rope_f32(q, k, seq_len, hq, hkv, d, position_offset, rotary_dims, theta); });
}

int32_t orc_prefixed_causal_attention_f32(const float* q, const float* k, const float* v,
                                          int64_t query_len, int64_t cache_len, int64_t hq,
                                          int64_t hkv, int64_t d, float* out) {
  return guard([&] { orc::prefixed_causal_attention_f32(q, k, v, query_len, cache_len, hq, hkv, d, out); });
}

int32_t orc_cached_prefixed_causal_attention_f32(const float* q, const float* ck, const float* cv,
                                                 int64_t cache_len, const float* ks,
                                                 const float* vs, int64_t query_len, int64_t hq,
                                                 int64_t hkv, int64_t d, float* out) {
  return guard([&] {
    orc::cached_prefixed_causal_attention_f32(q, ck, cv, cache_len, ks, vs, query_len, hq, hkv, d, out);
  });
}

int32_t orc_decode_causal_attention_f32(const float* q, const float* ck, const float* cv,
                                        int64_t cache_len, const float* kslot,
                                        const float* vslot, int64_t hq, int64_t hkv, int64_t d,
                                        float* out) {
  return guard([&] { orc::decode_causal_attention_f32(q, ck, cv, cache_len, kslot, vslot, hq, hkv, d, out); });
}

int32_t orc_silu_f32_in_place(float* x, int64_t n) {
  return guard([&] { orc::silu_f32_in_place(x, n); });
}
int32_t orc_mul_f32_in_place(float* out, const float* rhs, int64_t n) {
  return guard([&] { orc::mul_f32_in_place(out, rhs, n); });
}
int32_t orc_add_f32_in_place(float* out, const float* rhs, int64_t n) {
  return guard([&] { orc::add_f32_in_place(out, rhs, n); });
}

void orc_f32_to_bf16_rne(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc::f32_to_bf16_rne(src[i]);
}
void orc_bf16_to_f32(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc::bf16_to_f32(src[i]);
}

}  // extern "C"
