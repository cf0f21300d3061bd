// Oracle restatement of crates/ferrisinfer-kernel/src/cpu/{attention,matmul,reduction,
// elementwise}.rs — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Thread fan-out mirrors the reference's std::thread::scope splits and thresholds so
// the CPU baseline is timed with the same parallelism; results never depend on the
// thread count except the fused-argmax probability (matmul.rs:232-270), exactly as in
// the reference.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <thread>

#include "oracle.h"

namespace orc {

static size_t g_parallelism = 0;

void fail(ErrorKind kind, const std::string& message) { throw OracleError{kind, message}; }

size_t available_parallelism() {
  if (g_parallelism != 0) return g_parallelism;
  unsigned hc = std::thread::hardware_concurrency();
  return hc == 0 ? 1 : hc;
}

void set_available_parallelism(size_t threads) { g_parallelism = threads; }

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

static size_t sat_mul(size_t a, size_t b) {
  if (a != 0 && b > std::numeric_limits<size_t>::max() / a) return std::numeric_limits<size_t>::max();
  return a * b;
}

// Runs body(chunk_start, chunk_end) over [0, total) split into chunks of `per_chunk`,
// one std::thread per chunk (the shape of the reference's chunks_mut + scope.spawn).
static void scoped_chunks(size_t total, size_t per_chunk,
                          const std::function<void(size_t, size_t)>& body) {
  std::vector<std::thread> threads;
  for (size_t start = 0; start < total; start += per_chunk) {
    size_t end = std::min(total, start + per_chunk);
    threads.emplace_back([&body, start, end]() { body(start, end); });
  }
  for (auto& t : threads) t.join();
}

// ---------------------------------------------------------------------------
// attention.rs:3-99 embedding_gather_f32
// ---------------------------------------------------------------------------
static size_t preferred_embedding_thread_count(size_t rows, size_t hidden) {
  // attention.rs:1203-1213
  const size_t kMin = 131072;
  if (rows < 2 || sat_mul(rows, hidden) < kMin) return 1;
  return std::min(available_parallelism(), rows);
}

void embedding_gather_f32(const float* embedding, size_t vocab, size_t hidden,
                          const uint32_t* token_ids, size_t rows, float* out) {
  for (size_t r = 0; r < rows; ++r) {
    if (token_ids[r] >= vocab) {
      fail(ErrorKind::InvalidShape, "token id " + std::to_string(token_ids[r]) +
                                        " is out of vocabulary range " + std::to_string(vocab));
    }
  }
  size_t threads = preferred_embedding_thread_count(rows, hidden);
  auto body = [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) {
      std::memcpy(out + r * hidden, embedding + static_cast<size_t>(token_ids[r]) * hidden,
                  hidden * sizeof(float));
    }
  };
  if (threads == 1) {
    body(0, rows);
  } else {
    scoped_chunks(rows, div_ceil(rows, threads), body);
  }
}

// ---------------------------------------------------------------------------
// reduction.rs:3-73 rms_norm_f32
// ---------------------------------------------------------------------------
static size_t preferred_rowwise_thread_count(size_t rows, size_t hidden) {
  // reduction.rs:143-154
  const size_t kMin = 131072;
  if (rows < 2 || sat_mul(rows, hidden) < kMin) return 1;
  return std::min(available_parallelism(), rows);
}

void rms_norm_f32(const float* input, const float* weight, size_t rows, size_t hidden,
                  float eps, float* out) {
  if (hidden == 0) fail(ErrorKind::InvalidShape, "rms_norm_f32 requires at least one dimension");
  auto body = [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) {
      const float* row = input + r * hidden;
      float sum = -0.0f;  // f32 Sum folds from -0.0
      for (size_t c = 0; c < hidden; ++c) {
        float sq = row[c] * row[c];
        sum = sum + sq;
      }
      float mean_square = sum / static_cast<float>(hidden);
      float inv_rms = 1.0f / std::sqrt(mean_square + eps);
      for (size_t c = 0; c < hidden; ++c) {
        float t = row[c] * inv_rms;
        out[r * hidden + c] = t * weight[c];
      }
    }
  };
  size_t threads = preferred_rowwise_thread_count(rows, hidden);
  if (threads == 1) {
    body(0, rows);
  } else {
    scoped_chunks(rows, div_ceil(rows, threads), body);
  }
}

// ---------------------------------------------------------------------------
// matmul.rs:46-118, 424-499 matmul_f32 ([M,K] x [K,N]); zero lhs terms skipped
// ---------------------------------------------------------------------------
static size_t preferred_thread_count(size_t rows, size_t cols, size_t inner) {
  // matmul.rs:620-634
  const size_t kMin = 131072;
  if (rows < 2) return 1;
  if (sat_mul(sat_mul(rows, cols), inner) < kMin) return 1;
  return std::min(available_parallelism(), rows);
}

static size_t preferred_single_row_thread_count(size_t cols, size_t inner) {
  // matmul.rs:636-651
  const size_t kMinWork = 8388608;
  const size_t kMinCols = 8192;
  if (cols < kMinCols) return 1;
  if (sat_mul(cols, inner) < kMinWork) return 1;
  return std::min(available_parallelism(), cols);
}

static void compute_single_row_chunk(const float* lhs, size_t k, const float* rhs,
                                     float* out_chunk, size_t total_cols, size_t col_start,
                                     size_t col_end) {
  // matmul.rs:479-499
  size_t width = col_end - col_start;
  for (size_t c = 0; c < width; ++c) out_chunk[c] = 0.0f;
  for (size_t inner = 0; inner < k; ++inner) {
    float lv = lhs[inner];
    if (lv == 0.0f) continue;
    const float* rhs_row = rhs + inner * total_cols + col_start;
    for (size_t c = 0; c < width; ++c) {
      float p = lv * rhs_row[c];
      out_chunk[c] = out_chunk[c] + p;
    }
  }
}

void matmul_f32(const float* lhs, const float* rhs, size_t m, size_t k, size_t n, float* out) {
  if (m == 1) {
    // compute_single_row_matmul, matmul.rs:450-477
    size_t threads = preferred_single_row_thread_count(n, k);
    if (threads == 1) {
      compute_single_row_chunk(lhs, k, rhs, out, n, 0, n);
    } else {
      scoped_chunks(n, div_ceil(n, threads), [&](size_t c0, size_t c1) {
        compute_single_row_chunk(lhs, k, rhs, out + c0, n, c0, c1);
      });
    }
    return;
  }
  std::fill(out, out + m * n, 0.0f);
  auto body = [&](size_t r0, size_t r1) {
    // compute_row_chunk, matmul.rs:424-448
    for (size_t row = r0; row < r1; ++row) {
      const float* lhs_row = lhs + row * k;
      float* out_row = out + row * n;
      for (size_t inner = 0; inner < k; ++inner) {
        float lv = lhs_row[inner];
        if (lv == 0.0f) continue;
        const float* rhs_row = rhs + inner * n;
        for (size_t c = 0; c < n; ++c) {
          float p = lv * rhs_row[c];
          out_row[c] = out_row[c] + p;
        }
      }
    }
  };
  size_t threads = preferred_thread_count(m, n, k);
  if (threads == 1) {
    body(0, m);
  } else {
    scoped_chunks(m, div_ceil(m, threads), body);
  }
}

// runtime/reference.rs:1135-1191 linear_f32_with_bias: matmul, then += bias per row
void linear_f32_with_bias(const float* input, const float* weight, const float* bias,
                          size_t m, size_t k, size_t n, float* out) {
  matmul_f32(input, weight, m, k, n, out);
  if (bias == nullptr) return;
  for (size_t r = 0; r < m; ++r) {
    for (size_t c = 0; c < n; ++c) out[r * n + c] = out[r * n + c] + bias[c];
  }
}

// ---------------------------------------------------------------------------
// matmul.rs:120-188, 501-523 matmul_rhs_transposed_f32 ([M,K] x [N,K]^T)
// ---------------------------------------------------------------------------
void matmul_rhs_transposed_f32(const float* lhs, const float* rhs, size_t m, size_t k,
                               size_t n, float* out) {
  auto body = [&](size_t r0, size_t r1) {
    for (size_t row = r0; row < r1; ++row) {
      const float* in = lhs + row * k;
      for (size_t col = 0; col < n; ++col) {
        const float* w = rhs + col * k;
        float sum = 0.0f;
        for (size_t i = 0; i < k; ++i) {
          float p = in[i] * w[i];
          sum = sum + p;
        }
        out[row * n + col] = sum;
      }
    }
  };
  size_t threads = preferred_thread_count(m, n, k);  // preferred_transposed_thread_count
  if (threads == 1) {
    body(0, m);
  } else {
    scoped_chunks(m, div_ceil(m, threads), body);
  }
}

// ---------------------------------------------------------------------------
// matmul.rs:190-274, 532-589 fused lm_head GEMV + first-max argmax + softmax denominator
// ---------------------------------------------------------------------------
struct ProjectionArgmax {
  size_t best_index;
  float max_logit;
  float scaled_sum;
};

static ProjectionArgmax compute_projection_argmax_chunk(const float* input, const float* weight,
                                                        size_t k, size_t col_start,
                                                        size_t col_end) {
  ProjectionArgmax a{col_start, -std::numeric_limits<float>::infinity(), 0.0f};
  for (size_t col = col_start; col < col_end; ++col) {
    const float* w = weight + col * k;
    float sum = 0.0f;
    for (size_t i = 0; i < k; ++i) {
      float p = input[i] * w[i];
      sum = sum + p;
    }
    if (sum > a.max_logit) {
      if (std::isfinite(a.max_logit)) {
        float e = std::exp(a.max_logit - sum);
        float t = a.scaled_sum * e;
        a.scaled_sum = t + 1.0f;
      } else {
        a.scaled_sum = 1.0f;
      }
      a.max_logit = sum;
      a.best_index = col;
    } else {
      float e = std::exp(sum - a.max_logit);
      a.scaled_sum = a.scaled_sum + e;
    }
  }
  return a;
}

static ProjectionArgmax merge_projection_argmax_chunks(ProjectionArgmax left,
                                                       ProjectionArgmax right) {
  if (left.max_logit >= right.max_logit) {
    float e = std::exp(right.max_logit - left.max_logit);
    float t = right.scaled_sum * e;
    return {left.best_index, left.max_logit, left.scaled_sum + t};
  }
  float e = std::exp(left.max_logit - right.max_logit);
  float t = left.scaled_sum * e;
  return {right.best_index, right.max_logit, right.scaled_sum + t};
}

static size_t preferred_projection_thread_count(size_t out_width, size_t input_width) {
  // matmul.rs:670-686
  const size_t kMin = 131072;
  if (out_width < 2) return 1;
  if (sat_mul(out_width, input_width) < kMin) return 1;
  return std::min(available_parallelism(), out_width);
}

void matmul_rhs_transposed_argmax_f32(const float* lhs, const float* rhs, size_t k, size_t n,
                                      uint32_t* best_index, float* probability) {
  if (n == 0) {
    fail(ErrorKind::InvalidShape,
         "matmul_rhs_transposed_argmax_f32 requires a non-empty output width");
  }
  size_t threads = preferred_projection_thread_count(n, k);
  ProjectionArgmax agg;
  if (threads == 1) {
    agg = compute_projection_argmax_chunk(lhs, rhs, k, 0, n);
  } else {
    size_t cols_per_chunk = div_ceil(n, threads);
    std::vector<ProjectionArgmax> chunks;
    std::vector<std::thread> pool;
    for (size_t ci = 0; ci < threads; ++ci) {
      size_t c0 = ci * cols_per_chunk;
      if (c0 >= n) break;
      chunks.push_back({});
    }
    for (size_t ci = 0; ci < chunks.size(); ++ci) {
      size_t c0 = ci * cols_per_chunk;
      size_t c1 = std::min(n, c0 + cols_per_chunk);
      pool.emplace_back([&, ci, c0, c1]() {
        chunks[ci] = compute_projection_argmax_chunk(lhs, rhs, k, c0, c1);
      });
    }
    for (auto& t : pool) t.join();
    agg = chunks[0];
    for (size_t ci = 1; ci < chunks.size(); ++ci) agg = merge_projection_argmax_chunks(agg, chunks[ci]);
  }
  *best_index = static_cast<uint32_t>(agg.best_index);
  *probability = 1.0f / agg.scaled_sum;
}

// runtime/sampler.rs:77-119 argmax_last_token: last max index on ties (max_by/total_cmp)
static int32_t total_cmp_key(float v) {
  int32_t bits;
  std::memcpy(&bits, &v, 4);
  return bits ^ static_cast<int32_t>(static_cast<uint32_t>(bits >> 31) >> 1);
}

void argmax_last_token(const float* logits, size_t seq_len, size_t vocab, uint32_t* token_id,
                       float* probability) {
  if (seq_len == 0 || vocab == 0) fail(ErrorKind::InvalidShape, "argmax_last_token requires non-empty logits");
  const float* row = logits + (seq_len - 1) * vocab;
  size_t best = 0;
  for (size_t i = 1; i < vocab; ++i) {
    // Iterator::max_by keeps the later element when it compares >= the current max.
    if (total_cmp_key(row[i]) >= total_cmp_key(row[best])) best = i;
  }
  float max_logit = row[best];
  float denominator = 0.0f;
  for (size_t i = 0; i < vocab; ++i) {
    float e = std::exp(row[i] - max_logit);
    denominator = denominator + e;
  }
  *token_id = static_cast<uint32_t>(best);
  *probability = 1.0f / denominator;
}

// runtime/sampler.rs:55-75 SamplerState: seed 0 becomes the golden-ratio constant; next_f32
// is one xorshift64 step, then the xorshift64* multiplier, keeping the top 24 bits / 2^24.
uint64_t sampler_state_new(uint64_t seed) { return seed == 0 ? 0x9e3779b97f4a7c15ULL : seed; }

float sampler_next_f32(uint64_t* state) {
  uint64_t x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  const uint64_t value = x * 0x2545F4914F6CDD1DULL;
  const uint32_t upper = static_cast<uint32_t>(value >> 40);
  return static_cast<float>(upper) / static_cast<float>(1u << 24);
}

// runtime/sampler.rs:40-42 SamplerConfig::is_greedy
bool sampler_is_greedy(float temperature, size_t top_k, float top_p) {
  return temperature <= 0.0f || top_k == 1 || top_p <= 0.0f;
}

// runtime/sampler.rs:121-241 sample_last_token.  The top-k candidates are kept by streaming
// replacement (the first minimum in list order, by total_cmp, is replaced by a strictly larger
// logit); the list is stably sorted by total_cmp descending; weights exp(l/T - l0/T), the top-p
// prefix and the threshold walk are sequential f32 sums in list order.
void sample_last_token(const float* logits, size_t seq_len, size_t vocab, float temperature, size_t top_k,
                       float top_p, uint64_t* state, uint32_t* token_id, float* probability) {
  if (sampler_is_greedy(temperature, top_k, top_p)) {
    argmax_last_token(logits, seq_len, vocab, token_id, probability);
    return;
  }
  if (seq_len == 0 || vocab == 0) fail(ErrorKind::InvalidShape, "sample_last_token requires non-empty logits");
  const float* row = logits + (seq_len - 1) * vocab;
  const size_t k = std::min(std::max(top_k, static_cast<size_t>(1)), vocab);
  std::vector<std::pair<size_t, float>> cand;
  cand.reserve(k);
  if (k == vocab) {
    for (size_t i = 0; i < vocab; ++i) cand.emplace_back(i, row[i]);
  } else {
    for (size_t i = 0; i < vocab; ++i) {
      if (cand.size() < k) {
        cand.emplace_back(i, row[i]);
        continue;
      }
      size_t min_pos = 0;  // Iterator::min_by keeps the first of equal minima
      for (size_t j = 1; j < cand.size(); ++j) {
        if (total_cmp_key(cand[j].second) < total_cmp_key(cand[min_pos].second)) min_pos = j;
      }
      if (row[i] > cand[min_pos].second) cand[min_pos] = {i, row[i]};
    }
  }
  std::stable_sort(cand.begin(), cand.end(), [](const std::pair<size_t, float>& a, const std::pair<size_t, float>& b) {
    return total_cmp_key(a.second) > total_cmp_key(b.second);
  });
  const float temp = std::fmax(temperature, FLT_EPSILON);  // f32::max ignores a NaN operand
  const float scaled_max = cand[0].second / temp;
  std::vector<float> weight(cand.size());
  float total_weight = 0.0f;
  for (size_t i = 0; i < cand.size(); ++i) {
    weight[i] = std::exp((cand[i].second / temp) - scaled_max);
    total_weight = total_weight + weight[i];
  }
  if (!std::isfinite(total_weight) || total_weight <= 0.0f) {
    fail(ErrorKind::Runtime, "failed to build a finite sampling distribution");
  }
  float p = top_p;  // f32::clamp(0, 1); a NaN stays NaN
  if (p < 0.0f) p = 0.0f;
  if (p > 1.0f) p = 1.0f;
  const float cutoff = p >= 1.0f ? total_weight : total_weight * p;
  float retained_weight = 0.0f;
  size_t retained = 0;
  for (size_t i = 0; i < cand.size(); ++i) {
    retained_weight = retained_weight + weight[i];
    ++retained;
    if (retained_weight >= cutoff) break;
  }
  retained = std::max(retained, static_cast<size_t>(1));
  float retained_total = 0.0f;
  for (size_t i = 0; i < retained; ++i) retained_total = retained_total + weight[i];
  float threshold = sampler_next_f32(state) * retained_total;
  size_t selected = 0;
  for (size_t i = 0; i < retained; ++i) {
    threshold = threshold - weight[i];
    if (threshold <= 0.0f) {
      selected = i;
      break;
    }
  }
  *token_id = static_cast<uint32_t>(cand[selected].first);
  *probability = weight[selected] / retained_total;
}

// ---------------------------------------------------------------------------
// attention.rs:165-220, 1242-1292 rope_f32 (NeoX half-split, iterated inverse frequency)
// ---------------------------------------------------------------------------
void rope_f32(float* query, float* key, size_t seq_len, size_t query_heads, size_t key_heads,
              size_t head_dim, size_t position_offset, size_t rotary_dims, float theta) {
  if (rotary_dims == 0) return;
  if (rotary_dims > head_dim || rotary_dims % 2 != 0) {
    fail(ErrorKind::InvalidShape, "rotary_dims must be an even value no larger than head_dim");
  }
  if (!(theta > 0.0f)) fail(ErrorKind::InvalidConfig, "rope theta must be positive");
  size_t pairs = rotary_dims / 2;
  float step_exponent = -2.0f / static_cast<float>(head_dim);
  float step = std::pow(theta, step_exponent);
  for (size_t p = 0; p < seq_len; ++p) {
    float absolute_position = static_cast<float>(position_offset + p);
    float inv = 1.0f;
    for (size_t j = 0; j < pairs; ++j) {
      float angle = absolute_position * inv;
      float s = std::sin(angle);
      float c = std::cos(angle);
      size_t lo = j, hi = j + pairs;
      for (size_t h = 0; h < query_heads; ++h) {
        float* base = query + (p * query_heads + h) * head_dim;
        float l = base[lo], r = base[hi];
        float a = l * c, b = r * s, e = r * c, f = l * s;
        base[lo] = a - b;
        base[hi] = e + f;
      }
      for (size_t h = 0; h < key_heads; ++h) {
        float* base = key + (p * key_heads + h) * head_dim;
        float l = base[lo], r = base[hi];
        float a = l * c, b = r * s, e = r * c, f = l * s;
        base[lo] = a - b;
        base[hi] = e + f;
      }
      inv = inv * step;
    }
  }
}

// ---------------------------------------------------------------------------
// attention.rs:1090-1149 dot product + online softmax accumulator
// ---------------------------------------------------------------------------
static inline float dot(const float* a, const float* b, size_t n) {
  float sum = -0.0f;  // Iterator::sum over f32 folds from -0.0
  for (size_t i = 0; i < n; ++i) {
    float p = a[i] * b[i];
    sum = sum + p;
  }
  return sum;
}

static inline float update_online_softmax(float* out_row, size_t d, float* max_score,
                                          float* score_sum, float score) {
  if (score > *max_score) {
    float rescale = std::isfinite(*max_score) ? std::exp(*max_score - score) : 0.0f;
    for (size_t i = 0; i < d; ++i) out_row[i] = out_row[i] * rescale;
    *score_sum = *score_sum * rescale;
    *max_score = score;
    *score_sum = *score_sum + 1.0f;
    return 1.0f;
  }
  float weight = std::exp(score - *max_score);
  *score_sum = *score_sum + weight;
  return weight;
}

static inline void accumulate(float* out_row, const float* v, float w, size_t d) {
  for (size_t i = 0; i < d; ++i) {
    float p = w * v[i];
    out_row[i] = out_row[i] + p;
  }
}

static inline void finish_row(float* out_row, float score_sum, size_t d) {
  float inv = 1.0f / score_sum;
  for (size_t i = 0; i < d; ++i) out_row[i] = out_row[i] * inv;
}

static size_t preferred_attention_thread_count(size_t query_len, size_t heads, size_t head_dim,
                                               size_t attended_len) {
  // attention.rs:1185-1201
  const size_t kMin = 131072;
  if (query_len < 2) return 1;
  size_t work = sat_mul(sat_mul(sat_mul(query_len, heads), head_dim), attended_len);
  if (work < kMin) return 1;
  return std::min(available_parallelism(), query_len);
}

static float attention_scale(size_t head_dim) {
  return 1.0f / std::sqrt(static_cast<float>(head_dim));
}

static void check_gqa(size_t hq, size_t hkv) {
  if (hkv == 0 || hq % hkv != 0) {
    fail(ErrorKind::InvalidShape, "number of query heads must be divisible by number of KV heads");
  }
}

// attention.rs:222-330, 729-781 compute_attention_chunk over keys [0, cache_len + t]
void prefixed_causal_attention_f32(const float* query, const float* key, const float* value,
                                   size_t query_len, size_t cache_len, size_t hq, size_t hkv,
                                   size_t d, float* out) {
  check_gqa(hq, hkv);
  size_t group = hq / hkv;
  float scale = attention_scale(d);
  auto body = [&](size_t t0, size_t t1) {
    for (size_t t = t0; t < t1; ++t) {
      size_t last = cache_len + t;
      for (size_t h = 0; h < hq; ++h) {
        size_t kvh = h / group;
        const float* q = query + (t * hq + h) * d;
        float* o = out + (t * hq + h) * d;
        std::fill(o, o + d, 0.0f);
        float m = -std::numeric_limits<float>::infinity();
        float s = 0.0f;
        for (size_t p = 0; p <= last; ++p) {
          float score = dot(q, key + (p * hkv + kvh) * d, d) * scale;
          float w = update_online_softmax(o, d, &m, &s, score);
          accumulate(o, value + (p * hkv + kvh) * d, w, d);
        }
        finish_row(o, s, d);
      }
    }
  };
  size_t threads = preferred_attention_thread_count(query_len, hq, d, cache_len + query_len);
  if (threads == 1) {
    body(0, query_len);
  } else {
    scoped_chunks(query_len, div_ceil(query_len, threads), body);
  }
}

// attention.rs:332-518, 783-870 keys < cache_len from the cache, the rest from the suffix
void cached_prefixed_causal_attention_f32(const float* query, const float* cached_key,
                                          const float* cached_value, size_t cache_len,
                                          const float* key_suffix, const float* value_suffix,
                                          size_t query_len, size_t hq, size_t hkv, size_t d,
                                          float* out) {
  check_gqa(hq, hkv);
  size_t group = hq / hkv;
  float scale = attention_scale(d);
  auto body = [&](size_t t0, size_t t1) {
    for (size_t t = t0; t < t1; ++t) {
      size_t last = cache_len + t;
      for (size_t h = 0; h < hq; ++h) {
        size_t kvh = h / group;
        const float* q = query + (t * hq + h) * d;
        float* o = out + (t * hq + h) * d;
        std::fill(o, o + d, 0.0f);
        float m = -std::numeric_limits<float>::infinity();
        float s = 0.0f;
        for (size_t p = 0; p <= last; ++p) {
          const float* kr;
          const float* vr;
          if (p < cache_len) {
            kr = cached_key + (p * hkv + kvh) * d;
            vr = cached_value + (p * hkv + kvh) * d;
          } else {
            kr = key_suffix + ((p - cache_len) * hkv + kvh) * d;
            vr = value_suffix + ((p - cache_len) * hkv + kvh) * d;
          }
          float score = dot(q, kr, d) * scale;
          float w = update_online_softmax(o, d, &m, &s, score);
          accumulate(o, vr, w, d);
        }
        finish_row(o, s, d);
      }
    }
  };
  size_t threads = preferred_attention_thread_count(query_len, hq, d, cache_len + query_len);
  if (threads == 1) {
    body(0, query_len);
  } else {
    scoped_chunks(query_len, div_ceil(query_len, threads), body);
  }
}

static size_t preferred_decode_attention_thread_count(size_t heads, size_t head_dim,
                                                      size_t attended_len) {
  // attention.rs:1215-1231
  const size_t kMin = 32768;
  size_t work = sat_mul(sat_mul(heads, head_dim), attended_len);
  if (work < kMin || heads < 2) return 1;
  return std::min(available_parallelism(), heads);
}

// attention.rs:520-686, 965-1025: cache positions [0, cache_len) first, the slot last
void decode_causal_attention_f32(const float* query, const float* cached_key,
                                 const float* cached_value, size_t cache_len,
                                 const float* key_slot, const float* value_slot, size_t hq,
                                 size_t hkv, size_t d, float* out) {
  check_gqa(hq, hkv);
  size_t group = hq / hkv;
  float scale = attention_scale(d);
  auto body = [&](size_t h0, size_t h1) {
    for (size_t h = h0; h < h1; ++h) {
      size_t kvh = h / group;
      const float* q = query + h * d;
      float* o = out + h * d;
      std::fill(o, o + d, 0.0f);
      float m = -std::numeric_limits<float>::infinity();
      float s = 0.0f;
      for (size_t p = 0; p < cache_len; ++p) {
        float score = dot(q, cached_key + (p * hkv + kvh) * d, d) * scale;
        float w = update_online_softmax(o, d, &m, &s, score);
        accumulate(o, cached_value + (p * hkv + kvh) * d, w, d);
      }
      float slot_score = dot(q, key_slot + kvh * d, d) * scale;
      float w = update_online_softmax(o, d, &m, &s, slot_score);
      accumulate(o, value_slot + kvh * d, w, d);
      finish_row(o, s, d);
    }
  };
  size_t threads = preferred_decode_attention_thread_count(hq, d, cache_len + 1);
  if (threads == 1) {
    body(0, hq);
  } else {
    scoped_chunks(hq, div_ceil(hq, threads), body);
  }
}

// ---------------------------------------------------------------------------
// elementwise.rs:48-207 (in-place add / mul / SiLU)
// ---------------------------------------------------------------------------
static size_t preferred_elementwise_thread_count(size_t count) {
  // elementwise.rs:209-219
  const size_t kMin = 131072;
  if (count < kMin) return 1;
  return std::min(available_parallelism(), count);
}

static void elementwise(size_t count, const std::function<void(size_t, size_t)>& body) {
  size_t threads = preferred_elementwise_thread_count(count);
  if (threads == 1) {
    body(0, count);
  } else {
    scoped_chunks(count, div_ceil(count, threads), body);
  }
}

void silu_f32_in_place(float* values, size_t count) {
  elementwise(count, [&](size_t i0, size_t i1) {
    for (size_t i = i0; i < i1; ++i) {
      float v = values[i];
      float e = std::exp(-v);
      float sigmoid = 1.0f / (1.0f + e);
      values[i] = v * sigmoid;
    }
  });
}

void mul_f32_in_place(float* out, const float* rhs, size_t count) {
  elementwise(count, [&](size_t i0, size_t i1) {
    for (size_t i = i0; i < i1; ++i) out[i] = out[i] * rhs[i];
  });
}

void add_f32_in_place(float* out, const float* rhs, size_t count) {
  elementwise(count, [&](size_t i0, size_t i1) {
    for (size_t i = i0; i < i1; ++i) out[i] = out[i] + rhs[i];
  });
}

// ---------------------------------------------------------------------------
// bf16 storage
// ---------------------------------------------------------------------------
float bf16_to_f32(uint16_t bits) {
  uint32_t w = static_cast<uint32_t>(bits) << 16;
  float f;
  std::memcpy(&f, &w, 4);
  return f;
}

uint16_t f32_to_bf16_rne(float value) {
  uint32_t w;
  std::memcpy(&w, &value, 4);
  if ((w & 0x7f800000u) == 0x7f800000u && (w & 0x007fffffu) != 0) {
    return static_cast<uint16_t>((w >> 16) | 0x0040u);  // quiet NaN, sign kept
  }
  uint32_t lsb = (w >> 16) & 1u;
  w += 0x7fffu + lsb;
  return static_cast<uint16_t>(w >> 16);
}

}  // namespace orc
