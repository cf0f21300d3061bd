// Device-side token sampling: sample_last_token (runtime/sampler.rs:121-241) and, for greedy
// configurations, argmax_last_token (sampler.rs:77-119), one workgroup of 8 waves per logits
// row.
//
// Top-k.  The reference keeps its k candidates by streaming replacement: the first k logits
// fill the list; a later logit that is strictly larger (IEEE >) than the list's minimum
// replaces the FIRST minimum in list order (Iterator::min_by over total_cmp).  Replacement
// keeps the list's values equal to the k largest values of the prefix scanned so far, so:
//   * fast path, one pass: a logit below the k+1-th largest value of some part of the row
//     cannot be among the k + 1 largest.  Each wave buffers in LDS only the logits at or above
//     its running bound (the k+1-th largest of what it has buffered, raised to the other
//     waves' bounds) and compacts the buffer by radix selection when it fills.  When the k+1
//     largest values of the row are strictly decreasing and the row holds no NaN, the final
//     list is exactly the k largest logits, in value order.  With equal values among them the
//     list still holds the same values in the same sorted order (equal values, equal weights),
//     so the total, the top-p prefix and the drawn position are exact; only the token at the
//     drawn position can differ, when its value is shared with another logit;
//   * then, or with a NaN in the row, list positions decide which equal logit is kept and how
//     equal candidates are ordered, and the replacement is replayed: in rounds of one
//     1024-logit step per wave, every wave keeps the logits of its step above the list
//     minimum published at the round's start (the minimum never falls, so a logit not above
//     it cannot enter later), in index order; wave 0, holding the list in registers, applies
//     them one by one against the current minimum.  The list is then sorted stably by
//     total_cmp descending.
// top_k above 1024 (up to the vocabulary) runs in sample_large_kernel over an area the host
// reserves (fi_sample_reserve): a radix sort of the row's candidates and sequential walks over
// the sorted weights, with the same replay, over a tree of list minima, for a shared drawn
// value.
// Weights exp(l / T - l0 / T) are computed in parallel; one lane then forms the total, the
// top-p prefix, the retained total, the xorshift64* draw and the threshold walk, sequentially
// in f32 in list order.  The exponential is the device expf; the reference's is the host
// libm's, so a weight may differ in its last bit.
#include <algorithm>

#include "fi_common.h"
#include "fi_device.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxTopK = 1024;
constexpr int kPerLane = 16;          // logits per lane per wave step
constexpr int kStep = 64 * kPerLane;  // logits per wave step
constexpr int kGroup = 256;           // logits per wave appended between buffer checks
constexpr int kRegion = 1536;         // buffered candidates per wave: k + 1 (at most 1025), equal ones, one group
constexpr int kSortMax = 2048;        // fast-path candidates sorted at the end
constexpr int kRankSortMax = 256;     // at most this many: rank counting, else a bitonic sort
constexpr int kIntMin = static_cast<int>(0x80000000u);

// total_cmp as a signed-integer order
__device__ __forceinline__ int32_t total_key(float v) {
  const int32_t b = __float_as_int(v);
  return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
}

__device__ __forceinline__ float key_value(int32_t key) {
  return __int_as_float(key ^ static_cast<int32_t>(static_cast<uint32_t>(key >> 31) >> 1));
}

__device__ __forceinline__ int lanes_below(uint64_t ballot) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(ballot), 0)));
}

template <int VEC>
__device__ __forceinline__ void load_vec(const float* p, float (&v)[VEC]) {
  if constexpr (VEC == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
  } else {
    v[0] = *p;
  }
}

// Logit e (0..kPerLane) of this lane in wave step s: groups of VEC consecutive logits, lanes
// ascending within a group, groups ascending.
template <int VEC>
__device__ __forceinline__ int step_index(int s, int lane, int e) {
  return s * kStep + ((e / VEC) * 64 + lane) * VEC + (e % VEC);
}

// The kPerLane logits of wave step s (addresses clamped into the row; step_index < vocab
// tells which are real).
template <int VEC>
__device__ __forceinline__ void load_step(const float* row, int vocab, int s, int lane, float (&v)[kPerLane]) {
  const int last = vocab - VEC;  // last vector start (vocab % VEC == 0)
#pragma unroll
  for (int j = 0; j < kPerLane / VEC; ++j) {
    float t[VEC];
    load_vec<VEC>(row + min(step_index<VEC>(s, lane, j * VEC), last), t);
#pragma unroll
    for (int u = 0; u < VEC; ++u) v[j * VEC + u] = t[u];
  }
}

// Runs f(logits, s) over wave steps first, first + stride, ... with a ring of four step
// buffers (the first three primed by prime_steps with the same range): three steps of loads
// are in flight while one is processed.  Every call is made
// unconditionally (steps at or past nsteps hold no real logit; f masks them by index) so that
// no load is sunk into a branch next to its use.  Those steps load step nsteps - 1 again, which
// the range has just read, instead of the logits past the range (another segment's, which
// would be read from memory twice).
// The ring's first three steps, loaded by prime_steps before the row's configuration is read
// (the loads do not depend on it), so the configuration's round trip overlaps them.
struct StepRing {
  float b0[kPerLane], b1[kPerLane], b2[kPerLane];
};

template <int VEC>
__device__ __forceinline__ void prime_steps(const float* row, int vocab, int first, int stride, int nsteps, int lane,
                                            StepRing& ring) {
  const int last = max(nsteps - 1, 0);
  load_step<VEC>(row, vocab, min(first, last), lane, ring.b0);
  load_step<VEC>(row, vocab, min(first + stride, last), lane, ring.b1);
  load_step<VEC>(row, vocab, min(first + 2 * stride, last), lane, ring.b2);
}

template <int VEC, typename F>
__device__ __forceinline__ void stream_steps(const float* row, int vocab, int first, int stride, int nsteps, int lane,
                                             StepRing& ring, F&& f) {
  const int last = max(nsteps - 1, 0);
  float(&b0)[kPerLane] = ring.b0;
  float(&b1)[kPerLane] = ring.b1;
  float(&b2)[kPerLane] = ring.b2;
  float b3[kPerLane];
  for (int s = first; s < nsteps; s += 4 * stride) {
    load_step<VEC>(row, vocab, min(s + 3 * stride, last), lane, b3);
    f(b0, s);
    load_step<VEC>(row, vocab, min(s + 4 * stride, last), lane, b0);
    f(b1, s + stride);
    load_step<VEC>(row, vocab, min(s + 5 * stride, last), lane, b1);
    f(b2, s + 2 * stride);
    load_step<VEC>(row, vocab, min(s + 6 * stride, last), lane, b2);
    f(b3, s + 3 * stride);
  }
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Inclusive prefix sum over the wave in DPP moves (no LDS round trips): row_shr 1, 2, 4, 8
// scan each row of 16 lanes (lanes shifted in from outside the row add 0), row_bcast:15 adds
// the last lane of rows 0 and 2 to rows 1 and 3, row_bcast:31 the last lane of row 1 to rows
// 2 and 3.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  return x;
}

// Radix selection, one 8-bit digit: hist[256] holds the counts of the candidates matching the
// digits chosen so far; returns the digit of the element of descending rank `want` among them
// and makes `want` its rank within that digit (one wave).
__device__ __forceinline__ int pick_digit_desc(const int* hist, int lane, int& want) {
  int c[4];
  int tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c[q] = hist[255 - (4 * lane + q)];  // lanes ascending = digits descending
    tot += c[q];
  }
  const int incl = wave_inclusive_sum(tot);
  const int excl = incl - tot;
  const bool here = excl <= want && want < incl;
  int digit = 0, below = 0, acc = excl;
  bool found = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (here && !found && want < acc + c[q]) {
      digit = 255 - (4 * lane + q);
      below = acc;
      found = true;
    }
    acc += c[q];
  }
  const int src = __builtin_ctzll(__ballot(here));
  digit = __builtin_amdgcn_readlane(digit, src);
  below = __builtin_amdgcn_readlane(below, src);
  want -= below;
  return digit;
}

// Key of descending rank `rank` among key[0, n) (one wave; n > rank).
__device__ int wave_select_desc(const int* key, int n, int rank, int* hist, int lane) {
  uint32_t prefix = 0, mask = 0;
  int want = rank;
  for (int d = 24; d >= 0; d -= 8) {
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[lane + 64 * q] = 0;
    wave_sync();
    for (int i = lane; i < n; i += 64) {
      const uint32_t u = static_cast<uint32_t>(key[i]) ^ 0x80000000u;
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> d) & 255u], 1);
    }
    wave_sync();
    const int digit = pick_digit_desc(hist, lane, want);
    prefix |= static_cast<uint32_t>(digit) << d;
    mask |= 255u << d;
    wave_sync();
  }
  return static_cast<int>(prefix ^ 0x80000000u);
}

// Keeps the entries of key/idx[0, n) with key >= bound, in place; returns their count (one wave).
__device__ int wave_compact(int* key, int* idx, int n, int bound, int lane) {
  int out = 0;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const bool in = i < n;
    const int kk = in ? key[i] : 0;
    const int ii = in ? idx[i] : 0;
    const bool keep = in && kk >= bound;
    const uint64_t b = __ballot(keep);
    wave_sync();  // the chunk is read before any of it is overwritten
    if (keep) {
      const int pos = out + lanes_below(b);
      key[pos] = kk;
      idx[pos] = ii;
    }
    out += __popcll(b);
    wave_sync();
  }
  return out;
}

// (key, id) before (key', id') in (key descending, id ascending) order.
__device__ __forceinline__ bool before(int ka, int ia, int kb, int ib) { return ka > kb || (ka == kb && ia < ib); }

// Sorts key/id[0, n) into (key descending, id ascending) order in place (whole workgroup;
// the arrays hold at least the next power of two >= n entries).
__device__ void block_bitonic_sort(int* key, int* id, int n, int tid) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int i = n + tid; i < n2; i += kThreads) {
    key[i] = kIntMin;
    id[i] = 0x7fffffff;
  }
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < (n2 >> 1); t += kThreads) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const int ka = key[i], ia = id[i], kb = key[j], ib = id[j];
        const bool up = (i & size) == 0;
        if (up ? before(kb, ib, ka, ia) : before(ka, ia, kb, ib)) {
          key[i] = kb;
          id[i] = ib;
          key[j] = ka;
          id[j] = ia;
        }
      }
      __syncthreads();
    }
  }
}

// Minimum of wave 0's register list by total_cmp, first list position among equal minima.
template <int NS>
__device__ __forceinline__ void list_min(const float (&val)[NS], int k, int lane, int* pos, float* minv) {
  int best_key = 0x7fffffff, best_pos = 0x7fffffff;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    const int key = total_key(val[s]);
    if (p < k && key < best_key) {  // slots ascend, so the first equal minimum stays
      best_key = key;
      best_pos = p;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int ok = __shfl_xor(best_key, off, 64);
    const int op = __shfl_xor(best_pos, off, 64);
    if (ok < best_key || (ok == best_key && op < best_pos)) {
      best_key = ok;
      best_pos = op;
    }
  }
  *pos = best_pos;
  float v = 0.0f;  // the owner lane's slot value (every slot is read so the list stays in registers)
#pragma unroll
  for (int s = 0; s < NS; ++s) v = (s == (best_pos >> 6)) ? val[s] : v;
  *minv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), best_pos & 63));
}

struct SampleShared {
  int key[kWaves][kRegion];  // per-wave candidate buffers (fast path: total_cmp keys; replay: logit bits)
  int idx[kWaves][kRegion];  // their logit indices
  int hist[kWaves][256];
  union {
    struct {
      int key[kSortMax];
      int idx[kSortMax];
    } fast;  // candidates at or above the k+1-th largest logit, then sorted
    struct {
      float val[kMaxTopK];
      int idx[kMaxTopK];
    } list;  // the replayed list, by position
  } u;
  float s_val[kMaxTopK + 1];  // the sorted list
  int s_idx[kMaxTopK + 1];
  alignas(16) float wts[kMaxTopK];  // its weights (zero past k)
  int bound[kWaves];    // each wave's current lower bound (a total_cmp key)
  int count[kWaves];
  int flags;  // bit 0: NaN seen, bit 1: buffer overflow, bit 2: not strictly decreasing
  int sel[2];
  int m;
  int draw;       // the drawn list position, -1 when the row faulted
  float pub_min;  // replay: the list minimum at the start of the round
  float red_f[kWaves][2];
  int red_i[kWaves][3];
};

// The reference's replacement over the whole row, replayed exactly (whole workgroup; wave 0
// holds the list, NS slots per lane).  Leaves list position p in sh.u.list.val[p] / idx[p].
template <int VEC, int NS>
__device__ __forceinline__ void replay_top_k(const float* row, int vocab, int k, int w, int lane, SampleShared& sh) {
  float val[NS];
  int idx[NS];
  int min_pos = 0;
  float min_val = 0.0f;
  if (w == 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int p = s * 64 + lane;
      val[s] = p < k ? row[p] : 0.0f;
      idx[s] = p;
    }
    list_min<NS>(val, k, lane, &min_pos, &min_val);
    if (lane == 0) sh.pub_min = min_val;
  }
  __syncthreads();
  const int nsteps = (vocab + kStep - 1) / kStep;
  const int first = k / kStep;  // the first step holding an index >= k
  float cur[kPerLane], nxt[kPerLane];
  load_step<VEC>(row, vocab, first + w, lane, cur);
  for (int r0 = first; r0 < nsteps; r0 += kWaves) {
    const int s = r0 + w;
    load_step<VEC>(row, vocab, s + kWaves, lane, nxt);
    // this wave's step: logits above the published minimum, in index order
    const float bound = sh.pub_min;
    const bool full = s * kStep >= k && (s + 1) * kStep <= vocab;
    int cnt = 0;
#pragma unroll
    for (int g = 0; g < kPerLane / VEC; ++g) {
      uint64_t b[VEC];
      int before_lane = 0;
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        const int i = step_index<VEC>(s, lane, g * VEC + u);
        b[u] = __ballot((full || (i >= k && i < vocab)) && cur[g * VEC + u] > bound);
        before_lane += lanes_below(b[u]);
      }
      int within = 0;
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        if ((b[u] >> lane) & 1) {
          const int pos = cnt + before_lane + within;
          sh.key[w][pos] = __float_as_int(cur[g * VEC + u]);
          sh.idx[w][pos] = step_index<VEC>(s, lane, g * VEC + u);
          ++within;
        }
      }
#pragma unroll
      for (int u = 0; u < VEC; ++u) cnt += __popcll(b[u]);
    }
    if (lane == 0) sh.count[w] = cnt;
    __syncthreads();
    if (w == 0) {
      for (int q = 0; q < kWaves; ++q) {
        const int c = sh.count[q];
        for (int base = 0; base < c; base += 64) {
          const int i = base + lane;
          const bool in = i < c;
          const float x = in ? __int_as_float(sh.key[q][i]) : 0.0f;
          const int id = in ? sh.idx[q][i] : 0;
          uint64_t ball = __ballot(in && x > min_val);
          while (ball) {  // wave-uniform, in index order
            const int j = __builtin_ctzll(ball);
            ball &= ball - 1;
            const float xj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
            if (xj > min_val) {
              const int idj = __builtin_amdgcn_readlane(id, j);
              const int slot = min_pos >> 6, owner = min_pos & 63;
#pragma unroll
              for (int t = 0; t < NS; ++t) {
                if (t == slot && lane == owner) {
                  val[t] = xj;
                  idx[t] = idj;
                }
              }
              list_min<NS>(val, k, lane, &min_pos, &min_val);
            }
          }
        }
      }
      if (lane == 0) sh.pub_min = min_val;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kPerLane; ++e) cur[e] = nxt[e];
  }
  if (w == 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int p = s * 64 + lane;
      if (p < k) {
        sh.u.list.val[p] = val[s];
        sh.u.list.idx[p] = idx[s];
      }
    }
  }
  __syncthreads();
}

// A sampling weight's exponential, f32 in and out: the f64 exponential rounded once to f32,
// which is the correctly rounded f32 result except when the exact value lies within an f64
// error of an f32 rounding midpoint.  The reference calls the host libm's expf; glibc 2.35's
// equals this on all but 0.0086 % of the floats in [-104, 0] (every 7th bit pattern checked),
// where the device's own f32 exponential, accurate to about an ulp, differs far more often.
// One differing weight can change the rounding of every later partial sum, so with hundreds
// of thousands of weights in one sequential sum the closer exponential keeps the drawn token
// the reference's.
__device__ __forceinline__ float weight_exp(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

__device__ __forceinline__ uint64_t xorshift_step(uint64_t x) {
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  return x;
}

__device__ __forceinline__ void sampling_fault(uint32_t* faults, uint32_t bit, int32_t* token, float* prob, int r) {
  atomicOr(faults, bit);
  token[r] = -1;
  prob[r] = 0.0f;
}

constexpr float kLog2e = 1.4426950408889634f;

// Combines two (running maximum, sum of 2^(x - maximum)) pairs in log2 units; a maximum of
// -inf carries no mass.
__device__ __forceinline__ void merge_softmax(float& m, float& sum, float om, float os) {
  const float nm = fmaxf(m, om);
  sum = (m > -INFINITY ? sum * __builtin_amdgcn_exp2f(m - nm) : 0.0f) +
        (om > -INFINITY ? os * __builtin_amdgcn_exp2f(om - nm) : 0.0f);
  m = nm;
}

// ---- shared phases of the two launches ----
// Each phase takes the kernel's LDS object by reference and is force-inlined: compiled as a
// separate function (a call from the kernel), the fast path's results were wrong.

constexpr int kMaxSegs = kWaves;  // row segments: segment j's candidates fill wave buffer j of the finish

// One segment's greedy partial: last maximal key / index, (running maximum, sum of 2^(x - max))
// in log2 units, and whether a NaN or +inf was seen.
struct GreedyPart {
  int key;
  int idx;
  float m;
  float sum;
  int bad;
  int pad[3];
};

// What the scan leaves per (row, segment): its candidate count and flags (bit 0 NaN, bit 1 a
// buffer overflowed), or the greedy partial.
struct ScanMeta {
  int count;
  int flags;
  int pad[2];
  GreedyPart g;
};

__device__ __forceinline__ bool greedy_row(float T, int K, float P) {  // SamplerConfig::is_greedy (sampler.rs:40-42)
  return T <= 0.0f || K == 1 || P <= 0.0f;
}

// Greedy pass over wave steps [s0, s1) (logit indices below lim), whole workgroup: the last
// maximal key by total_cmp (later equal maxima win: indices ascend per lane) and the sum of
// exp(l - max) against a running maximum raised once per 16 logits (base-2 exponentials of
// log2e-scaled logits); a NaN or +inf marks the row bad.  tid 0 returns the workgroup's part.
template <int VEC>
__device__ __forceinline__ GreedyPart greedy_pass(const float* row, int vocab, int s0, int s1, int lim, int w, int lane, int tid,
                                  SampleShared& sh, StepRing& ring) {
  int bk = kIntMin, bi = -1;
  float m = -INFINITY, sum = 0.0f;
  bool bad = false;
  stream_steps<VEC>(row, vocab, s0 + w, kWaves, s1, lane, ring, [&](const float (&v)[kPerLane], int s) {
    const int valid = lim - s * kStep;
    if (valid <= 0) return;  // a ring slot past the segment (wave-uniform)
    if (valid >= kStep) {
      // A whole step.  Its maximum (NaN-propagating, -0 below +0, so for NaN-free steps it is
      // the maximum by total_cmp) gates the per-logit key comparisons, which then run only
      // where a lane's best can move.  A step holding a NaN or +inf takes the path below.
      float top = v[0];
#pragma unroll
      for (int e = 1; e < kPerLane; ++e) top = __builtin_elementwise_maximum(top, v[e]);
      if (!__ballot(!(top < INFINITY))) {
        if (__ballot(total_key(top) >= bk)) {
#pragma unroll
          for (int e = 0; e < kPerLane; ++e) {
            const int key = total_key(v[e]);
            const bool take = key >= bk;
            bk = take ? key : bk;
            bi = take ? s * kStep + step_index<VEC>(0, lane, e) : bi;
          }
        }
        // the same running maximum and sum as below (x * log2e is monotonic in x)
        const float nm = fmaxf(m, top * kLog2e);
        sum = (nm > m) ? sum * __builtin_amdgcn_exp2f(m - nm) : sum;
        m = nm;
        const float base = m > -INFINITY ? m : 0.0f;
#pragma unroll
        for (int e = 0; e < kPerLane; ++e) sum += __builtin_amdgcn_exp2f(v[e] * kLog2e - base);
        return;
      }
    }
    float xs[kPerLane];
    float smax = -INFINITY;
#pragma unroll
    for (int e = 0; e < kPerLane; ++e) {
      const int off = step_index<VEC>(0, lane, e);
      const bool in = off < valid;
      const float x = v[e];
      const int key = total_key(x);
      const bool take = in && key >= bk;
      bk = take ? key : bk;
      bi = take ? s * kStep + off : bi;
      bad = bad || (in && !(x < INFINITY));
      xs[e] = (in && x > -INFINITY && x < INFINITY) ? x * kLog2e : -INFINITY;
      smax = fmaxf(smax, xs[e]);
    }
    const float nm = fmaxf(m, smax);
    sum = (nm > m) ? sum * __builtin_amdgcn_exp2f(m - nm) : sum;  // m = -inf: sum is 0
    m = nm;
    const float base = m > -INFINITY ? m : 0.0f;
#pragma unroll
    for (int e = 0; e < kPerLane; ++e) sum += __builtin_amdgcn_exp2f(xs[e] - base);
  });
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int ok = __shfl_xor(bk, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ok > bk || (ok == bk && oi > bi)) {
      bk = ok;
      bi = oi;
    }
    merge_softmax(m, sum, __shfl_xor(m, off, 64), __shfl_xor(sum, off, 64));
  }
  bad = __ballot(bad) != 0;
  if (lane == 0) {
    sh.red_i[w][0] = bk;
    sh.red_i[w][1] = bi;
    sh.red_i[w][2] = bad;
    sh.red_f[w][0] = m;
    sh.red_f[w][1] = sum;
  }
  __syncthreads();
  GreedyPart g{bk, bi, m, sum, bad ? 1 : 0, {0, 0, 0}};
  if (tid == 0) {
    for (int i = 1; i < kWaves; ++i) {
      if (sh.red_i[i][0] > g.key || (sh.red_i[i][0] == g.key && sh.red_i[i][1] > g.idx)) {
        g.key = sh.red_i[i][0];
        g.idx = sh.red_i[i][1];
      }
      merge_softmax(g.m, g.sum, sh.red_f[i][0], sh.red_f[i][1]);
      g.bad = g.bad || sh.red_i[i][2];
    }
  }
  return g;
}

// One pass over wave steps [s0, s1) (logit indices below lim): each wave buffers in its LDS
// region the logits that can be among the k+1 largest of what the workgroup has seen (whole
// workgroup).  Leaves sh.count[w] and sets sh.flags bit 0 (NaN) / bit 1 (a region overflowed
// with equal logits).
template <int VEC>
__device__ __forceinline__ void buffer_pass(const float* row, int vocab, int s0, int s1, int lim, int k, int w, int lane,
                            SampleShared& sh, StepRing& ring) {
  int* rkey = sh.key[w];
  int* ridx = sh.idx[w];
  int bound = kIntMin, cnt = 0;
  uint32_t nan_bits = 0;  // max of |bits|: above 0x7f800000 when a NaN was seen
  stream_steps<VEC>(row, vocab, s0 + w, kWaves, s1, lane, ring, [&](const float (&v)[kPerLane], int s) {
    const int valid = lim - s * kStep;  // logits of this step below lim: step_index offsets < valid
    if (valid <= 0) return;             // a ring slot past the segment (wave-uniform)
    if (k < 64 && s < s0 + kWaves) {
      // the wave's first step seeds its bound: the (k+1)-th largest of the 64 lane maxima.
      // k+1 distinct logits of the step are at or above it, so nothing below it can be among
      // the k+1 largest (empty lanes hold the minimum key).  It is the largest t with at least
      // k+1 lane maxima at or above t, built bit by bit from the top over order-preserving
      // unsigned keys, one ballot a bit.  Later steps raise the bound by compaction.
      int lmax = kIntMin;
#pragma unroll
      for (int e = 0; e < kPerLane; ++e)
        lmax = max(lmax, step_index<VEC>(0, lane, e) < valid ? total_key(v[e]) : kIntMin);
      const uint32_t u = static_cast<uint32_t>(lmax) ^ 0x80000000u;
      uint32_t t = 0;
#pragma unroll
      for (int b = 31; b >= 0; --b) {
        const uint32_t c = t | (1u << b);
        t = __popcll(__ballot(u >= c)) > k ? c : t;
      }
      bound = max(bound, static_cast<int>(t ^ 0x80000000u));
      // published at once, so the other waves filter their later steps against it too (the
      // wave buffers the k+1 logits that make it valid in this step)
      if (lane == 0) atomicMax(&sh.bound[w], bound);
    }
    int hits = 0;
    if (valid >= kStep) {
      // a whole step: its NaN-propagating maximum (-0 below +0) decides whether any logit
      // reaches the bound; a NaN marks the row and sends the step to the appends, which
      // test every logit
      float top = v[0];
#pragma unroll
      for (int e = 1; e < kPerLane; ++e) top = __builtin_elementwise_maximum(top, v[e]);
      const bool nan = top != top;
      nan_bits = nan ? 0x7fffffffu : nan_bits;
      hits = (nan || total_key(top) >= bound) ? 1 : 0;
    } else {
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) {
        const bool in = step_index<VEC>(0, lane, e) < valid;
        const uint32_t bits = __float_as_uint(v[e]);
        nan_bits = max(nan_bits, in ? bits & 0x7fffffffu : 0u);
        hits += (in && total_key(v[e]) >= bound) ? 1 : 0;
      }
    }
    if (__ballot(hits > 0)) {  // rare once the bound has risen: append a group at a time
#pragma unroll
      for (int g = 0; g < kPerLane / (kGroup / 64); ++g) {
#pragma unroll
        for (int e = g * (kGroup / 64); e < (g + 1) * (kGroup / 64); ++e) {
          const bool pass = step_index<VEC>(0, lane, e) < valid && total_key(v[e]) >= bound;
          const uint64_t ball = __ballot(pass);
          if (pass) {
            const int pos = cnt + lanes_below(ball);
            rkey[pos] = total_key(v[e]);
            ridx[pos] = step_index<VEC>(s, lane, e);
          }
          cnt += __popcll(ball);
        }
        if (cnt > kRegion - kGroup) {
          wave_sync();
          bound = max(bound, wave_select_desc(rkey, cnt, k, sh.hist[w], lane));
          cnt = wave_compact(rkey, ridx, cnt, bound, lane);
          if (lane == 0) atomicMax(&sh.bound[w], bound);
          if (cnt > kRegion - kGroup) {  // equal logits fill the buffer: the row is replayed
            if (lane == 0) atomicOr(&sh.flags, 2);
            cnt = 0;
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      bound = max(bound, __hip_atomic_load(&sh.bound[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    }
  });
  if (__ballot(nan_bits > 0x7f800000u) && lane == 0) atomicOr(&sh.flags, 1);
  if (lane == 0) sh.count[w] = cnt;
  __syncthreads();
}

// The key of descending rank `rank` over the wave buffers' sh.count[q] entries (radix
// selection, 8 bits a round; whole workgroup; the buffers hold more than `rank` entries).
__device__ __forceinline__ int select_desc(SampleShared& sh, int rank, int tid, int w, int lane) {
  // Up to kOwn candidates a thread (flattened over the wave buffers) are read into registers
  // once, so each round's histogram is a few compares and increments instead of a loop whose
  // bounds and keys are LDS reads; larger sets read the buffers every round.
  constexpr int kOwn = 4;
  int cnt[kWaves];
  int total = 0;
#pragma unroll
  for (int q = 0; q < kWaves; ++q) {
    cnt[q] = sh.count[q];
    total += cnt[q];
  }
  const bool held = total <= kOwn * kThreads;  // workgroup-uniform
  uint32_t own[kOwn];
#pragma unroll
  for (int j = 0; j < kOwn; ++j) {
    own[j] = 0;
    int rem = held && tid + j * kThreads < total ? tid + j * kThreads : -1;
    int qsel = -1, isel = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      if (rem >= 0 && qsel < 0) {
        if (rem < cnt[q]) {
          qsel = q;
          isel = rem;
        } else {
          rem -= cnt[q];
        }
      }
    }
    // candidate tid + j * kThreads (held when below total) as an order-preserving unsigned key
    if (qsel >= 0) own[j] = static_cast<uint32_t>(sh.key[qsel][isel]) ^ 0x80000000u;
  }
  uint32_t prefix = 0, mask = 0;
  int want = rank;
  for (int d = 24; d >= 0; d -= 8) {
    if (tid < 256) sh.hist[0][tid] = 0;
    __syncthreads();
    if (held) {
#pragma unroll
      for (int j = 0; j < kOwn; ++j) {
        if (tid + j * kThreads < total && (own[j] & mask) == prefix) atomicAdd(&sh.hist[0][(own[j] >> d) & 255u], 1);
      }
    } else {
      for (int q = 0; q < kWaves; ++q) {
        for (int i = tid; i < cnt[q]; i += kThreads) {
          const uint32_t u = static_cast<uint32_t>(sh.key[q][i]) ^ 0x80000000u;
          if ((u & mask) == prefix) atomicAdd(&sh.hist[0][(u >> d) & 255u], 1);
        }
      }
    }
    __syncthreads();
    if (w == 0) {
      const int digit = pick_digit_desc(sh.hist[0], lane, want);
      if (lane == 0) {
        sh.sel[0] = digit;
        sh.sel[1] = want;
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sh.sel[0]) << d;
    mask |= 255u << d;
    want = sh.sel[1];
    __syncthreads();
  }
  return static_cast<int>(prefix ^ 0x80000000u);
}

// Fast path after the buffering: the k+1-th largest key over the wave buffers, the candidates
// at or above it sorted by (key descending, index ascending) into s_val / s_idx.  Sets flags
// bit 2 unless the top k+1 are strictly decreasing (the list is then exactly the top k in value
// order; otherwise tie_at decides whether the drawn token needs the replay).  Returns false,
// sending the row to the replay, when more candidates share the boundary value than it sorts.
__device__ __forceinline__ bool fast_top_k(SampleShared& sh, int k, int tid, int w, int lane) {
  int total = 0;
  for (int q = 0; q < kWaves; ++q) total += sh.count[q];
  if (total <= kRankSortMax) {
    // few candidates (every buffer holds more than k of them together): all of them go to the
    // rank sort, whose order is total, so no selection round is needed
    int base = 0;
    for (int q = 0; q < kWaves; ++q) {
      for (int i = tid; i < sh.count[q]; i += kThreads) {
        sh.u.fast.key[base + i] = sh.key[q][i];
        sh.u.fast.idx[base + i] = sh.idx[q][i];
      }
      base += sh.count[q];
    }
    if (tid == 0) sh.m = total;
  } else {
    const int kth = select_desc(sh, k, tid, w, lane);
    for (int q = 0; q < kWaves; ++q) {
      for (int i = tid; i < sh.count[q]; i += kThreads) {
        if (sh.key[q][i] >= kth) {
          const int pos = atomicAdd(&sh.m, 1);
          if (pos < kSortMax) {
            sh.u.fast.key[pos] = sh.key[q][i];
            sh.u.fast.idx[pos] = sh.idx[q][i];
          }
        }
      }
    }
  }
  __syncthreads();
  const int m = sh.m;
  if (m > kSortMax) return false;
  // ---- ranks 0..k by (key descending, index ascending) ----
  if (m <= kRankSortMax) {
    for (int i = tid; i < m; i += kThreads) {
      const int key = sh.u.fast.key[i], id = sh.u.fast.idx[i];
      int rank = 0;
      for (int j = 0; j < m; ++j) rank += before(sh.u.fast.key[j], sh.u.fast.idx[j], key, id);
      if (rank <= k) {
        sh.s_val[rank] = key_value(key);
        sh.s_idx[rank] = id;
      }
    }
  } else {
    block_bitonic_sort(sh.u.fast.key, sh.u.fast.idx, m, tid);
    for (int i = tid; i <= k; i += kThreads) {
      sh.s_val[i] = key_value(sh.u.fast.key[i]);
      sh.s_idx[i] = sh.u.fast.idx[i];
    }
  }
  __syncthreads();
  for (int i = tid; i < k; i += kThreads) {
    if (!(sh.s_val[i] > sh.s_val[i + 1])) atomicOr(&sh.flags, 4);
  }
  __syncthreads();
  return true;
}

// With equal values among the k+1 largest (flags bit 2) the fast path's list holds the values
// of the reference's list, in the same sorted order, but not necessarily its indices where
// values are equal.  Equal values have equal weights, so the total, the top-p prefix and the
// drawn position are the reference's; the token at that position is too unless its value is
// shared with another logit of the row (IEEE equality, so +0 with -0).  Such a value's other
// logits are all among the candidates (their keys reach the k+1-th largest), and sorted next
// to it.  Zero is sent to the replay whenever flags bit 2 is set: a -0 below the candidates
// can stand in the reference's list for a +0 here.
__device__ __forceinline__ bool tie_at(const SampleShared& sh, int sel) {
  const float v = sh.s_val[sel];
  return v == 0.0f || (sel > 0 && sh.s_val[sel - 1] == v) || sh.s_val[sel + 1] == v;
}

// The reference's replacement over the whole row, replayed; then a stable sort by total_cmp
// into s_val / s_idx (whole workgroup).
template <int VEC>
__device__ __forceinline__ void replay_sorted(const float* row, int vocab, int k, int tid, int w, int lane,
                                              SampleShared& sh) {
  if (k < vocab) {
    if (k <= 64) {
      replay_top_k<VEC, 1>(row, vocab, k, w, lane, sh);
    } else if (k <= 256) {
      replay_top_k<VEC, 4>(row, vocab, k, w, lane, sh);
    } else {
      replay_top_k<VEC, 16>(row, vocab, k, w, lane, sh);
    }
  } else {
    for (int p = tid; p < k; p += kThreads) {
      sh.u.list.val[p] = row[p];
      sh.u.list.idx[p] = p;
    }
    __syncthreads();
  }
  if (k <= kRankSortMax) {
    for (int i = tid; i < k; i += kThreads) {
      const int key = total_key(sh.u.list.val[i]);
      int rank = 0;
      for (int j = 0; j < k; ++j) rank += before(total_key(sh.u.list.val[j]), j, key, i);
      sh.s_val[rank] = sh.u.list.val[i];
      sh.s_idx[rank] = sh.u.list.idx[i];
    }
  } else {  // (key, list position) pairs in the first wave buffer
    for (int i = tid; i < k; i += kThreads) {
      sh.key[0][i] = total_key(sh.u.list.val[i]);
      sh.idx[0][i] = i;
    }
    __syncthreads();
    block_bitonic_sort(sh.key[0], sh.idx[0], k, tid);
    for (int i = tid; i < k; i += kThreads) {
      sh.s_val[i] = sh.u.list.val[sh.idx[0][i]];
      sh.s_idx[i] = sh.u.list.idx[sh.idx[0][i]];
    }
  }
  __syncthreads();
}

// Weights (parallel), then the total, top-p, draw and threshold walk (one lane, in the
// reference's sequential f32 order) over the sorted list s_val / s_idx of k candidates.  Leaves
// the drawn list position in sh.draw and writes the probability, or faults the row (sh.draw
// -1).  Every thread returns after the closing barrier.
// SamplerState::next_f32 (sampler.rs:62-75): advances rng[r] and returns the draw.
__device__ __forceinline__ float next_draw(uint64_t* rng, int r) {
  const uint64_t x = xorshift_step(rng[r]);
  rng[r] = x;
  const uint32_t upper = static_cast<uint32_t>((x * 0x2545F4914F6CDD1DULL) >> 40);
  return static_cast<float>(upper) / 16777216.0f;
}

// The total, top-p prefix, draw and threshold walk of sampler.rs:190-233 over k weights in
// list order (one lane; wts 16-byte aligned and zero from k to the next multiple of 8).  The
// top-p loop's running sum repeats the total's additions in the same order from the same +0,
// so the retained total, summed again from the start by the reference, is the running sum
// where that loop stops.  Returns the drawn position and writes the probability, or faults the
// row and returns -1.
__device__ __forceinline__ int draw_one(const float* wts, int k, float P, uint64_t* rng, int32_t* token, float* prob,
                                        uint32_t* faults, int r) {
#pragma clang fp contract(off)
  const float4* w4 = reinterpret_cast<const float4*>(wts);  // + 0.0f past k leaves a sum >= +0 unchanged
  float total = 0.0f;
  for (int i = 0; i < k; i += 8) {
    const float4 a = w4[i / 4], b = w4[i / 4 + 1];
    total = total + a.x;
    total = total + a.y;
    total = total + a.z;
    total = total + a.w;
    total = total + b.x;
    total = total + b.y;
    total = total + b.z;
    total = total + b.w;
  }
  if (!(total <= 3.402823466e+38f) || total <= 0.0f) {  // not finite, or no mass
    sampling_fault(faults, FI_FAULT_SAMPLE_NONFINITE, token, prob, r);
    return -1;
  }
  float p = P;  // f32::clamp(0, 1): a NaN stays NaN
  if (p < 0.0f) p = 0.0f;
  if (p > 1.0f) p = 1.0f;
  const float cutoff = p >= 1.0f ? total : total * p;
  float kept = 0.0f;
  int retained = 0;
  for (int i = 0; i < k; i += 4) {
    const float4 a = w4[i / 4];
    const float t[4] = {a.x, a.y, a.z, a.w};
    bool reached = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!reached && i + j < k) {
        kept = kept + t[j];
        ++retained;
        reached = kept >= cutoff;
      }
    }
    if (reached) break;
  }
  const float retained_total = kept;  // retained >= 1: the loop adds at least one weight
  float threshold = next_draw(rng, r) * retained_total;
  int sel = 0;
  for (int i = 0; i < retained; i += 4) {
    const float4 a = w4[i / 4];
    const float t[4] = {a.x, a.y, a.z, a.w};
    bool hit = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!hit && i + j < retained) {
        threshold = threshold - t[j];
        if (threshold <= 0.0f) {
          sel = i + j;
          hit = true;
        }
      }
    }
    if (hit) break;
  }
  prob[r] = wts[sel] / retained_total;
  return sel;
}

__device__ __forceinline__ void weights_and_draw(SampleShared& sh, int k, float T, float P, uint64_t* rng,
                                                 int32_t* token, float* prob, uint32_t* faults, int r, int tid) {
  const float temp = fmaxf(T, 1.1920929e-7f);  // max(f32::EPSILON); a NaN temperature gives EPSILON
  const float scaled_max = sh.s_val[0] / temp;
  for (int i = tid; i < kMaxTopK; i += kThreads) sh.wts[i] = i < k ? weight_exp((sh.s_val[i] / temp) - scaled_max) : 0.0f;
  __syncthreads();
  if (tid == 0) sh.draw = draw_one(sh.wts, k, P, rng, token, prob, faults, r);
  __syncthreads();
}

// The token at the drawn position (whole workgroup, after weights_and_draw): the fast path's
// list answers unless tie_at finds the drawn value shared, in which case the reference's
// replacement is replayed for the order of the equal values (their weights, and so the drawn
// position, are unchanged).
template <int VEC>
__device__ __forceinline__ void write_token(SampleShared& sh, const float* row, int vocab, int k, bool fast,
                                            int32_t* token, int r, int tid, int w, int lane) {
  const int sel = sh.draw;
  if (sel < 0) return;  // faulted
  if (fast && (sh.flags & 4) && tie_at(sh, sel)) replay_sorted<VEC>(row, vocab, k, tid, w, lane, sh);
  if (tid == 0) token[r] = sh.s_idx[sel];
}

// ---- launch 1: one workgroup per (row segment, row) ----
// Segment j covers wave steps [j * seg_steps, (j + 1) * seg_steps).  Greedy rows leave their
// segment's partial; sampled rows with k < vocab and k <= 1024 leave every logit of the segment
// at or above the segment's k+1-th largest (a superset of the row's top k+1 that lies in the
// segment) in the workspace, unordered; a flag (NaN, overflow, more than one region of
// candidates) sends the row to the full replay in the finish.
template <int VEC>
__global__ __launch_bounds__(kThreads) void sample_scan_kernel(const float* __restrict__ logits, int ld, int vocab,
                                                               int segs, int seg_steps,
                                                               const float* __restrict__ temperature,
                                                               const int32_t* __restrict__ top_k,
                                                               const float* __restrict__ top_p, ScanMeta* __restrict__ meta,
                                                               int* __restrict__ cand_key, int* __restrict__ cand_idx) {
  __shared__ SampleShared sh;
  const int seg = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float* row = logits + (size_t)r * ld;
  const int nsteps = (vocab + kStep - 1) / kStep;
  const int s0 = seg * seg_steps, s1 = min(nsteps, s0 + seg_steps);
  const int lim = min(vocab, s1 * kStep);
  ScanMeta* out = meta + (size_t)r * segs + seg;
  StepRing ring;
  prime_steps<VEC>(row, vocab, s0 + w, kWaves, s1, lane, ring);
  if (greedy_row(temperature[r], top_k[r], top_p[r])) {
    const GreedyPart g = greedy_pass<VEC>(row, vocab, s0, s1, lim, w, lane, tid, sh, ring);
    if (tid == 0) out->g = g;
    return;
  }
  const int k = min(max(top_k[r], 1), vocab);
  if (k > kMaxTopK || k >= vocab) return;  // the finish handles these rows alone
  if (tid < kWaves) sh.bound[tid] = kIntMin;
  if (tid == 0) {
    sh.flags = 0;
    sh.m = 0;
  }
  __syncthreads();
  buffer_pass<VEC>(row, vocab, s0, s1, lim, k, w, lane, sh, ring);
  int total = 0;
  for (int q = 0; q < kWaves; ++q) total += sh.count[q];
  int* okey = cand_key + ((size_t)r * segs + seg) * kRegion;
  int* oidx = cand_idx + ((size_t)r * segs + seg) * kRegion;
  if (sh.flags == 0) {
    // the segment's k+1-th largest (every buffered logit when the segment holds at most k+1)
    const int kth = total > k + 1 ? select_desc(sh, k, tid, w, lane) : kIntMin;
    for (int q = 0; q < kWaves; ++q) {
      for (int i = tid; i < sh.count[q]; i += kThreads) {
        if (sh.key[q][i] >= kth) {
          const int pos = atomicAdd(&sh.m, 1);
          if (pos < kRegion) {
            okey[pos] = sh.key[q][i];
            oidx[pos] = sh.idx[q][i];
          }
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    out->count = min(sh.m, kRegion);
    out->flags = sh.flags | (sh.m > kRegion ? 2 : 0);
  }
}

// ---- launch 2: one workgroup per row ----
// Greedy rows merge their segments' partials in segment order; sampled rows gather the
// segments' candidates into the wave buffers and take the fast path, or replay the reference's
// replacement over the whole row; then the weights, top-p, draw and threshold walk.
template <int VEC>
__global__ __launch_bounds__(kThreads) void sample_finish_kernel(
    const float* __restrict__ logits, int ld, int vocab, int segs, const float* __restrict__ temperature,
    const int32_t* __restrict__ top_k, const float* __restrict__ top_p, uint64_t* __restrict__ rng,
    const ScanMeta* __restrict__ meta, const int* __restrict__ cand_key, const int* __restrict__ cand_idx,
    int32_t* __restrict__ token, float* __restrict__ prob, uint32_t* __restrict__ faults, int large) {
  __shared__ SampleShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float* row = logits + (size_t)r * ld;
  const float T = temperature[r];
  const int K = top_k[r];
  const float P = top_p[r];
  const ScanMeta* rm = meta + (size_t)r * segs;

  if (greedy_row(T, K, P)) {
    if (tid == 0) {
      // every segment's part loaded at once (indices clamped, so the loads need no branch),
      // then merged in segment order
      GreedyPart parts[kMaxSegs];
#pragma unroll
      for (int j = 0; j < kMaxSegs; ++j) parts[j] = rm[min(j, segs - 1)].g;
      GreedyPart g = parts[0];
#pragma unroll
      for (int j = 1; j < kMaxSegs; ++j) {
        if (j >= segs) break;
        const GreedyPart o = parts[j];
        if (o.key > g.key || (o.key == g.key && o.idx > g.idx)) {
          g.key = o.key;
          g.idx = o.idx;
        }
        merge_softmax(g.m, g.sum, o.m, o.sum);
        g.bad = g.bad || o.bad;
      }
      token[r] = g.idx;
      prob[r] = (g.bad || !(g.sum > 0.0f)) ? __int_as_float(0x7fc00000) : 1.0f / g.sum;
    }
    return;
  }

  const int k = min(max(K, 1), vocab);  // top_k.max(1).min(vocab_size)
  if (k > kMaxTopK) {  // sample_large_kernel's row when the context reserved for it
    if (!large && tid == 0) sampling_fault(faults, FI_FAULT_SAMPLE_TOPK, token, prob, r);
    return;
  }
  // Wave q copies segment q's candidates (segs <= kWaves).  Its count and first 64 entries are
  // loaded here, beside tid 0's flag loads, so a segment of at most 64 candidates costs no
  // further memory round trip (the entries past the count are never used).
  int c = 0, key0 = 0, idx0 = 0;
  const int* ck = nullptr;
  const int* ci = nullptr;
  if (w < segs) {
    ck = cand_key + ((size_t)r * segs + w) * kRegion;
    ci = cand_idx + ((size_t)r * segs + w) * kRegion;
    c = rm[w].count;
    key0 = ck[lane];
    idx0 = ci[lane];
  }
  if (tid == 0) {
    int f = 0;
#pragma unroll
    for (int j = 0; j < kMaxSegs; ++j) f |= rm[min(j, segs - 1)].flags;  // clamped: loads issued together
    sh.flags = k < vocab ? f : 0;
    sh.m = 0;
  }
  __syncthreads();

  bool sorted = false;  // s_val / s_idx hold the sorted list
  if (k < vocab && sh.flags == 0) {
    if (w < segs) {
      if (lane < c) {
        sh.key[w][lane] = key0;
        sh.idx[w][lane] = idx0;
      }
      for (int i = lane + 64; i < c; i += 64) {
        sh.key[w][i] = ck[i];
        sh.idx[w][i] = ci[i];
      }
    }
    if (lane == 0) sh.count[w] = c;
    __syncthreads();
    sorted = fast_top_k(sh, k, tid, w, lane);
  }

  if (!sorted) replay_sorted<VEC>(row, vocab, k, tid, w, lane, sh);
  weights_and_draw(sh, k, T, P, rng, token, prob, faults, r, tid);
  write_token<VEC>(sh, row, vocab, k, sorted, token, r, tid, w, lane);
}

// ---- the single-launch form: one workgroup per row over the whole row ----
// For launches where a row gets one segment (rows enough to fill the device): the scan's
// buffering and the finish's fast path run back to back on the wave buffers, with no
// workspace round trip.
template <int VEC>
__global__ __launch_bounds__(kThreads) void sample_row_kernel(const float* __restrict__ logits, int ld, int vocab,
                                                              const float* __restrict__ temperature,
                                                              const int32_t* __restrict__ top_k,
                                                              const float* __restrict__ top_p,
                                                              uint64_t* __restrict__ rng, int32_t* __restrict__ token,
                                                              float* __restrict__ prob, uint32_t* __restrict__ faults,
                                                              int large) {
  __shared__ SampleShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float* row = logits + (size_t)r * ld;
  const float T = temperature[r];
  const int K = top_k[r];
  const float P = top_p[r];
  const int nsteps = (vocab + kStep - 1) / kStep;
  StepRing ring;
  prime_steps<VEC>(row, vocab, w, kWaves, nsteps, lane, ring);
  if (greedy_row(T, K, P)) {
    const GreedyPart g = greedy_pass<VEC>(row, vocab, 0, nsteps, vocab, w, lane, tid, sh, ring);
    if (tid == 0) {
      token[r] = g.idx;
      prob[r] = (g.bad || !(g.sum > 0.0f)) ? __int_as_float(0x7fc00000) : 1.0f / g.sum;
    }
    return;
  }
  const int k = min(max(K, 1), vocab);  // top_k.max(1).min(vocab_size)
  if (k > kMaxTopK) {  // sample_large_kernel's row when the context reserved for it
    if (!large && tid == 0) sampling_fault(faults, FI_FAULT_SAMPLE_TOPK, token, prob, r);
    return;
  }
  if (tid < kWaves) sh.bound[tid] = kIntMin;
  if (tid == 0) {
    sh.flags = 0;
    sh.m = 0;
  }
  __syncthreads();
  bool sorted = false;
  if (k < vocab) {
    buffer_pass<VEC>(row, vocab, 0, nsteps, vocab, k, w, lane, sh, ring);
    if (sh.flags == 0) sorted = fast_top_k(sh, k, tid, w, lane);
  }
  if (!sorted) replay_sorted<VEC>(row, vocab, k, tid, w, lane, sh);
  weights_and_draw(sh, k, T, P, rng, token, prob, faults, r, tid);
  write_token<VEC>(sh, row, vocab, k, sorted, token, r, tid, w, lane);
}

// ---- rows whose top-k (clamped) exceeds 1024: one workgroup per row over a reserved area ----
// Row r owns large_row_ints(vocab) ints of the area fi_sample_reserve allocates: two (key,
// index) arrays of vocab entries and room for the replay's block minima.
//   1. A NaN among the first k logits stays in the reference's list (nothing is strictly
//      larger than NaN, so -NaN, the total_cmp minimum, is never replaced, and +NaN, the
//      maximum, is never the minimum): its weight makes the total NaN, the Runtime fault.  A
//      NaN past the first k never enters.
//   2. The row is sorted by total_cmp descending, equal keys by index (stable LSD radix sort;
//      NaN past the first k last).
//   3. Its first k entries hold the values of the reference's list in the reference's sorted
//      order (the list always holds the k largest values of the prefix; with k == vocab the
//      list is the row in index order and the stable sort is exactly the reference's).  The
//      total, top-p prefix and threshold walk run as in draw_one, one lane walking chunks of
//      weights that the other waves stage in LDS one chunk ahead.
//   4. k < vocab and the drawn value shared with another logit (IEEE equality): equal values
//      have equal weights, so only the token at the drawn position can differ, and the
//      reference's replacement is replayed for it.  The list's first minimum (smallest key,
//      then smallest slot) is kept in a three-level tree of minima (64 slots a block, 64
//      blocks a superblock), so an insertion costs three wave reductions instead of a pass
//      over the list.
constexpr int kWalkChunk = 4096;                              // weights staged per walk step
constexpr int kLargeMaxVocab = 1 << 20;                       // vocabularies the large path takes
constexpr int kMaxWalkChunks = kLargeMaxVocab / kWalkChunk;   // also bounds the superblocks
constexpr int kListLds = 16384;                               // replay list keys held in LDS up to this k
constexpr int kSortBatch = 16;                                // 64-key groups a wave loads at once in the sort
constexpr int kStageIters = (kWalkChunk + 447) / 448;         // staging loads per thread (at least 7 waves)
constexpr int kIntMax = 0x7fffffff;

constexpr size_t large_row_ints(int vocab) {
  return 4 * static_cast<size_t>(vocab) + 2 * static_cast<size_t>((vocab + 63) / 64);
}

// total_cmp as an unsigned order, with NaN (which never enters the list past its first k
// slots) below every logit.  Its complement is the sort key: ascending is total_cmp descending.
__device__ __forceinline__ uint32_t select_key(float v) {
  return v != v ? 0u : static_cast<uint32_t>(total_key(v)) ^ 0x80000000u;
}

__device__ __forceinline__ float sort_key_value(uint32_t u) {
  return key_value(static_cast<int32_t>(~u ^ 0x80000000u));
}

// f(x, i) for every logit of the row, in no particular order (whole workgroup; 16 loads in
// flight a thread).
template <typename F>
__device__ __forceinline__ void row_pass(const float* row, int vocab, int tid, F&& f) {
  for (int i0 = 0; i0 < vocab; i0 += 16 * kThreads) {
    float x[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) x[u] = row[min(i0 + u * kThreads + tid, vocab - 1)];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = i0 + u * kThreads + tid;
      if (i < vocab) f(x[u], i);
    }
  }
}

// f(x, g0) over [beg, end) in order, kSortBatch groups of 64 logits at a time (lane l's x[u] is
// logit g0 + 64 u + l, clamped into the range; f masks by index), the next batch's loads issued
// before f runs (one wave).
template <typename F>
__device__ __forceinline__ void range_pass(const float* row, int beg, int end, int lane, F&& f) {
  if (beg >= end) return;
  const int last = end - 1;
  float cur[kSortBatch];
#pragma unroll
  for (int u = 0; u < kSortBatch; ++u) cur[u] = row[min(beg + u * 64 + lane, last)];
  for (int g0 = beg; g0 < end; g0 += kSortBatch * 64) {
    float nxt[kSortBatch];
    const int g1 = g0 + kSortBatch * 64;
    if (g1 < end) {
#pragma unroll
      for (int u = 0; u < kSortBatch; ++u) nxt[u] = row[min(g1 + u * 64 + lane, last)];
    }
    f(cur, g0);
#pragma unroll
    for (int u = 0; u < kSortBatch; ++u) cur[u] = nxt[u];
  }
}

struct LargeShared {
  union {
    struct {
      int hist[kWaves][256];  // each wave's digit counts
      int off[kWaves][256];   // then each wave's running output offset per digit
      int tot[256];
      int base[256];
      int single;  // one digit holds every key: the pass is skipped
    } sort;
    struct {
      alignas(16) float buf[2][kWalkChunk];
    } walk;
    struct {
      int list_key[kListLds];
      int bmin_key[kListLds / 64];
      int bmin_slot[kListLds / 64];
      int ckey[kWaves][kStep];  // each wave's step: logits above the published minimum
      int cidx[kWaves][kStep];
      int count[kWaves];
    } replay;
  } u;
  float chunk_end[kMaxWalkChunks];  // the running weight sum at each chunk's end
  int smin_key[kMaxWalkChunks];     // superblock minima
  int smin_slot[kMaxWalkChunks];
  int cnt_a[kThreads];  // replay result: members of the drawn value per thread's slot range
  int cnt_b[kThreads];
  int stop[2];
  int flag;
  int cut_chunk;  // the chunk where the top-p prefix reaches the cutoff, -1 for a NaN cutoff
  int sel;
  int retained;
  int target;
  int target_rank;
  int target_prim;
  float total;
  float rtotal;
  float wsel;
  float cutoff;
  float run;  // the total's running sum between chunks
  float thr;  // the threshold walk's running value between chunks
  float pub_min;
};

// Stable LSD radix sort of key/val[0, n) by unsigned key ascending, 8 bits a pass, between the
// two array pairs (whole workgroup).  Each wave scatters a contiguous range in order, 64 keys
// at a time: a key goes to its digit's running offset for the wave plus its rank among the
// lanes holding the same digit.  A pass whose digit is the same for every key is skipped.
// Returns true when the result is in the second pair.
__device__ __forceinline__ bool radix_sort_u32(uint32_t* k0, int* v0, uint32_t* k1, int* v1, int n, LargeShared& sh,
                                               int tid, int w, int lane) {
  const int per = (n + kWaves - 1) / kWaves;
  const int beg = min(n, w * per), end = min(n, beg + per);
  bool in1 = false;
  for (int shift = 0; shift < 32; shift += 8) {
    const uint32_t* sk = in1 ? k1 : k0;
    const int* sv = in1 ? v1 : v0;
    uint32_t* dk = in1 ? k0 : k1;
    int* dv = in1 ? v0 : v1;
    for (int d = lane; d < 256; d += 64) sh.u.sort.hist[w][d] = 0;
    wave_sync();
    // batches of kSortBatch groups, the next batch's loads issued before this one is counted
    // (addresses clamped into the range, so the loads need no branch)
    const int last = max(end - 1, beg);
    uint32_t kk[kSortBatch];
    if (beg < end) {
#pragma unroll
      for (int u = 0; u < kSortBatch; ++u) kk[u] = sk[min(beg + u * 64 + lane, last)];
    }
    for (int g0 = beg; g0 < end; g0 += kSortBatch * 64) {
      uint32_t nk[kSortBatch];
      const int g1 = g0 + kSortBatch * 64;
      if (g1 < end) {
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) nk[u] = sk[min(g1 + u * 64 + lane, last)];
      }
#pragma unroll
      for (int u = 0; u < kSortBatch; ++u) {
        if (g0 + u * 64 + lane < end) atomicAdd(&sh.u.sort.hist[w][(kk[u] >> shift) & 255u], 1);
      }
#pragma unroll
      for (int u = 0; u < kSortBatch; ++u) kk[u] = nk[u];
    }
    __syncthreads();
    if (tid < 256) {
      int t = 0;
      for (int q = 0; q < kWaves; ++q) {
        const int h = sh.u.sort.hist[q][tid];
        sh.u.sort.off[q][tid] = t;
        t += h;
      }
      sh.u.sort.tot[tid] = t;
    }
    __syncthreads();
    if (w == 0) {  // exclusive scan of the digit totals, four digits a lane
      int c[4], s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = sh.u.sort.tot[4 * lane + q];
        s += c[q];
      }
      int excl = wave_inclusive_sum(s) - s;
      bool all = false;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sh.u.sort.base[4 * lane + q] = excl;
        excl += c[q];
        all = all || c[q] == n;
      }
      const bool single = __ballot(all) != 0;
      if (lane == 0) sh.u.sort.single = single ? 1 : 0;
    }
    __syncthreads();
    if (!sh.u.sort.single) {
      if (tid < 256) {
        for (int q = 0; q < kWaves; ++q) sh.u.sort.off[q][tid] += sh.u.sort.base[tid];
      }
      __syncthreads();
      uint32_t sk_cur[kSortBatch];
      int sv_cur[kSortBatch];
      if (beg < end) {
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {
          const int i = min(beg + u * 64 + lane, last);
          sk_cur[u] = sk[i];
          sv_cur[u] = sv[i];
        }
      }
      for (int g0 = beg; g0 < end; g0 += kSortBatch * 64) {
        uint32_t sk_nxt[kSortBatch];
        int sv_nxt[kSortBatch];
        const int g1 = g0 + kSortBatch * 64;
        if (g1 < end) {
#pragma unroll
          for (int u = 0; u < kSortBatch; ++u) {
            const int i = min(g1 + u * 64 + lane, last);
            sk_nxt[u] = sk[i];
            sv_nxt[u] = sv[i];
          }
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {
          const uint32_t key = sk_cur[u];
          const bool in = g0 + u * 64 + lane < end;
          const uint32_t d = (key >> shift) & 255u;
          // the lanes holding the same digit: the AND over its 8 bits of the ballot of lanes
          // agreeing on that bit (32-bit halves, one select each)
          const uint64_t valid = __ballot(in);
          uint32_t plo = static_cast<uint32_t>(valid), phi = static_cast<uint32_t>(valid >> 32);
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t bb = __ballot(bit);
            const uint32_t blo = static_cast<uint32_t>(bb), bhi = static_cast<uint32_t>(bb >> 32);
            plo &= bit ? blo : ~blo;
            phi &= bit ? bhi : ~bhi;
          }
          const uint64_t peers = (static_cast<uint64_t>(phi) << 32) | plo;
          const int rank = lanes_below(peers);
          const int cnt = __popcll(peers);
          int* offp = &sh.u.sort.off[w][d];
          const int at = in ? *offp : 0;
          if (in) {
            dk[at + rank] = key;
            dv[at + rank] = sv_cur[u];
          }
          wave_sync();  // every lane has read its offset before the last of each digit moves it
          if (in && rank == cnt - 1) *offp = at + cnt;
          wave_sync();
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {
          sk_cur[u] = sk_nxt[u];
          sv_cur[u] = sv_nxt[u];
        }
      }
      in1 = !in1;
    }
    __syncthreads();
  }
  return in1;
}

// (key, slot) minimum over the wave, smaller slot among equal keys (the first minimum in list
// order); every lane returns it.
__device__ __forceinline__ void wave_min_pair(int& key, int& slot) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int ok = __shfl_xor(key, off, 64);
    const int os = __shfl_xor(slot, off, 64);
    if (ok < key || (ok == key && os < slot)) {
      key = ok;
      slot = os;
    }
  }
}

// The replay list's first minimum from the superblock minima (one wave; every lane returns it).
__device__ __forceinline__ void tree_root(const LargeShared& sh, int nsb, int lane, int& gkey, int& gslot) {
  gkey = kIntMax;
  gslot = kIntMax;
  for (int j = lane; j < nsb; j += 64) {
    const int kk = sh.smin_key[j], ss = sh.smin_slot[j];
    if (kk < gkey || (kk == gkey && ss < gslot)) {
      gkey = kk;
      gslot = ss;
    }
  }
  wave_min_pair(gkey, gslot);
}

__device__ __forceinline__ void wg_sync_memory() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

// Runs f(buf, c, n) on thread 0 for chunks c0, c0 + 1, ... of the weights of sorted positions
// [0, lim) (buf holds chunk c's n weights, zero to the chunk's end) until f returns true; the
// waves other than wave 0 stage the next chunk meanwhile (whole workgroup).
template <typename Weight, typename F>
__device__ __forceinline__ void walk_chunks(LargeShared& sh, int c0, int lim, int tid, Weight&& weight, F&& f) {
  const int nch = (lim + kWalkChunk - 1) / kWalkChunk;
  auto stage = [&](int c, int t0, int nt) {
    float* b = sh.u.walk.buf[c & 1];
    float v[kStageIters];
#pragma unroll
    for (int m = 0; m < kStageIters; ++m) {
      const int j = t0 + m * nt, q = c * kWalkChunk + j;
      v[m] = (j < kWalkChunk && q < lim) ? weight.value(q) : 0.0f;
    }
#pragma unroll
    for (int m = 0; m < kStageIters; ++m) {
      const int j = t0 + m * nt, q = c * kWalkChunk + j;
      if (j < kWalkChunk) b[j] = q < lim ? weight.of(v[m]) : 0.0f;
    }
  };
  if (c0 < nch) stage(c0, tid, kThreads);
  __syncthreads();
  for (int c = c0; c < nch; ++c) {
    if (tid >= 64 && c + 1 < nch) stage(c + 1, tid - 64, kThreads - 64);
    if (tid == 0) sh.stop[c & 1] = f(sh.u.walk.buf[c & 1], c, min(kWalkChunk, lim - c * kWalkChunk)) ? 1 : 0;
    __syncthreads();
    if (sh.stop[c & 1]) break;  // two flags: thread 0 sets the next while late waves read this one
  }
  __syncthreads();
}

// s + a.x + a.y + a.z + a.w and s - a.x - a.y - a.z - a.w, one rounding at a time in order.
__device__ __forceinline__ float add4(float s, float4 a) {
  s = s + a.x;
  s = s + a.y;
  s = s + a.z;
  return s + a.w;
}

__device__ __forceinline__ float sub4(float s, float4 a) {
  s = s - a.x;
  s = s - a.y;
  s = s - a.z;
  return s - a.w;
}

// exp(l / T - l0 / T) of a sorted position, as the reference forms it (sampler.rs:184-188).
struct SortedWeight {
  const uint32_t* keys;
  float temp;
  float scaled_max;
  __device__ float value(int q) const { return sort_key_value(keys[q]); }
  __device__ float of(float v) const { return weight_exp((v / temp) - scaled_max); }
};

template <int VEC>
__global__ __launch_bounds__(kThreads) void sample_large_kernel(const float* __restrict__ logits, int ld, int vocab,
                                                                const float* __restrict__ temperature,
                                                                const int32_t* __restrict__ top_k,
                                                                const float* __restrict__ top_p,
                                                                uint64_t* __restrict__ rng, int* __restrict__ area,
                                                                int32_t* __restrict__ token, float* __restrict__ prob,
                                                                uint32_t* __restrict__ faults) {
#pragma clang fp contract(off)
  __shared__ LargeShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float T = temperature[r];
  const int K = top_k[r];
  const float P = top_p[r];
  if (greedy_row(T, K, P)) return;
  const int k = min(max(K, 1), vocab);  // top_k.max(1).min(vocab_size)
  if (k <= kMaxTopK) return;            // the scan / finish kernels' row
  const float* row = logits + (size_t)r * ld;
  int* base = area + r * large_row_ints(vocab);
  uint32_t* key0 = reinterpret_cast<uint32_t*>(base);
  int* idx0 = base + vocab;
  uint32_t* key1 = reinterpret_cast<uint32_t*>(base + 2 * static_cast<size_t>(vocab));
  int* idx1 = base + 3 * static_cast<size_t>(vocab);
  int* aux = base + 4 * static_cast<size_t>(vocab);

  // ---- 1. candidates in index order: every logit when k == vocab, else those at or above the
  // k+1-th largest (a NaN past the first k counts as below every logit); a NaN among the
  // first k faults the row ----
  if (tid < 256) sh.u.sort.tot[tid] = 0;
  if (tid == 0) sh.flag = 0;
  __syncthreads();
  bool nan_early = false;
  row_pass(row, vocab, tid, [&](float x, int i) {
    nan_early = nan_early || (x != x && i < k);
    if (k < vocab) atomicAdd(&sh.u.sort.tot[select_key(x) >> 24], 1);
  });
  if (nan_early) sh.flag = 1;
  __syncthreads();
  if (sh.flag) {
    if (tid == 0) sampling_fault(faults, FI_FAULT_SAMPLE_NONFINITE, token, prob, r);
    return;
  }
  uint32_t bound = 0;  // select_key of the k+1-th largest
  if (k < vocab) {
    uint32_t prefix = 0, mask = 0;
    int want = k;
    for (int d = 24; d >= 0; d -= 8) {
      if (d < 24) {  // the first digit's counts came with the NaN check
        if (tid < 256) sh.u.sort.tot[tid] = 0;
        __syncthreads();
        row_pass(row, vocab, tid, [&](float x, int) {
          const uint32_t u = select_key(x);
          if ((u & mask) == prefix) atomicAdd(&sh.u.sort.tot[(u >> d) & 255u], 1);
        });
        __syncthreads();
      }
      if (w == 0) {
        const int digit = pick_digit_desc(sh.u.sort.tot, lane, want);
        if (lane == 0) {
          sh.target = digit;
          sh.target_rank = want;
        }
      }
      __syncthreads();
      prefix |= static_cast<uint32_t>(sh.target) << d;
      mask |= 255u << d;
      want = sh.target_rank;
      __syncthreads();
    }
    bound = prefix;
  }
  // each wave compacts its contiguous range in index order at its offset: counts, then copies
  const int span = ((vocab + kWaves - 1) / kWaves + 63) / 64 * 64;
  const int beg = min(vocab, w * span), end = min(vocab, beg + span);
  int mine = 0;
  range_pass(row, beg, end, lane, [&](const float* x, int g0) {
#pragma unroll
    for (int u = 0; u < kSortBatch; ++u) {
      mine += __popcll(__ballot(g0 + u * 64 + lane < end && select_key(x[u]) >= bound));
    }
  });
  if (lane == 0) sh.cnt_a[w] = mine;
  __syncthreads();
  int at = 0, m = 0;
  for (int q = 0; q < kWaves; ++q) {
    at += q < w ? sh.cnt_a[q] : 0;
    m += sh.cnt_a[q];
  }
  range_pass(row, beg, end, lane, [&](const float* x, int g0) {
#pragma unroll
    for (int u = 0; u < kSortBatch; ++u) {
      const int i = g0 + u * 64 + lane;
      const bool keep = i < end && select_key(x[u]) >= bound;
      const uint64_t b = __ballot(keep);
      if (keep) {
        const int pos = at + lanes_below(b);
        key0[pos] = ~select_key(x[u]);  // ascending = total_cmp descending; NaN last
        idx0[pos] = i;
      }
      at += __popcll(b);
    }
  });
  __syncthreads();

  // ---- 2. sort ----
  const bool in1 = radix_sort_u32(key0, idx0, key1, idx1, m, sh, tid, w, lane);
  const uint32_t* sk = in1 ? key1 : key0;
  const int* si = in1 ? idx1 : idx0;
  int* free_key = reinterpret_cast<int*>(in1 ? key0 : key1);
  int* free_idx = in1 ? idx0 : idx1;

  // ---- 3. total, top-p, draw (sampler.rs:184-233) ----
  const float temp = fmaxf(T, 1.1920929e-7f);  // max(f32::EPSILON); a NaN temperature gives EPSILON
  const SortedWeight wt{sk, temp, sort_key_value(sk[0]) / temp};
  // thread 0's running sums live in LDS between chunks (sh.run, sh.thr) and in a register
  // within one
  if (tid == 0) sh.run = 0.0f;
  walk_chunks(sh, 0, k, tid, wt, [&](const float* b, int c, int n) {
    // blocks of 64 weights: the block's 16 LDS reads issued together, so their latency is paid
    // once per 64 dependent additions (the chunk is zero-padded: + 0.0f leaves a sum >= +0
    // unchanged)
    const float4* b4 = reinterpret_cast<const float4*>(b);
    float s = sh.run;
    for (int q = 0; q < n; q += 64) {
      float4 x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = b4[q / 4 + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) s = add4(s, x[u]);
    }
    sh.run = s;
    sh.chunk_end[c] = s;
    return false;
  });
  if (tid == 0) {
    const float total = sh.run;
    sh.total = total;
    sh.flag = (!(total <= 3.402823466e+38f) || total <= 0.0f) ? 1 : 0;  // not finite, or no mass
    if (sh.flag) {
      sampling_fault(faults, FI_FAULT_SAMPLE_NONFINITE, token, prob, r);
    } else {
      float p = P;  // f32::clamp(0, 1): a NaN stays NaN
      if (p < 0.0f) p = 0.0f;
      if (p > 1.0f) p = 1.0f;
      const float cutoff = p >= 1.0f ? total : total * p;
      sh.cutoff = cutoff;
      sh.retained = k;  // a NaN cutoff is never reached: every candidate is kept
      sh.rtotal = total;
      sh.cut_chunk = -1;
      if (cutoff == cutoff) {
        int c = 0;  // the first chunk whose running sum reaches the cutoff (total >= cutoff)
        while (sh.chunk_end[c] < cutoff) ++c;
        sh.cut_chunk = c;
      }
    }
  }
  __syncthreads();
  if (sh.flag) return;
  if (sh.cut_chunk >= 0) {
    // the top-p loop's running sum is the total's (same additions, same order), so the walk
    // restarts at the crossing chunk from the sum at its start
    const int cc = sh.cut_chunk;
    const float cutoff = sh.cutoff;
    walk_chunks(sh, cc, k, tid, wt, [&](const float* b, int c, int n) {
      // the running sum never falls, so a block of 32 whose last sum is below the cutoff holds
      // no crossing; the first block that reaches it is walked again one weight at a time
      float s = c > 0 ? sh.chunk_end[c - 1] : 0.0f;
      for (int q = 0; q < n; q += 32) {
        float e = s;
#pragma unroll
        for (int j = 0; j < 32; ++j) e = e + b[q + j];
        if (e >= cutoff) {
          for (int j = 0; j < 32; ++j) {
            s = s + b[q + j];
            if (s >= cutoff) {
              sh.retained = c * kWalkChunk + q + j + 1;
              sh.rtotal = s;
              break;
            }
          }
          break;
        }
        s = e;
      }
      return true;
    });
  }
  if (tid == 0) {
    sh.thr = next_draw(rng, r) * sh.rtotal;
    sh.sel = 0;
    sh.wsel = wt.of(wt.value(0));
  }
  walk_chunks(sh, 0, sh.retained, tid, wt, [&](const float* b, int c, int n) {
    // the threshold never rises, so a block of 64 whose last value is above zero holds no hit;
    // the first block that reaches zero is walked again one weight at a time (weights past the
    // retained ones are zero-padded and leave the threshold as it is)
    const float4* b4 = reinterpret_cast<const float4*>(b);
    float t = sh.thr;
    int at = -1;  // the first block of 64 that brings the threshold to zero
    for (int q = 0; q < n; q += 64) {
      float4 x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = b4[q / 4 + u];
      float e = t;
#pragma unroll
      for (int u = 0; u < 16; ++u) e = sub4(e, x[u]);
      if (e <= 0.0f) {
        at = q;
        break;
      }
      t = e;
    }
    if (at >= 0) {  // walked again one weight at a time from the block's start
      for (int j = 0; j < 64; ++j) {
        t = t - b[at + j];
        if (t <= 0.0f) {
          sh.sel = c * kWalkChunk + at + j;
          sh.wsel = b[at + j];
          break;
        }
      }
    }
    sh.thr = t;
    return at >= 0;
  });
  const int sel = sh.sel;
  const float vsel = sort_key_value(sk[sel]);
  if (tid == 0) {
    prob[r] = sh.wsel / sh.rtotal;
    const bool tie = k < vocab && ((sel > 0 && sort_key_value(sk[sel - 1]) == vsel) ||
                                   (sel + 1 < m && sort_key_value(sk[sel + 1]) == vsel));
    sh.flag = tie ? 1 : 0;
    if (tie) {
      int lo = 0, hi = sel;  // the drawn value's first sorted position: everything before is larger
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sort_key_value(sk[mid]) > vsel) {
          lo = mid + 1;
        } else {
          hi = mid;
        }
      }
      sh.target_rank = sel - lo;
    } else {
      token[r] = si[sel];
    }
  }
  __syncthreads();
  if (!sh.flag) return;

  // ---- 4. replay of the replacement (sampler.rs:157-171) for the drawn value's order ----
  const bool in_lds = k <= kListLds;
  const int nb = (k + 63) / 64, nsb = (nb + 63) / 64;
  int* lkey = in_lds ? sh.u.replay.list_key : free_key;
  int* lidx = free_idx;
  int* bkey = in_lds ? sh.u.replay.bmin_key : aux;
  int* bslot = in_lds ? sh.u.replay.bmin_slot : aux + (vocab + 63) / 64;
  for (int p = tid; p < k; p += kThreads) {
    lkey[p] = total_key(row[p]);
    lidx[p] = p;
  }
  __syncthreads();
  for (int b = w; b < nb; b += kWaves) {
    const int slot = b * 64 + lane;
    int kk = slot < k ? lkey[slot] : kIntMax, ss = slot;
    wave_min_pair(kk, ss);
    if (lane == 0) {
      bkey[b] = kk;
      bslot[b] = ss;
    }
  }
  __syncthreads();
  for (int q = w; q < nsb; q += kWaves) {
    const int j = q * 64 + lane;
    int kk = j < nb ? bkey[j] : kIntMax, ss = j < nb ? bslot[j] : kIntMax;
    wave_min_pair(kk, ss);
    if (lane == 0) {
      sh.smin_key[q] = kk;
      sh.smin_slot[q] = ss;
    }
  }
  __syncthreads();
  int gkey = kIntMax, gslot = kIntMax;  // wave 0: the list's first minimum
  float min_val = 0.0f;
  if (w == 0) {
    tree_root(sh, nsb, lane, gkey, gslot);
    min_val = key_value(gkey);
    if (lane == 0) sh.pub_min = min_val;
  }
  __syncthreads();
  const int nsteps = (vocab + kStep - 1) / kStep;
  for (int r0 = k / kStep; r0 < nsteps; r0 += kWaves) {
    // each wave keeps the logits of its step above the published minimum, in index order
    const int s = r0 + w;
    float v[kPerLane];
    load_step<VEC>(row, vocab, min(s, nsteps - 1), lane, v);
    const float bound = sh.pub_min;
    int cnt = 0;
#pragma unroll
    for (int g = 0; g < kPerLane / VEC; ++g) {
      uint64_t bl[VEC];
      int before_lane = 0;
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        const int i = step_index<VEC>(s, lane, g * VEC + u);
        bl[u] = __ballot(i >= k && i < vocab && v[g * VEC + u] > bound);
        before_lane += lanes_below(bl[u]);
      }
      int within = 0;
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        if ((bl[u] >> lane) & 1) {
          const int pos = cnt + before_lane + within;
          sh.u.replay.ckey[w][pos] = __float_as_int(v[g * VEC + u]);
          sh.u.replay.cidx[w][pos] = step_index<VEC>(s, lane, g * VEC + u);
          ++within;
        }
      }
#pragma unroll
      for (int u = 0; u < VEC; ++u) cnt += __popcll(bl[u]);
    }
    if (lane == 0) sh.u.replay.count[w] = cnt;
    __syncthreads();
    if (w == 0) {
      for (int q = 0; q < kWaves; ++q) {
        const int c = sh.u.replay.count[q];
        for (int base_i = 0; base_i < c; base_i += 64) {
          const int i = base_i + lane;
          const bool in = i < c;
          const float x = in ? __int_as_float(sh.u.replay.ckey[q][i]) : 0.0f;
          const int id = in ? sh.u.replay.cidx[q][i] : 0;
          uint64_t ball = __ballot(in && x > min_val);
          while (ball) {  // wave-uniform, in index order
            const int j = __builtin_ctzll(ball);
            ball &= ball - 1;
            const float xj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
            if (!(xj > min_val)) continue;
            // the logit replaces the first minimum; its block, superblock and the root follow
            const int slot = gslot, b = slot >> 6, sb = b >> 6;
            if (lane == 0) {
              lkey[slot] = total_key(xj);
              lidx[slot] = __builtin_amdgcn_readlane(id, j);
            }
            wg_sync_memory();
            int kk = b * 64 + lane < k ? lkey[b * 64 + lane] : kIntMax, ss = b * 64 + lane;
            wave_min_pair(kk, ss);
            if (lane == 0) {
              bkey[b] = kk;
              bslot[b] = ss;
            }
            wg_sync_memory();
            const int jb = sb * 64 + lane;
            kk = jb < nb ? bkey[jb] : kIntMax;
            ss = jb < nb ? bslot[jb] : kIntMax;
            wave_min_pair(kk, ss);
            if (lane == 0) {
              sh.smin_key[sb] = kk;
              sh.smin_slot[sb] = ss;
            }
            wg_sync_memory();
            tree_root(sh, nsb, lane, gkey, gslot);
            min_val = key_value(gkey);
          }
        }
      }
      if (lane == 0) sh.pub_min = min_val;
    }
    __syncthreads();
  }

  // The drawn value's entries of the final list, in the stable sort's order (total_cmp
  // descending, then slot): one key, or for zero +0 then -0.  The token is the one of rank
  // target_rank.
  const bool zero = vsel == 0.0f;
  const int kp = zero ? 0 : total_key(vsel);  // total_key(+0.0f) == 0, total_key(-0.0f) == -1
  const int per = (k + kThreads - 1) / kThreads;
  const int p0 = min(k, tid * per), p1 = min(k, p0 + per);
  int ca = 0, cb = 0;
  for (int p = p0; p < p1; ++p) {
    const int kk = lkey[p];
    ca += kk == kp;
    cb += zero && kk == -1;
  }
  sh.cnt_a[tid] = ca;
  sh.cnt_b[tid] = cb;
  __syncthreads();
  if (tid == 0) {
    int na = 0;
    for (int t = 0; t < kThreads; ++t) na += sh.cnt_a[t];
    int want = sh.target_rank;
    const bool prim = want < na;
    if (!prim) want -= na;
    int t = 0;
    for (; t < kThreads; ++t) {
      const int c = prim ? sh.cnt_a[t] : sh.cnt_b[t];
      if (want < c) break;
      want -= c;
    }
    sh.target = t;
    sh.target_rank = want;
    sh.target_prim = prim ? 1 : 0;
    if (t == kThreads) token[r] = si[sel];  // not reached: the list holds the drawn value
  }
  __syncthreads();
  if (tid == sh.target) {
    const int want_key = sh.target_prim ? kp : -1;
    int want = sh.target_rank;
    for (int p = p0; p < p1; ++p) {
      if (lkey[p] == want_key) {
        if (want == 0) {
          token[r] = lidx[p];
          break;
        }
        --want;
      }
    }
  }
}

}  // namespace

extern "C" {

int32_t fi_sample_tokens(fi_context* ctx, const float* d_logits, int32_t ld, int32_t rows, int32_t vocab,
                         const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                         uint64_t* d_rng_state, int32_t* d_token, float* d_prob) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab, FI_ERR_INVALID_SHAPE,
             "fi_sample_tokens: requires non-empty logits rows (vocab > 0, ld >= vocab)");
  if (rows == 0) return FI_OK;
  FI_REQUIRE(d_logits && d_temperature && d_top_k && d_top_p && d_rng_state && d_token && d_prob,
             FI_ERR_INVALID_CONFIG, "fi_sample_tokens: null pointer");
  FI_REQUIRE(rows <= 65535, FI_ERR_INVALID_SHAPE, "fi_sample_tokens: at most 65535 rows per call");
  // rows split only as far as it takes to give every CU a workgroup (one fits a CU): a short
  // segment buffers nearly all of its logits, so more segments cost more than they spread.
  // Segments hold at least four wave steps (4096 logits, more than k + 1 for any k the device
  // takes) and at most one per wave buffer of the finish.
  const int nsteps = (vocab + kStep - 1) / kStep;
  const int cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  const int fill = (cus + rows - 1) / rows;
  const int segs = std::max(1, std::min({kMaxSegs, nsteps / 4, fill}));
  const int seg_steps = (nsteps + segs - 1) / segs;
  const bool vec4 = vocab % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(d_logits) % 16 == 0;
  // rows with top-k above 1024 go to sample_large_kernel when the reserved area covers the call
  const bool large = ctx->sample_area != nullptr && vocab <= kLargeMaxVocab &&
                     static_cast<size_t>(rows) * large_row_ints(vocab) * sizeof(int) <= ctx->sample_bytes;
  const int large_arg = large ? 1 : 0;
  if (segs == 1) {
    if (vec4) {
      hipLaunchKernelGGL(sample_row_kernel<4>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         d_temperature, d_top_k, d_top_p, d_rng_state, d_token, d_prob, ctx->d_faults, large_arg);
    } else {
      hipLaunchKernelGGL(sample_row_kernel<1>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         d_temperature, d_top_k, d_top_p, d_rng_state, d_token, d_prob, ctx->d_faults, large_arg);
    }
    FI_CHECK_LAUNCH("sample_row_kernel");
  } else {
    const size_t meta_bytes = ((size_t)rows * segs * sizeof(ScanMeta) + 255) / 256 * 256;
    const size_t cand_bytes = (size_t)rows * segs * kRegion * sizeof(int);
    FI_TRY(fi::ensure_workspace(ctx, meta_bytes + 2 * cand_bytes));
    ScanMeta* meta = static_cast<ScanMeta*>(ctx->workspace);
    int* cand_key = reinterpret_cast<int*>(static_cast<char*>(ctx->workspace) + meta_bytes);
    int* cand_idx = reinterpret_cast<int*>(static_cast<char*>(ctx->workspace) + meta_bytes + cand_bytes);
    const dim3 scan_grid(static_cast<unsigned>(segs), static_cast<unsigned>(rows));
    if (vec4) {
      hipLaunchKernelGGL(sample_scan_kernel<4>, scan_grid, dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab, segs,
                         seg_steps, d_temperature, d_top_k, d_top_p, meta, cand_key, cand_idx);
      hipLaunchKernelGGL(sample_finish_kernel<4>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         segs, d_temperature, d_top_k, d_top_p, d_rng_state, meta, cand_key, cand_idx, d_token, d_prob,
                         ctx->d_faults, large_arg);
    } else {
      hipLaunchKernelGGL(sample_scan_kernel<1>, scan_grid, dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab, segs,
                         seg_steps, d_temperature, d_top_k, d_top_p, meta, cand_key, cand_idx);
      hipLaunchKernelGGL(sample_finish_kernel<1>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         segs, d_temperature, d_top_k, d_top_p, d_rng_state, meta, cand_key, cand_idx, d_token, d_prob,
                         ctx->d_faults, large_arg);
    }
    FI_CHECK_LAUNCH("sample_finish_kernel");
  }
  if (large) {
    int* area = static_cast<int*>(ctx->sample_area);
    if (vec4) {
      hipLaunchKernelGGL(sample_large_kernel<4>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         d_temperature, d_top_k, d_top_p, d_rng_state, area, d_token, d_prob, ctx->d_faults);
    } else {
      hipLaunchKernelGGL(sample_large_kernel<1>, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, ld, vocab,
                         d_temperature, d_top_k, d_top_p, d_rng_state, area, d_token, d_prob, ctx->d_faults);
    }
    FI_CHECK_LAUNCH("sample_large_kernel");
  }
  return FI_OK;
}

int32_t fi_sample_reserve(fi_context* ctx, int32_t rows, int32_t vocab) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && rows <= 65535 && vocab >= 0, FI_ERR_INVALID_SHAPE,
             "fi_sample_reserve: rows must be in [0, 65535] and vocab non-negative");
  FI_REQUIRE(vocab <= kLargeMaxVocab, FI_ERR_UNSUPPORTED,
             "fi_sample_reserve: top-k above 1024 is served for vocabularies of at most 1048576 logits");
  const size_t bytes = static_cast<size_t>(rows) * large_row_ints(vocab) * sizeof(int);
  if (bytes == 0 || bytes <= ctx->sample_bytes) return FI_OK;
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_sample_reserve: cannot allocate during graph capture");
  if (ctx->sample_area != nullptr) {
    FI_TRY_HIP(hipStreamSynchronize(ctx->stream));  // queued sampling may still read the old area
    FI_TRY_HIP(hipFree(ctx->sample_area));
    ctx->sample_area = nullptr;
    ctx->sample_bytes = 0;
  }
  FI_TRY_HIP(hipMalloc(&ctx->sample_area, bytes));
  ctx->sample_bytes = bytes;
  ctx->workspace_generation += 1;  // graphs captured before hold the old launch sequence
  return FI_OK;
}

}  // extern "C"
