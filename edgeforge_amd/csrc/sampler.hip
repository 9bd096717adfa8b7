// Next-token selection on the device: kern::argmax and ef::Sampler::sample for a batch of
// independent sequences, one workgroup per sequence (src/sampler.cpp:13-70, src/kernels.cpp:105-111).
//
// Bit-exactness with the reference, given identical logits:
//  * penalty (l > 0 ? l / p : l * p), temperature (l / T) and w - mx are single IEEE float ops
//    (correctly rounded divide, no contraction);
//  * the kept set and its order follow the reference comparator exactly: every logit becomes a
//    unique 64-bit key (order-preserving float bits with +0 == -0, then the inverted id), so
//    "higher logit, then lower id" is plain descending key order.  Top-k (k <= 1024) is a radix
//    select over the keys plus a bitonic sort of the k winners in LDS; top-k off (or > 1024) is a
//    full bitonic sort of all keys in the workspace;
//  * the softmax over the kept ids, the top-p cut, its renormalisation and the CDF walk are the
//    reference's left-to-right double sums: on one thread in the same order (the top-k path and
//    more than 32768 kept ids), stopping at the first term that leaves the running sum unchanged
//    (the terms are sorted, non-negative and non-increasing, so no later one can change it), or
//    reproduced exactly in parallel rounds that count each term's rounding within the running
//    sum's binade (exact_scan, below);
//  * the draw is std::uniform_real_distribution<double>(0, 1) over a std::mt19937_64 kept on the
//    device (one state per sequence), advanced once per call exactly when temperature > 0.
// The one libm call, exp(double), is exp_libm (exp_f64.h): glibc's exp to the last bit.
#include <cmath>

#include "common.h"
#include "exp_f64.h"
#include "sampler.h"

#pragma clang fp contract(off)

namespace efh {
namespace {

constexpr int kThreads = 1024;
constexpr int kRegSlots = 32;  // logits per thread on the register path (V <= 32768)
constexpr int kMaxTopK = 1024;
constexpr int kFloorMaxRank = 4;     // top-k by a key floor for k <= 4 * waves (the rest: radix select)
constexpr int kMaxGathered = 2 * kThreads;  // keys above the floor that one LDS sort takes
constexpr int kScanPer = 32;  // sums over sorted terms: terms per thread, contiguous (kScanPer * thread + i)
// The softmax-term region of a sequence's workspace: V rounded up to whole kScanPer-term columns
// (rank_merge_kernel stores term j at (j % kScanPer) * columns + j / kScanPer).
__host__ __device__ constexpr size_t prob_region_bytes(size_t v) {
  return (((v + kScanPer - 1) / kScanPer) * kScanPer * 8 + 255) & ~size_t{255};
}
constexpr int kMtN = 312, kMtM = 156;

// ---- std::mt19937_64 on the device (ISO C++ [rand.predef]) -------------------------------------------
struct MtState {
  uint64_t mt[kMtN];
  int idx;
  int pad[3];
};
static_assert(sizeof(MtState) <= kRngStateBytes, "rng state size");

__device__ void mt_seed(MtState* s, uint64_t seed) {
  s->mt[0] = seed;
  for (int i = 1; i < kMtN; ++i) s->mt[i] = 6364136223846793005ull * (s->mt[i - 1] ^ (s->mt[i - 1] >> 62)) + i;
  s->idx = kMtN;
}

__device__ uint64_t mt_next(MtState* s) {
  if (s->idx >= kMtN) {
    for (int i = 0; i < kMtN; ++i) {
      const uint64_t y = (s->mt[i] & 0xFFFFFFFF80000000ull) | (s->mt[(i + 1) % kMtN] & 0x7FFFFFFFull);
      s->mt[i] = s->mt[(i + kMtM) % kMtN] ^ (y >> 1) ^ ((y & 1ull) ? 0xB5026F5AA96619E9ull : 0ull);
    }
    s->idx = 0;
  }
  uint64_t y = s->mt[s->idx++];
  y ^= (y >> 29) & 0x5555555555555555ull;
  y ^= (y << 17) & 0x71D67FFFEDA60000ull;
  y ^= (y << 37) & 0xFFF7EEE000000000ull;
  y ^= y >> 43;
  return y;
}

// libstdc++ generate_canonical<double, 53> with one 64-bit word, then uniform (0, 1).
__device__ double mt_uniform(MtState* s) {
  const double r = __ull2double_rn(mt_next(s)) * 0x1p-64;
  return r >= 1.0 ? 0x1.fffffffffffffp-1 : r;
}

// Advances every state by k draws (std::mt19937_64::discard).
__global__ void rng_discard_kernel(uint8_t* states, int batch, int k) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  MtState* st = reinterpret_cast<MtState*>(states + static_cast<size_t>(b) * kRngStateBytes);
  for (int i = 0; i < k; ++i) (void)mt_next(st);
}

__global__ void rng_seed_kernel(uint8_t* states, const uint64_t* seeds, int batch) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < batch) mt_seed(reinterpret_cast<MtState*>(states + static_cast<size_t>(b) * kRngStateBytes), seeds[b]);
}

// ---- keys ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_bits(float v) {
  uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);  // +0 and -0 compare equal in the reference
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint64_t make_key(float v, uint32_t id) {
  return (static_cast<uint64_t>(order_bits(v)) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - id);
}
__device__ __forceinline__ uint32_t key_id(uint64_t k) { return 0xFFFFFFFFu - static_cast<uint32_t>(k); }
// The logit a key was made from (-0 comes back as +0, which no later operation tells apart).
__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t u = static_cast<uint32_t>(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// First maximum (strict >, scan order) of x[0..n): returns the index.  NaN never replaces the
// running best; a NaN at index 0 is the answer, as in the sequential scan (kern::argmax,
// src/kernels.cpp:107-115).  Each thread scans its elements in increasing index order (float4
// loads through a buffer resource, all issued before the compares); the merge keeps the larger
// value and, on ties, the lower index, which is the sequential scan's answer.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxUnroll = 8;

__device__ __forceinline__ void take(float v, int i, float& bv, int& bi) {
  if (v == v && (bi == 0x7FFFFFFF || v > bv)) {
    bv = v;
    bi = i;
  }
}

__device__ int block_argmax(const float* x, int n, float* s_val, int* s_idx) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(x, static_cast<uint32_t>(n) * 4u);
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  const int step = blockDim.x * 4;
  for (int base = 0; base < n; base += step * kArgmaxUnroll) {
    float4 v[kArgmaxUnroll];
#pragma unroll
    for (int j = 0; j < kArgmaxUnroll; ++j)
      v[j] = buf_f4(r, static_cast<uint32_t>(base + j * step + threadIdx.x * 4) * 4u);
#pragma unroll
    for (int j = 0; j < kArgmaxUnroll; ++j) {
      const int i = base + j * step + threadIdx.x * 4;
      if (i < n) take(v[j].x, i, bv, bi);
      if (i + 1 < n) take(v[j].y, i + 1, bv, bi);
      if (i + 2 < n) take(v[j].z, i + 2, bv, bi);
      if (i + 3 < n) take(v[j].w, i + 3, bv, bi);
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || ov > bv || (ov == bv && oi < bi))) {
      bv = ov;
      bi = oi;
    }
  }
  const int w = threadIdx.x / kWave, nw = blockDim.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    s_val[w] = bv;
    s_idx[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = s_val[0];
    int i = s_idx[0];
    for (int k = 1; k < nw; ++k) {
      if (s_idx[k] != 0x7FFFFFFF && (i == 0x7FFFFFFF || s_val[k] > v || (s_val[k] == v && s_idx[k] < i))) {
        v = s_val[k];
        i = s_idx[k];
      }
    }
    const float x0 = x[0];
    s_idx[0] = (x0 != x0 || i == 0x7FFFFFFF) ? 0 : i;
  }
  __syncthreads();
  const int res = s_idx[0];
  __syncthreads();
  return res;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* x, int n, long ld, int32_t* out) {
  __shared__ float s_val[kArgmaxThreads / kWave];
  __shared__ int s_idx[kArgmaxThreads / kWave];
  const int r = block_argmax(x + blockIdx.x * ld, n, s_val, s_idx);
  if (threadIdx.x == 0) out[blockIdx.x] = r;
}

// Greedy pick fused with the step bookkeeping of the decode engine (one workgroup per sequence):
// the token becomes the input at p + 1, joins the history, lands in the output list at
// p - (n_prompt - 1); the last workgroup to finish advances the shared position (every workgroup
// has read it before it counts itself in) and re-arms the counter for the next step.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_finish_kernel(const float* x, int n, long ld, StepArgs f) {
  __shared__ float s_val[kArgmaxThreads / kWave];
  __shared__ int s_idx[kArgmaxThreads / kWave];
  const int b = blockIdx.x;
  const int p = *f.pos;
  const int tok = block_argmax(x + b * ld, n, s_val, s_idx);
  if (threadIdx.x == 0) {
    f.next[b] = tok;
    const int k = p - (*f.n_prompt - 1);
    if (p + 1 < f.hist_ld) f.hist[b * f.hist_ld + p + 1] = tok;
    f.hist_len[b] = p + 2 < f.hist_ld ? p + 2 : static_cast<int32_t>(f.hist_ld);
    if (k >= 0 && k < f.out_ld) f.out[b * f.out_ld + k] = tok;
    __threadfence();
    if (atomicAdd(f.counter, 1u) == gridDim.x - 1) {
      *f.pos = p + 1;
      atomicExch(f.counter, 0u);
    }
  }
}

// ---- bitonic sorts (descending) --------------------------------------------------------------------------
__device__ void bitonic_lds(uint64_t* a, int n) {  // n power of two, <= 2 * blockDim
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int l = i ^ j;
        if (l > i) {
          const uint64_t x = a[i], y = a[l];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            a[i] = y;
            a[l] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Full sort of n (power of two, >= kChunk) keys in global memory, descending.  Each kChunk-key
// chunk is held in registers, kChunk / kThreads keys per thread (thread t holds chunk positions
// t + kThreads u), and a compare-exchange step of distance j runs where the partners are: in the
// same thread (j >= kThreads), in the same wave (j < 64, a shuffle), or across waves (one LDS
// exchange, double-buffered, one barrier).  Distances of a chunk or more go through memory.
constexpr int kChunk = 4096;
constexpr int kKeysPerThread = kChunk / kThreads;  // 4

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const int lo = __shfl_xor(static_cast<int>(v & 0xFFFFFFFFu), m, kWave);
  const int hi = __shfl_xor(static_cast<int>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Sort of n <= 64 keys (power of two) in LDS, descending, by wave 0 alone: one key per lane,
// partners exchanged by shuffles, no barrier inside.
__device__ void bitonic_wave(uint64_t* a, int n) {
  if (threadIdx.x < kWave) {
    const int i = threadIdx.x;
    uint64_t x = i < n ? a[i] : 0ull;
    for (int k = 2; k <= n; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        const uint64_t y = shfl_xor_u64(x, j);
        const bool take_max = ((i & k) == 0) == ((i & j) == 0);
        x = take_max ? (x > y ? x : y) : (x < y ? x : y);
      }
    }
    if (i < n) a[i] = x;
  }
  __syncthreads();
}

// Steps j = jmax .. 1 of bitonic stage k on the chunk at global index `base` (x: this thread's keys).
// Every thread of the block calls it (it has barriers); buf holds 2 * kChunk keys.
__device__ void chunk_steps(uint64_t (&x)[kKeysPerThread], int base, int k, int jmax, uint64_t* buf, int& parity) {
  const int t = threadIdx.x;
  for (int j = jmax; j > 0; j >>= 1) {
    uint64_t y[kKeysPerThread];
    static_assert(kKeysPerThread == 4, "partner selection below");
    if (j >= kThreads) {  // partners in this thread: u ^ (j / kThreads), spelled out (no indexing)
      if (j == kThreads) {
        y[0] = x[1];
        y[1] = x[0];
        y[2] = x[3];
        y[3] = x[2];
      } else {
        y[0] = x[2];
        y[1] = x[3];
        y[2] = x[0];
        y[3] = x[1];
      }
    } else if (j >= kWave) {
      uint64_t* b = buf + parity * kChunk;
#pragma unroll
      for (int u = 0; u < kKeysPerThread; ++u) b[t + kThreads * u] = x[u];
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kKeysPerThread; ++u) y[u] = b[(t ^ j) + kThreads * u];
      parity ^= 1;  // the next exchange writes the other buffer, so no second barrier is needed
    } else {
#pragma unroll
      for (int u = 0; u < kKeysPerThread; ++u) y[u] = shfl_xor_u64(x[u], j);
    }
#pragma unroll
    for (int u = 0; u < kKeysPerThread; ++u) {
      const int i = base + t + kThreads * u;
      const bool desc = (i & k) == 0, lower = (i & j) == 0;
      // descending pair: the lower index keeps the larger key (keys are distinct, or equal padding)
      const bool take_max = desc == lower;
      x[u] = (x[u] > y[u]) == take_max ? x[u] : y[u];
    }
  }
}

__device__ void bitonic_global(uint64_t* g, int n, uint64_t* buf) {
  const int t = threadIdx.x;
  if (n < kChunk) {  // small vocabularies: the whole array in LDS
    for (int i = t; i < n; i += blockDim.x) buf[i] = g[i];
    __syncthreads();
    bitonic_lds(buf, n);
    for (int i = t; i < n; i += blockDim.x) g[i] = buf[i];
    __syncthreads();
    return;
  }
  int parity = 0;
  auto load = [&](uint64_t (&x)[kKeysPerThread], int base) {
#pragma unroll
    for (int u = 0; u < kKeysPerThread; ++u) x[u] = g[base + t + kThreads * u];
  };
  auto store = [&](const uint64_t (&x)[kKeysPerThread], int base) {
#pragma unroll
    for (int u = 0; u < kKeysPerThread; ++u) g[base + t + kThreads * u] = x[u];
  };
  for (int base = 0; base < n; base += kChunk) {  // every stage k <= kChunk inside the chunk
    uint64_t x[kKeysPerThread];
    load(x, base);
    for (int k = 2; k <= kChunk; k <<= 1) chunk_steps(x, base, k, k >> 1, buf, parity);
    store(x, base);
  }
  __syncthreads();
  for (int k = kChunk * 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j >= kChunk; j >>= 1) {
      // the pairs (i, i ^ j) with bit j of i clear: q-th pair i = (q & (j-1)) | ((q & ~(j-1)) << 1)
      const int half = n >> 1;
      for (int q0 = t; q0 < half; q0 += 8 * blockDim.x) {
        uint64_t xa[8], ya[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int q = q0 + u * blockDim.x;
          const int i = (q & (j - 1)) | ((q & ~(j - 1)) << 1);
          xa[u] = q < half ? g[i] : 0ull;
          ya[u] = q < half ? g[i | j] : 0ull;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int q = q0 + u * blockDim.x;
          if (q >= half) continue;
          const int i = (q & (j - 1)) | ((q & ~(j - 1)) << 1);
          const bool desc = (i & k) == 0;
          if (desc ? (xa[u] < ya[u]) : (xa[u] > ya[u])) {
            g[i] = ya[u];
            g[i | j] = xa[u];
          }
        }
      }
      __syncthreads();
    }
    for (int base = 0; base < n; base += kChunk) {
      uint64_t x[kKeysPerThread];
      load(x, base);
      chunk_steps(x, base, k, kChunk >> 1, buf, parity);
      store(x, base);
    }
    __syncthreads();
  }
}

// ---- sequential loops of the sampler ---------------------------------------------------------------
// The reference's double sums, nucleus cut and CDF walk are left-to-right loops; thread 0 runs them
// in that order.  A global array is staged into LDS kStage values at a time, double-buffered: while
// thread 0 consumes one block the waves after the first stage the next, so thread 0 reads LDS and
// never waits on global memory after the first block; an array already in LDS is read in place.
// step(v, cnt, first) consumes values in order and returns where the loop ends; every thread
// returns thread 0's stop index (n if none).  `stage` holds 2 kStage doubles.
constexpr int kStage = 4096;
// Thread 0's pass over an array already in LDS (the top-k path's kept terms, at most a few hundred),
// eight values per group: the reads of a group overlap, and step(v, cnt, first) consumes cnt <= 8
// values in order, returning the position in the group where the loop ends (-1: go on).  Returns
// the index where it ended, or m.
template <typename F>
__device__ __forceinline__ int consume(const double* src, int m, int base, F& step) {
  int i = 0;
  for (; i + 8 <= m; i += 8) {  // whole groups: the count is a constant once step is inlined
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[i + u];
    const int e = step(v, 8, base + i);
    if (e >= 0) return i + e;
  }
  if (i < m) {
    const int cnt = m - i;
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = u < cnt ? src[i + u] : 0.0;
    const int e = step(v, cnt, base + i);
    if (e >= 0) return i + e;
  }
  return m;
}

// The same over a staged block of a global array (element i is number base + i): the first
// m - m % 32 values go through a ring of four groups, three groups' reads in flight ahead of the one
// being consumed (an LDS read takes longer than a group's eight dependent adds), the rest as above.
template <typename F>
__device__ __forceinline__ int consume_pipelined(const double* src, int m, int base, F& step) {
  auto load8 = [&](double (&v)[8], int i) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[i + u];
  };
  const int ng = (m / 32) * 4;  // groups through the ring, a multiple of four
  if (ng > 0) {
    double v0[8], v1[8], v2[8], v3[8];
    load8(v0, 0);
    load8(v1, 8);
    load8(v2, 16);
    for (int g = 0; g < ng; g += 4) {
      load8(v3, 8 * (g + 3));
      int e = step(v0, 8, base + 8 * g);
      if (e >= 0) return 8 * g + e;
      if (g + 4 < ng) load8(v0, 8 * (g + 4));
      e = step(v1, 8, base + 8 * (g + 1));
      if (e >= 0) return 8 * (g + 1) + e;
      if (g + 5 < ng) load8(v1, 8 * (g + 5));
      e = step(v2, 8, base + 8 * (g + 2));
      if (e >= 0) return 8 * (g + 2) + e;
      if (g + 6 < ng) load8(v2, 8 * (g + 6));
      e = step(v3, 8, base + 8 * (g + 3));
      if (e >= 0) return 8 * (g + 3) + e;
    }
  }
  const int i0 = 8 * ng;
  const int e = consume(src + i0, m - i0, base + i0, step);
  return i0 + e;
}

template <typename F>
__device__ int serial_loop(const double* p, int n, bool in_lds, double* stage, int* s_stop, F&& step) {
  if (in_lds) {
    if (threadIdx.x == 0) *s_stop = consume(p, n, 0, step);
    __syncthreads();
    const int r = *s_stop;
    __syncthreads();
    return r;
  }
  const int m0 = min(kStage, n);
  for (int i = threadIdx.x; i < m0; i += blockDim.x) stage[i] = p[i];
  __syncthreads();
  int stop = n;
  for (int base = 0; base < n; base += kStage) {
    const int m = min(kStage, n - base), c = base / kStage;
    const double* cur = stage + (c & 1) * kStage;
    if (threadIdx.x < kWave) {
      if (threadIdx.x == 0) {
        const int i = consume_pipelined(cur, m, base, step);
        *s_stop = i < m ? base + i : n;
      }
    } else if (base + kStage < n) {  // the next block into the other buffer
      double* nxt = stage + ((c + 1) & 1) * kStage;
      const int nb = base + kStage, mn = min(kStage, n - nb);
      for (int i = static_cast<int>(threadIdx.x) - kWave; i < mn; i += static_cast<int>(blockDim.x) - kWave)
        nxt[i] = p[nb + i];
    }
    __syncthreads();
    stop = *s_stop;
    __syncthreads();  // s_stop is rewritten next round
    if (stop < n) break;
  }
  return stop;
}

// ---- the sampler --------------------------------------------------------------------------------------------
struct SampleArgs {
  const float* logits;
  long ld;
  int vocab;
  float temperature, top_p, penalty;
  int top_k;
  const int32_t* hist;
  const int32_t* hist_len;
  long hist_ld;
  uint8_t* rng;
  int32_t* out;
  uint8_t* ws;  // workspace base
  size_t ws_stride;
  int npow2;
  int eos_id;     // with eos_p: P(eos_id) under softmax(logits) per sequence
  double* eos_p;  // [batch] or null
  int phase;      // 0: one launch; 1: stop once the keys are written (the sort runs in other launches)
  int fast;       // 1: nucleus_kernel ran first; the full-sort launches take only the sequences it left
};

// P(id) under softmax of the raw logits, in double (prob_of, src/chat.cpp:35-42): max, then the sum
// of exp(l - max) over the vocabulary (per-thread partial sums combined in a fixed order; the
// reference adds left to right, a difference in the last bits of a double).  Thread 0 returns it.
__device__ double softmax_prob(const float* lg, int V, int id, double* red, const uint64_t* etab) {
  const int t = threadIdx.x, nw = blockDim.x / kWave;
  double m = -INFINITY;
  for (int i = t; i < V; i += blockDim.x) m = fmax(m, static_cast<double>(lg[i]));
  for (int o = kWave / 2; o > 0; o >>= 1) m = fmax(m, __shfl_xor(m, o, kWave));
  if ((t & (kWave - 1)) == 0) red[t / kWave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < nw; ++w) m = fmax(m, red[w]);
  __syncthreads();
  double s = 0.0;
  for (int i = t; i < V; i += blockDim.x) s += exp_libm(static_cast<double>(lg[i]) - m, etab);
  s = wave_sum_d(s);
  if ((t & (kWave - 1)) == 0) red[t / kWave] = s;
  __syncthreads();
  double tot = 0.0;
  for (int w = 0; w < nw; ++w) tot += red[w];
  __syncthreads();
  if (id < 0 || id >= V) return 0.0;
  return exp_libm(static_cast<double>(lg[id]) - m, etab) / tot;
}

// The sampler after the sort (src/sampler.cpp:42-69): softmax over the kept ids, the nucleus, the
// draw and the CDF walk.  `sorted` holds the keys in descending order, `stage` 2 kStage doubles of LDS.
__device__ void sample_tail(const SampleArgs& a, int b, const uint64_t* sorted, int keep, bool topk, double* prob,
                            double* s_prob, double* stage, int& s_stop, double& s_sum, int& s_keep,
                            const uint64_t* etab) {
  // softmax over the kept ids in double (src/sampler.cpp:42-49); with top-k the kept probabilities
  // live in LDS, otherwise the sequential loops below stage them through the sort buffer (free
  // once the keys are sorted)
  const bool in_lds = topk;
  if (topk) prob = s_prob;
  const float mx = key_value(sorted[0]);
  for (int i = threadIdx.x; i < keep; i += blockDim.x)
    prob[i] = exp_libm(static_cast<double>(key_value(sorted[i]) - mx), etab);
  __threadfence_block();
  __syncthreads();
  {
    // thread 0's running sum; a group that leaves it unchanged ends the loop (terms after the
    // first unchanged one add nothing either, so checking once per group gives the same sum)
    double sum = 0.0;
    serial_loop(prob, keep, in_lds, stage, &s_stop, [&](const double (&v)[8], int cnt, int) {
      const double before = sum;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (u < cnt) sum = sum + v[u];
      return (sum == before && before > 0.0) ? 0 : -1;
    });
    if (threadIdx.x == 0) s_sum = sum;
    __syncthreads();
  }
  const double sum = s_sum;
  for (int i = threadIdx.x; i < keep; i += blockDim.x) prob[i] = prob[i] / sum;
  __threadfence_block();
  __syncthreads();
  if (a.top_p < 1.0f) {  // nucleus (src/sampler.cpp:50-61)
    double cum = 0.0;
    const double tp = static_cast<double>(a.top_p);
    // n = the number of terms taken; once cum is final and below top_p the loop would take all
    // the running sums of a group in registers; the first that reaches top_p ends the loop, a
    // group that leaves cum unchanged ends it with all terms kept
    // the group's running sums form one chain of adds; the comparisons read them off the chain
    // (values past cnt are zeros: the sums stay put, so the first crossing is inside the group)
    int n = serial_loop(prob, keep, in_lds, stage, &s_stop, [&](const double (&v)[8], int, int) {
      const double before = cum;
      double c[8], x = cum;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        x = x + v[u];
        c[u] = x;
      }
      int hit = -1;
#pragma unroll
      for (int u = 7; u >= 0; --u)
        if (c[u] >= tp) hit = u;
      if (hit >= 0) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u == hit) cum = c[u];
        return hit;
      }
      cum = x;
      return (cum == before && before > 0.0) ? 0 : -1;
    });
    if (threadIdx.x == 0) s_keep = n < keep && cum >= tp ? n + 1 : keep;  // cum < tp: every term
    __syncthreads();
    const int kp = s_keep > 1 ? s_keep : 1;
    // the reference's s2 (the kept terms summed from 0.0 in order, src/sampler.cpp:57-59) adds the
    // same terms in the same order as cum did up to the cut, so it is cum, bit for bit
    if (threadIdx.x == 0) s_sum = cum;
    __syncthreads();
    keep = kp;
    const double s2b = s_sum;
    for (int i = threadIdx.x; i < keep; i += blockDim.x) prob[i] = prob[i] / s2b;
    __threadfence_block();
    __syncthreads();
  }
  // draw and CDF walk (src/sampler.cpp:62-69)
  double r = 0.0;
  if (threadIdx.x == 0) {
    MtState* st = reinterpret_cast<MtState*>(a.rng + static_cast<size_t>(b) * kRngStateBytes);
    r = mt_uniform(st);
  }
  double cum = 0.0;
  int pick = keep - 1;  // the first i with r < cum; the last kept id when the sum ends below r
  serial_loop(prob, keep, in_lds, stage, &s_stop, [&](const double (&v)[8], int, int first) {
    const double before = cum;
    double c[8], x = cum;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      x = x + v[u];
      c[u] = x;
    }
    int hit = -1;
#pragma unroll
    for (int u = 7; u >= 0; --u)
      if (r < c[u]) hit = u;
    if (hit >= 0) {
      pick = first + hit;
      return hit;
    }
    cum = x;
    return (cum == before && before > 0.0) ? 0 : -1;  // cum is final and r >= cum
  });
  if (threadIdx.x == 0) a.out[b] = static_cast<int>(key_id(sorted[pick]));
}

// The logits of ids t + kThreads j (t = threadIdx.x) in registers, the repetition penalty applied
// to every in-range history id once and the temperature (src/sampler.cpp:16-27).  A history id
// t' + kThreads j' sets bit j' of its owner t''s word in s_seen (kThreads words), so each thread
// reads one word for its 32 slots.  V <= kRegSlots * kThreads.
__device__ void load_tempered(const SampleArgs& a, int b, float (&rv)[kRegSlots], uint32_t* s_seen) {
  const int V = a.vocab;
  const float* lg = a.logits + b * a.ld;
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) {
    const int id = threadIdx.x + kThreads * j;
    rv[j] = id < V ? lg[id] : 0.0f;
  }
  if (a.penalty != 1.0f) {
    const int n = a.hist_len[b];
    const int32_t* h = a.hist + b * a.hist_ld;
    s_seen[threadIdx.x] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int t = h[i];
      if (t >= 0 && t < V) atomicOr(&s_seen[t % kThreads], 1u << (t / kThreads));
    }
    __syncthreads();
    const uint32_t marks = s_seen[threadIdx.x];
#pragma unroll
    for (int j = 0; j < kRegSlots; ++j)
      if (marks >> j & 1u) rv[j] = rv[j] > 0.0f ? __fdiv_rn(rv[j], a.penalty) : rv[j] * a.penalty;
  }
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) rv[j] = __fdiv_rn(rv[j], a.temperature);
}

// The `need` largest keys by a radix select, 8 bits per pass from the top: on return the keys k
// with (k & sh.mask) >= sh.prefix are exactly those (keys are unique).  for_each_key(f) calls f on
// every key this thread owns.  Each wave counts into its own histogram (keys of similar logits
// share their top digits, and one shared histogram serialises those atomics across the waves).
// The digit d kept is the largest with S(d) = (keys still in play with digit >= d) >= need, found
// by a parallel suffix sum; need then drops by S(d + 1).  Every thread of the block calls it.
struct SelectShared {
  uint32_t whist[kThreads / kWave * 256];
  uint32_t hist[256], sfx[256];
  uint64_t prefix, mask;
  int need, done;
};

template <typename F>
__device__ void radix_select(int need, F&& for_each_key, SelectShared& sh) {
  constexpr int kWaves = kThreads / kWave;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  if (threadIdx.x == 0) {
    sh.prefix = 0;
    sh.mask = 0;
    sh.need = need;
    sh.done = 0;
  }
  __syncthreads();
  for (int shift = 56; shift >= 0 && !sh.done; shift -= 8) {
    for (int i = threadIdx.x; i < kWaves * 256; i += blockDim.x) sh.whist[i] = 0u;
    __syncthreads();
    const uint64_t prefix = sh.prefix, mask = sh.mask;
    for_each_key([&](uint64_t k) {
      if ((k & mask) == prefix) atomicAdd(&sh.whist[wave * 256 + ((k >> shift) & 255u)], 1u);
    });
    __syncthreads();
    if (threadIdx.x < 256) {  // digit d = threadIdx.x: 4 waves of 64 digits
      const int d = threadIdx.x;
      uint32_t c = 0;
      for (int w = 0; w < kWaves; ++w) c += sh.whist[w * 256 + d];
      sh.hist[d] = c;
      uint32_t sfx = c;  // suffix sum over the wave's digits >= d
      for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t v = __shfl_down(sfx, o, kWave);
        if (lane + o < kWave) sfx += v;
      }
      sh.sfx[d] = sfx;
    }
    __syncthreads();
    if (threadIdx.x < 256) {
      const int d = threadIdx.x, nd = sh.need;
      uint32_t above = 0;  // the waves of higher digits
      for (int w = d / kWave + 1; w < 4; ++w) above += sh.sfx[w * kWave];
      const uint32_t S = sh.sfx[d] + above, S1 = S - sh.hist[d];  // S(d), S(d + 1)
      if ((static_cast<int>(S) >= nd || d == 0) && static_cast<int>(S1) < nd) {
        const int rest = nd - static_cast<int>(S1);
        sh.need = rest;
        sh.prefix = prefix | (static_cast<uint64_t>(d) << shift);
        sh.mask = mask | (255ull << shift);
        if (static_cast<int>(sh.hist[d]) == rest) sh.done = 1;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a) {
  __shared__ uint64_t s_keys[2 * kChunk];  // 64 KB: top-k candidates / sort exchange buffers
  constexpr int kWaves = kThreads / kWave;
  __shared__ SelectShared s_sel;
  __shared__ uint32_t s_floor[kWaves * kFloorMaxRank];  // each wave's largest lane maxima (order bits)
  __shared__ uint32_t s_floor_bits;
  __shared__ float s_val[kThreads / kWave];
  __shared__ int s_idx[kThreads / kWave];
  __shared__ int s_cnt, s_keep, s_stop;
  __shared__ double s_sum;
  __shared__ uint32_t s_seen[(32768 + 31) / 32];  // history marks: a bitmap (V <= 32768), or a word per thread
  __shared__ double s_prob[kMaxTopK];  // the kept probabilities of the top-k path

  const int b = blockIdx.x, V = a.vocab;
  uint8_t* ws = a.ws + static_cast<size_t>(b) * a.ws_stride;
  float* work = reinterpret_cast<float*>(ws);                                   // [V]
  double* prob = reinterpret_cast<double*>(ws + ((V * 4 + 255) & ~255));        // [V] (no top-k)
  uint64_t* keys = reinterpret_cast<uint64_t*>(ws + ((V * 4 + 255) & ~255) + prob_region_bytes(V));  // [npow2]
  const float* lg = a.logits + b * a.ld;
  __shared__ uint64_t s_exp[256];  // exp_libm's table: P(eos) takes V / 1024 terms per thread
  stage_exp_table(s_exp);
  __syncthreads();

  if (a.eos_p != nullptr) {
    __shared__ double s_red[kThreads / kWave];
    const double pe = softmax_prob(lg, V, a.eos_id, s_red, s_exp);
    if (threadIdx.x == 0) a.eos_p[b] = pe;
  }
  // Sampled top-k with V <= kRegSlots * kThreads keeps the logits in registers (thread t holds ids
  // t + kThreads j): penalty, temperature and the radix select never go through memory.
  const bool topk = a.top_k > 0 && a.top_k < V && a.top_k <= kMaxTopK;
  const bool reg = a.temperature > 0.0f && topk && V <= kRegSlots * kThreads;
  float rv[kRegSlots];
  auto ov = [&](int j) { return order_bits(rv[j]); };  // the high half of slot j's key
  auto for_each_key = [&](auto&& f) {
    if (reg) {
#pragma unroll
      for (int j = 0; j < kRegSlots; ++j) {
        const int id = threadIdx.x + kThreads * j;
        if (id < V) f((static_cast<uint64_t>(ov(j)) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - id));
      }
    } else {
      for (int i = threadIdx.x; i < V; i += blockDim.x) f(make_key(work[i], i));
    }
  };
  if (reg) {
    load_tempered(a, b, rv, s_seen);
  } else {
  for (int i = threadIdx.x; i < V; i += blockDim.x) work[i] = lg[i];
  __syncthreads();
  // repetition penalty: each unique in-range history id once (src/sampler.cpp:16-24).  The result
  // depends only on which ids occur (each penalised value is a function of its own logit), so the
  // history entries are taken in parallel: the entry whose atomicOr sets its id's bit applies it.
  if (a.penalty != 1.0f) {
    const int n = a.hist_len[b];
    const int32_t* h = a.hist + b * a.hist_ld;
    if (V <= 32768) {
      for (int i = threadIdx.x; i < (V + 31) / 32; i += blockDim.x) s_seen[i] = 0u;
      __syncthreads();
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = h[i];
        if (t < 0 || t >= V) continue;
        const uint32_t bit = 1u << (t & 31);
        if (atomicOr(&s_seen[t >> 5], bit) & bit) continue;
        const float l = work[t];
        work[t] = l > 0.0f ? __fdiv_rn(l, a.penalty) : l * a.penalty;
      }
    } else {  // large vocabularies: the first occurrence of each id applies it
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = h[i];
        if (t < 0 || t >= V) continue;
        bool dup = false;
        for (int j = 0; j < i && !dup; ++j) dup = h[j] == t;
        if (dup) continue;
        const float l = work[t];
        work[t] = l > 0.0f ? __fdiv_rn(l, a.penalty) : l * a.penalty;
      }
    }
    __threadfence_block();
    __syncthreads();
  }
  if (!(a.temperature > 0.0f)) {  // greedy: argmax, no draw (src/sampler.cpp:25)
    const int r = block_argmax(work, V, s_val, s_idx);
    if (threadIdx.x == 0) a.out[b] = r;
    return;
  }
  for (int i = threadIdx.x; i < V; i += blockDim.x) work[i] = __fdiv_rn(work[i], a.temperature);
  __threadfence_block();
  __syncthreads();
  }

  int keep = V;
  const uint64_t* sorted = nullptr;
  if (topk) {
    if (threadIdx.x == 0) s_cnt = 0;
    __syncthreads();
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    // Candidates by a floor (k <= 64, logits in registers), on the keys' high halves (order bits):
    // each wave records its m largest lane maxima (m >= k / waves; one more than that, at most 4,
    // for a closer floor), every round removing the lanes that hold the recorded maximum, and the
    // floor is the k-th largest of the kWaves * m records.  Each record >= floor stands for a lane
    // of its own whose largest key has order bits >= floor, so at least k keys do, and the k largest
    // keys are all among them (a floor of 0 takes every key).  Those keys (for spread logits about
    // k + k / 8) are gathered and sorted; the first k are the kept set, the same keys the radix
    // select below finds.  Empty lanes have maximum 0.
    int n_keys = -1;  // keys gathered in s_keys, or -1 when the radix select runs
    const int m_min = (a.top_k + kWaves - 1) / kWaves, m = min(kFloorMaxRank, m_min + 1);
    if (reg && m_min <= kFloorMaxRank) {
      uint32_t cur = 0;
#pragma unroll
      for (int j = 0; j < kRegSlots; ++j)
        if (static_cast<int>(threadIdx.x) + kThreads * j < V) cur = max(cur, ov(j));
      for (int r = 0; r < m; ++r) {
        const uint32_t wm = wave_max_u32_dpp(cur);
        if (lane == 0) s_floor[wave * kFloorMaxRank + r] = wm;
        if (cur == wm) cur = 0;
      }
      if (lane == 0)
        for (int r = m; r < kFloorMaxRank; ++r) s_floor[wave * kFloorMaxRank + r] = 0u;  // rank below every record
      __syncthreads();
      if (wave == 0) {  // the k-th largest record: rank by (value, then position)
        static_assert(kWaves * kFloorMaxRank == kWave, "one record per lane");
        const uint32_t v = s_floor[lane];
        int rank = 0;
#pragma unroll
        for (int j = 0; j < kWave; ++j) {
          const uint32_t u = s_floor[j];
          rank += (u > v || (u == v && j < lane)) ? 1 : 0;
        }
        if (rank == a.top_k - 1) s_floor_bits = v;
      }
      __syncthreads();
      const uint32_t floor_bits = s_floor_bits;
#pragma unroll
      for (int j = 0; j < kRegSlots; ++j) {
        const int id = threadIdx.x + kThreads * j;
        if (id < V && ov(j) >= floor_bits) {
          const int pos = atomicAdd(&s_cnt, 1);
          if (pos < kMaxGathered)
            s_keys[pos] = (static_cast<uint64_t>(ov(j)) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - id);
        }
      }
      __syncthreads();
      n_keys = s_cnt;
      __syncthreads();
      if (n_keys > kMaxGathered) {  // more than one sort in LDS takes: the radix select instead
        n_keys = -1;
        if (threadIdx.x == 0) s_cnt = 0;
        __syncthreads();
      }
    }
    if (n_keys < 0) {
    radix_select(a.top_k, for_each_key, s_sel);
    const uint64_t prefix = s_sel.prefix, mask = s_sel.mask;
    for_each_key([&](uint64_t k) {
      if ((k & mask) >= prefix) {
        const int pos = atomicAdd(&s_cnt, 1);
        if (pos < kChunk) s_keys[pos] = k;
      }
    });
    __syncthreads();
    n_keys = a.top_k;
    }
    int n2 = 1;
    while (n2 < n_keys) n2 <<= 1;
    for (int i = n_keys + threadIdx.x; i < n2; i += blockDim.x) s_keys[i] = 0ull;
    __syncthreads();
    if (n2 <= kWave) {
      bitonic_wave(s_keys, n2);
    } else {
      bitonic_lds(s_keys, n2);
    }
    keep = a.top_k;
    sorted = s_keys;
  } else {
    if (a.top_k > 0 && a.top_k < V) keep = a.top_k;  // k above the LDS path: full sort, keep k
    for (int i = threadIdx.x; i < a.npow2; i += blockDim.x) keys[i] = i < V ? make_key(work[i], i) : 0ull;
    if (a.phase == 1) return;  // chunk_sort_kernel, rank_merge_kernel and sample_tail_kernel follow
    __threadfence_block();
    __syncthreads();
    bitonic_global(keys, a.npow2, s_keys);
    sorted = keys;
  }
  static_assert(sizeof(s_keys) >= 2 * kStage * sizeof(double), "staging buffers");
  sample_tail(a, b, sorted, keep, topk, prob, s_prob, reinterpret_cast<double*>(s_keys), s_stop, s_sum, s_keep,
              s_exp);
}

// ---- the full sort across workgroups (no top-k, large vocabularies) ---------------------------------
// Workspace of one sequence: work [V] floats, prob [V] doubles, keys [npow2], merged [npow2].
__device__ __forceinline__ uint64_t* keys_of(const SampleArgs& a, int b) {
  uint8_t* ws = a.ws + static_cast<size_t>(b) * a.ws_stride;
  return reinterpret_cast<uint64_t*>(ws + ((a.vocab * 4 + 255) & ~255) + prob_region_bytes(a.vocab));
}
__device__ __forceinline__ double* prob_of(const SampleArgs& a, int b) {
  return reinterpret_cast<double*>(a.ws + static_cast<size_t>(b) * a.ws_stride + ((a.vocab * 4 + 255) & ~255));
}
__device__ __forceinline__ uint64_t* merged_of(const SampleArgs& a, int b) {
  return keys_of(a, b) + ((static_cast<size_t>(a.npow2) * 8 + 255) & ~size_t{255}) / 8;
}

// The last 256 bytes of a sequence's workspace: nucleus_kernel's verdict, 1 when the sequence still
// needs the full sort (written on every call before the full-sort launches read it).
__device__ __forceinline__ int32_t* full_sort_flag(const SampleArgs& a, int b) {
  return reinterpret_cast<int32_t*>(a.ws + static_cast<size_t>(b) * a.ws_stride + a.ws_stride - 256);
}
__device__ __forceinline__ bool skip_full(const SampleArgs& a, int b) { return a.fast && *full_sort_flag(a, b) == 0; }

// Each kChunk-key run of the keys sorted in place (descending), one workgroup per run.
__global__ __launch_bounds__(kThreads) void chunk_sort_kernel(SampleArgs a) {
  __shared__ uint64_t s_keys[2 * kChunk];
  bitonic_global(keys_of(a, blockIdx.y) + static_cast<size_t>(blockIdx.x) * kChunk, kChunk, s_keys);
}

// The same runs with their keys formed here (no key-writing launch before): workgroup r takes ids
// kChunk r .. kChunk r + kChunk - 1, applies the repetition penalty to those of them in the history
// (each once) and the temperature, exactly as sample_kernel does (src/sampler.cpp:16-27), forms
// the keys in registers (ids past the vocabulary get key 0, below every key), sorts them and
// stores the run.
__global__ __launch_bounds__(kThreads) void key_sort_kernel(SampleArgs a) {
  __shared__ uint64_t s_keys[2 * kChunk];
  __shared__ uint32_t s_seen[kChunk / 32];
  const int b = blockIdx.y, t = threadIdx.x, base = blockIdx.x * kChunk, V = a.vocab;
  if (skip_full(a, b)) return;
  const float* lg = a.logits + b * a.ld;
  float v[kKeysPerThread];
#pragma unroll
  for (int u = 0; u < kKeysPerThread; ++u) {
    const int id = base + t + kThreads * u;
    v[u] = id < V ? lg[id] : 0.0f;
  }
  if (a.penalty != 1.0f) {
    for (int i = t; i < kChunk / 32; i += kThreads) s_seen[i] = 0u;
    __syncthreads();
    const int n = a.hist_len[b];
    const int32_t* h = a.hist + b * a.hist_ld;
    for (int i = t; i < n; i += kThreads) {
      const int id = h[i] - base;
      if (h[i] >= 0 && h[i] < V && id >= 0 && id < kChunk) atomicOr(&s_seen[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kKeysPerThread; ++u) {
      const int id = t + kThreads * u;
      if (base + id < V && (s_seen[id >> 5] >> (id & 31) & 1u))
        v[u] = v[u] > 0.0f ? __fdiv_rn(v[u], a.penalty) : v[u] * a.penalty;
    }
  }
  uint64_t x[kKeysPerThread];
#pragma unroll
  for (int u = 0; u < kKeysPerThread; ++u) {
    const int id = base + t + kThreads * u;
    x[u] = id < V ? make_key(__fdiv_rn(v[u], a.temperature), static_cast<uint32_t>(id)) : 0ull;
  }
  int parity = 0;
  for (int k = 2; k <= kChunk; k <<= 1) chunk_steps(x, 0, k, k >> 1, s_keys, parity);
  uint64_t* g = keys_of(a, b) + base;
#pragma unroll
  for (int u = 0; u < kKeysPerThread; ++u) g[t + kThreads * u] = x[u];
}

// The sorted runs merged in one pass: key i of run r goes to i + (keys of every run r' < r that are
// >= it) + (keys of every run r' > r that are > it): the runs' ties resolve by run index, so the
// positions are a permutation and the result is the descending order.  A workgroup's 256 keys are
// consecutive in one run, so in every other run the keys that fall between its first and its last
// key form one window: two binary searches in global memory per run bound it, the windows are
// copied to LDS with coalesced loads, and each key counts its place inside them in LDS.  A window
// that does not fit is searched in global memory as a whole.
constexpr int kMergeThreads = 256;
constexpr int kMergeWindow = 3072;  // keys of all windows held in LDS (24 KB; typically 7 x ~256 are used)
constexpr int kMaxRuns = 64;        // runs of kChunk keys: vocabularies up to 262144

__global__ __launch_bounds__(kMergeThreads) void rank_merge_kernel(SampleArgs a) {
  __shared__ uint64_t s_win[kMergeWindow];
  __shared__ int s_lo[kMaxRuns], s_hi[kMaxRuns], s_off[kMaxRuns];
  if (skip_full(a, blockIdx.y)) return;
  const uint64_t* keys = keys_of(a, blockIdx.y);
  uint64_t* out = merged_of(a, blockIdx.y);
  const int t = threadIdx.x, e0 = blockIdx.x * kMergeThreads, e = e0 + t;
  const int runs = a.npow2 / kChunk, r = e0 / kChunk;
  // keys before a key y in run q: q < r counts keys >= y, q > r keys > y (descending runs)
  auto count_before = [&](const uint64_t* run, int q, uint64_t y) {
    int lo = 0, hi = kChunk;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const bool before = q < r ? run[mid] >= y : run[mid] > y;
      if (before) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  const bool windows = runs <= kMaxRuns;  // more runs: every search in global memory
  if (windows && t < runs && t != r) {  // run t's window: the counts of the slice's largest and smallest key
    const uint64_t* run = keys + static_cast<size_t>(t) * kChunk;
    s_lo[t] = count_before(run, t, keys[e0]);
    s_hi[t] = count_before(run, t, keys[e0 + kMergeThreads - 1]);
  }
  __syncthreads();
  if (windows && t == 0) {  // LDS offsets of the windows that fit, in run order; -1: global search
    int off = 0;
    for (int q = 0; q < runs; ++q) {
      s_off[q] = -1;
      if (q == r) continue;
      const int w = s_hi[q] - s_lo[q];
      if (off + w <= kMergeWindow) {
        s_off[q] = off;
        off += w;
      }
    }
  }
  __syncthreads();
  if (windows) {
    for (int q = 0; q < runs; ++q) {
      if (q == r || s_off[q] < 0) continue;
      const uint64_t* run = keys + static_cast<size_t>(q) * kChunk + s_lo[q];
      uint64_t* w = s_win + s_off[q];
      for (int i = t; i < s_hi[q] - s_lo[q]; i += kMergeThreads) w[i] = run[i];
    }
  }
  __syncthreads();
  const uint64_t x = keys[e];
  int pos = e - r * kChunk;
  for (int q = 0; q < runs; ++q) {
    if (q == r) continue;
    if (!windows || s_off[q] < 0) {
      pos += count_before(keys + static_cast<size_t>(q) * kChunk, q, x);
      continue;
    }
    const uint64_t* w = s_win + s_off[q];
    int lo = 0, hi = s_hi[q] - s_lo[q];
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const bool before = q < r ? w[mid] >= x : w[mid] > x;
      if (before) lo = mid + 1;
      else hi = mid;
    }
    pos += s_lo[q] + lo;
  }
  out[pos] = x;
  // the softmax term of the key at its sorted position, exp(double(v - max)) as the reference
  // forms it (src/sampler.cpp:44-47; the maximum is the largest run head), laid out for
  // sample_scan_kernel: with C = ceil(V / kScanPer) columns, the term of position j goes to
  // (j % kScanPer) * C + j / kScanPer, so that thread t's contiguous terms j = kScanPer t + i are
  // read with term i of every thread adjacent (coalesced)
  if (pos < a.vocab) {
    uint64_t top = keys[0];
    for (int q = 1; q < runs; ++q) {
      const uint64_t h = keys[static_cast<size_t>(q) * kChunk];
      top = h > top ? h : top;
    }
    const int cols = (a.vocab + kScanPer - 1) / kScanPer;
    prob_of(a, blockIdx.y)[(pos % kScanPer) * cols + pos / kScanPer] =
        exp_libm(static_cast<double>(key_value(x) - key_value(top)));
  }
}

// ---- the reference's left-to-right double sums, in parallel and bit for bit -----------------------------
// s_j = RN(s_{j-1} + t_j) from s_{-1} = 0.  While s stays in one binade [2^e, 2^(e+1)) it is a
// multiple of u = 2^(e-52), and a step adds t_j rounded to a multiple of u: s_j = s_{j-1} + k_j u,
// k_j = t_j / u rounded to the nearest integer, provided s_{j-1} + t_j < 2^(e+1) and t_j / u is
// not halfway between integers (a tie rounds to the even multiple, which depends on s_{j-1}).  The
// k_j do not depend on each other, so a round takes every remaining step at the current binade:
// the k_j, their prefix sums (integers below 2^53, exact in doubles), and the first step that
// leaves the binade or is a tie.  Every step before that one is exact; that one is a plain double
// add by the thread that holds its term, and the next round starts after it in its binade.  A sum
// that passes through b binades takes about b + 1 rounds (the one-term start from 0 included).

// The first kScanHead terms are added one by one (thread 0, from LDS) before the rounds: a sum
// crosses most of its binades within its largest terms, where each crossing would cost a round.
constexpr int kScanHead = 256;

struct ScanShared {
  double head[kScanHead];
  double s, hit_sum;  // running sum before element j0; the running sum at the hit
  int j0, hit, done;
  double wsum[kThreads / kWave];
  int wbad[kThreads / kWave], whit[kThreads / kWave];
};

// Wave-wide unsigned minimum through DPP, on every lane.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_self_min(uint32_t v) {
  return min(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL,
                                                                   ROW_MASK, 0xF, false)));
}
__device__ __forceinline__ int wave_min_dpp(int v) {  // v >= 0
  uint32_t u = static_cast<uint32_t>(v);
  u = dpp_self_min<0xB1>(u);
  u = dpp_self_min<0x4E>(u);
  u = dpp_self_min<0x141>(u);
  u = dpp_self_min<0x140>(u);
  u = dpp_self_min<0x142, 0xA>(u);
  u = dpp_self_min<0x143, 0xC>(u);
  return __builtin_amdgcn_readlane(static_cast<int>(u), 63);
}

// A double moved by a DPP control; lanes without a source (or outside row_mask) read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_zero_d(double v) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b)), CTRL, ROW_MASK, 0xF, true));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b >> 32)), CTRL, ROW_MASK, 0xF, true));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Exclusive prefix sum over the wave's lanes (lane 0 gets 0): the lanes shifted by one, then an
// inclusive scan by DPP row shifts and row broadcasts.  A lane's prefix adds only lanes below it.
__device__ __forceinline__ double wave_excl_scan_dpp(double v) {
  double x = dpp_zero_d<0x138>(v);  // wave_shr:1
  x += dpp_zero_d<0x111>(x);        // row_shr:1
  x += dpp_zero_d<0x112>(x);        // row_shr:2
  x += dpp_zero_d<0x114>(x);        // row_shr:4
  x += dpp_zero_d<0x118>(x);        // row_shr:8
  x += dpp_zero_d<0x142, 0xA>(x);   // row_bcast:15 into rows 1 and 3
  x += dpp_zero_d<0x143, 0xC>(x);   // row_bcast:31 into rows 2 and 3
  return x;
}

__device__ __forceinline__ int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ double uniform_d(double v) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// MODE 0: the sum of t_0 .. t_{n-1}; 1: the first j with s_j >= x; 2: the first j with x < s_j.
// Returns that j (n when no step satisfies the predicate) on every thread and sets *sum to s_j
// (to the whole sum when none does).  Every term must be finite and >= 0.
// Control flow: every decision of a round is taken on values read from LDS and made wave-uniform
// (readfirstlane), with no early continue, so the loop stays one uniform loop and the step's owner
// runs its step inside the round.  (With the decisions left per lane, the compiler built the round
// as an inner loop that only the owner lane left, so the owner's wave never reached the step and
// the other lanes repeated the round.)  A round either ends the scan or takes one step, so n + 1
// rounds suffice; the bound makes every wave's exit certain.
template <int MODE, int PER = kScanPer, int HEAD = kScanHead>
__device__ int exact_scan(const double (&t)[PER], int n, double x, ScanShared& sh, double* sum, double init = 0.0) {
  static_assert(HEAD <= kScanHead, "scan head");
  // wave in a scalar register: a per-lane copy (the LDS addresses of the wave totals) was spilled
  // and reloaded inside every round
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid & (kWave - 1),
            base = tid * PER;
  constexpr int kW = kThreads / kWave;
  auto pred = [&](double s) { return MODE == 1 ? s >= x : (MODE == 2 ? x < s : false); };
  const int nh = min(n, HEAD);
  if (base < nh) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (base + i < nh) sh.head[base + i] = t[i];
  }
  __syncthreads();
  if (tid == 0) {  // the head, term by term as the reference adds them
    // groups of eight: the next group's LDS reads issued before this group's chain of adds, the
    // running sums read off the chain for the predicate (terms past the head are exact zeros,
    // which leave a nonnegative sum unchanged)
    double s = init, hs = 0.0;
    int hit = n;
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = u < nh ? sh.head[u] : 0.0;
    for (int j = 0; j < nh; j += 8) {
      double w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = j + 8 + u < nh ? sh.head[j + 8 + u] : 0.0;
      double c[8], x = s;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        x = x + v[u];
        c[u] = x;
      }
      if (MODE != 0) {
        int h = -1;
#pragma unroll
        for (int u = 7; u >= 0; --u)
          if (j + u < nh && pred(c[u])) h = u;
        if (h >= 0) {
          hit = j + h;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (u == h) hs = c[u];
          break;
        }
      }
      s = x;
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = w[u];
    }
    sh.s = s;
    sh.hit_sum = hs;
    sh.hit = hit;
    sh.j0 = nh;
    sh.done = hit < n || nh >= n;
  }
  for (int round = 0; round <= n + 1; ++round) {
    __syncthreads();
    const double s = uniform_d(sh.s);
    const int j0 = uniform_i(sh.j0), done = uniform_i(sh.done);
    __syncthreads();  // read before any thread rewrites the state
    if (done) break;
    int jb = j0, jh = n;  // the step taken as a plain add this round; the first hit
    double sp = s;        // the running sum before step jb (on its owner)
    const bool usable = s >= 0x1p-1000;  // s = m 2^ex, m in [0.5, 1): u = 2^(ex - 53), s / u = s 2^sc
    if (usable) {
      int ex;
      (void)frexp(s, &ex);
      const int sc = 53 - ex;
      const double M0 = ldexp(s, sc);
      const bool mine = base + PER > j0 && base < n;
      double T = 0.0;
      uint32_t tie_u = 0;
      if (mine) {
        // branch-free (a select per term, the tie as an integer): per-term branches cost scalar
        // exec-mask instructions, and the CU's one scalar unit serves all sixteen waves
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int j = base + i;
          const uint32_t in = static_cast<uint32_t>(j - j0) < static_cast<uint32_t>(n - j0) ? 1u : 0u;
          const double y = ldexp(t[i], sc), k = rint(y);
          T += in ? k : 0.0;
          tie_u |= in & (fabs(y - k) == 0.5 ? 1u : 0u);
        }
      }
      const bool tie = tie_u != 0;
      // exclusive prefix of the thread totals: lanes below this one, then the waves below (a
      // thread after the first inexact step may hold huge totals; they never enter the prefix of
      // a thread before it)
      double K = wave_excl_scan_dpp(T);
      if (lane == kWave - 1) sh.wsum[wave] = K + T;
      __syncthreads();
      for (int w = 0; w < wave; ++w) K += sh.wsum[w];
      // Only a thread that may hold the first inexact step or the first hit walks its terms.  A
      // step that leaves the binade without a tie has s_{j-1} / u + k_j >= 2^53 (its k_j rounds
      // t_j / u up past the boundary or t_j already reaches it), so a tie-free thread whose last
      // running sum is below 2^(e+1) has only exact steps; the running sums rise, so the last one
      // decides whether any step of the thread meets the predicate.
      int my_bad = n, my_hit = n;
      double my_hs = 0.0, Kb = 0.0;
      const double M_end = M0 + K + T;
      const bool walk = mine && (tie || !(M_end < 0x1p53) || (MODE != 0 && pred(ldexp(M_end, -sc))));
      if (walk) {
        bool stop = false;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int j = base + i;
          if (!stop && j >= j0 && j < n) {
            const double y = ldexp(t[i], sc), k = rint(y), Mp = M0 + K;  // s_{j-1} / u, exact
            if (fabs(y - k) == 0.5 || !(y < 0x1p53 - Mp)) {
              my_bad = j;
              Kb = Mp;
              stop = true;
            } else {
              K += k;
              if (MODE != 0) {
                const double sj = ldexp(M0 + K, -sc);
                if (pred(sj)) {
                  my_hit = j;
                  my_hs = sj;
                  stop = true;
                }
              }
            }
          }
        }
      }
      const int wb = wave_min_dpp(my_bad), wh = wave_min_dpp(my_hit);
      if (lane == 0) {
        sh.wbad[wave] = wb;
        sh.whit[wave] = wh;
      }
      __syncthreads();
      int b2 = n, h2 = n;
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        b2 = min(b2, sh.wbad[w]);
        h2 = min(h2, sh.whit[w]);
      }
      jb = uniform_i(b2);
      jh = uniform_i(h2);
      if (jh < jb) {  // a hit before any inexact step
        if (my_hit == jh) {
          sh.hit = jh;
          sh.hit_sum = my_hs;
          sh.done = 1;
        }
      } else if (jb >= n) {  // every remaining step exact: the total
        if (tid == 0) {
          double tot = 0.0;
          for (int w = 0; w < kW; ++w) tot += sh.wsum[w];
          sh.s = ldexp(M0 + tot, -sc);
          sh.done = 1;
        }
      } else {
        sp = ldexp(Kb, -sc);  // meaningful on the owner of jb only
      }
    }
    const bool take = !usable || (jh >= jb && jb < n);  // wave-uniform
    if (take && jb / PER == tid) {  // the step at jb as the reference takes it
      double tj = 0.0;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (base + i == jb) tj = t[i];
      const double sn = sp + tj;
      if (MODE != 0 && pred(sn)) {
        sh.hit = jb;
        sh.hit_sum = sn;
        sh.done = 1;
      } else {
        sh.s = sn;
        sh.j0 = jb + 1;
        sh.done = jb + 1 >= n;
      }
    }
  }
  __syncthreads();
  const int hit = sh.hit;
  *sum = hit < n ? sh.hit_sum : sh.s;
  __syncthreads();  // sh is reused by the next scan
  return hit;
}

// sample_tail with the kept terms in registers (keep <= kThreads * kScanPer) and every sequential
// loop an exact_scan: the same sums, cut and pick as the reference's loops (src/sampler.cpp:42-69).
// A term that is not finite is a NaN (a NaN logit, or +inf minus the +inf maximum): the reference's
// sum is then NaN, so are all its probabilities, no comparison holds, and the pick is the last
// kept id after one draw, which is what this returns.
__device__ void sample_tail_scan(const SampleArgs& a, int b, const uint64_t* sorted, int keep, ScanShared& sh,
                                 int& s_flag) {
  const int tid = threadIdx.x, base = tid * kScanPer;
  const double* p = prob_of(a, b);  // the sorted softmax terms, written by rank_merge_kernel
  const int cols = (a.vocab + kScanPer - 1) / kScanPer;
  double t[kScanPer];
  bool finite = true;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    const int j = base + i;
    t[i] = j < keep ? p[i * cols + tid] : 0.0;
    finite = finite && isfinite(t[i]);
  }
  if (tid == 0) s_flag = 0;
  __syncthreads();
  if (!finite) s_flag = 1;
  __syncthreads();
  if (s_flag) {
    if (tid == 0) {
      (void)mt_uniform(reinterpret_cast<MtState*>(a.rng + static_cast<size_t>(b) * kRngStateBytes));
      a.out[b] = static_cast<int>(key_id(sorted[keep - 1]));
    }
    return;
  }
  double sum;
  exact_scan<0>(t, keep, 0.0, sh, &sum);
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) t[i] = t[i] / sum;
  int kp = keep;
  if (a.top_p < 1.0f) {  // nucleus: the first n with cum >= top_p; s2 is cum there (or the whole sum)
    double cum;
    const int n = exact_scan<1>(t, keep, static_cast<double>(a.top_p), sh, &cum);
    kp = max(n < keep ? n + 1 : keep, 1);
#pragma unroll
    for (int i = 0; i < kScanPer; ++i) t[i] = t[i] / cum;
  }
  if (tid == 0) {
    MtState* st = reinterpret_cast<MtState*>(a.rng + static_cast<size_t>(b) * kRngStateBytes);
    sh.hit_sum = mt_uniform(st);
  }
  __syncthreads();
  const double r = sh.hit_sum;
  __syncthreads();
  double cum;
  const int i = exact_scan<2>(t, kp, r, sh, &cum);
  if (tid == 0) a.out[b] = static_cast<int>(key_id(sorted[i < kp ? i : kp - 1]));
}

// ---- top-p without top-k: the nucleus from the head of the order --------------------------------------
// The reference sorts the whole vocabulary (src/sampler.cpp:36-38), adds every softmax term in that
// order (:42-48), cuts the nucleus (:50-61) and walks it (:62-69).  When the nucleus ends within the
// head of the order only the head needs its order: one workgroup per sequence takes the keys within
// a bucket bound of the maximum (at most kTopM), sorts them in LDS and takes the head's sum, the cut
// and the walk with exact_scan.  The other terms (the tail) join the sum by exact_scan's binade
// argument, which needs no order: while the running sum s stays in [2^e, 2^(e+1)) a step adds
// rint(t / u) u, u = 2^(e-52), unless t / u is halfway between integers (a tie, rounded by the
// parity of s).  So the tail adds K u, K = the sum of rint(t / u) over it, when s / u + K < 2^53 and
// no tail term is a tie.  When the sum leaves its binade in the tail, the next buckets (at most
// kTopM keys) are sorted and added in order after the head's sum, and the rest is checked
// again.  A sum that still leaves its binade, a tie, a term that is not finite, or a nucleus that
// reaches past the head leaves the sequence to the full sort (the flag in its workspace), whose
// launches follow and return at once for every other sequence.
constexpr int kTopM = kChunk;              // the sorted head: one register chunk sort
constexpr int kTopPer = kTopM / kThreads;  // head terms per thread in the scans (contiguous)

// The logit whose order bits are u (the high half of a key).
__device__ __forceinline__ float ob_value(uint32_t u) { return key_value(static_cast<uint64_t>(u) << 32); }

// Bitonic sort of 4096 keys, descending, thread t holding positions 4t .. 4t + 3 in x: partners at
// distance 1 and 2 are in the thread, 4 .. 128 in the wave (a shuffle), 256 .. 2048 in other waves
// (one LDS exchange, double-buffered in buf's 2 x 4096 keys, one barrier).  Every thread calls it.
__device__ void sort4096_desc(uint64_t (&x)[4], uint64_t* buf) {
  static_assert(kThreads * 4 == 4096, "four keys per thread");
  const int t = threadIdx.x;
  int parity = 0;
  for (int k = 2; k <= 4096; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint64_t y[4];
      if (j >= 4 * kWave) {  // position 4t + u at u * kThreads + t: each access lane-contiguous
        uint64_t* bb = buf + parity * 4096;
#pragma unroll
        for (int u = 0; u < 4; ++u) bb[u * kThreads + t] = x[u];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u) y[u] = bb[u * kThreads + (t ^ (j >> 2))];
        parity ^= 1;  // the next exchange writes the other buffer, so no second barrier is needed
      } else if (j >= 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) y[u] = shfl_xor_u64(x[u], j >> 2);
      } else if (j == 2) {
        y[0] = x[2];
        y[1] = x[3];
        y[2] = x[0];
        y[3] = x[1];
      } else {
        y[0] = x[1];
        y[1] = x[0];
        y[2] = x[3];
        y[3] = x[2];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = 4 * t + u;
        const bool take_max = ((i & k) == 0) == ((i & j) == 0);  // descending: the lower index keeps the larger
        x[u] = (x[u] > y[u]) == take_max ? x[u] : y[u];
      }
    }
  }
}

// Block-wide sum (every thread gets it, added in a fixed order); red: one double per wave.
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = wave_sum_d(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  double s = 0.0;
  for (int w = 0; w < kThreads / kWave; ++w) s += red[w];
  __syncthreads();
  return uniform_d(s);
}
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const uint64_t u = shfl_xor_u64(v, o);
    v = u > v ? u : v;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  uint64_t m = 0;
  for (int w = 0; w < kThreads / kWave; ++w) m = red[w] > m ? red[w] : m;
  __syncthreads();
  return m;
}


// The keys of the slots whose bit is set in `in` (slot j of thread t: id t + kThreads j, order bits
// ob[j]) sorted descending into keys[0, n), keys[n, kTopM) zeros (below every key); keys[0, 2 kTopM)
// is the working space.  Returns n; more than kTopM keys sort nothing.  The keys are first gathered
// into keys[0, n) (in wave, slot and lane order), then each thread takes four of them: a bucket
// sort by fine bins of the logit, floor(256 (max - v)) (monotone in v, so bin order is key order),
// counted, their exclusive prefix giving each bin's place, the keys scattered to their bins, and
// each key's place inside its bin counted among the bin's keys.  A bin of more than kFineMax keys
// (many equal or nearly equal logits) takes the bitonic sort instead.  s_bin, s_start: kFineBins
// and kFineBins + 1 + kThreads / kWave words of LDS; s_cnt: one int per wave.  Every thread calls it.
constexpr int kFineBins = 4096;  // covers max - v < 16, past every head bucket
constexpr int kFineMax = 256;

__device__ __forceinline__ int gather_sort(uint32_t (&ob)[kRegSlots], uint32_t in, float mx, uint64_t* keys,
                                           uint32_t* s_bin, uint32_t* s_start, int* s_cnt) {
  static_assert(kFineBins == 4 * kThreads && kTopM == 4 * kThreads, "four bins and four keys per thread");
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid & (kWave - 1);
  auto fine = [&](float v) {
    const float d = (mx - v) * 256.0f;
    return d < static_cast<float>(kFineBins - 1) ? static_cast<int>(d) : kFineBins - 1;
  };
  auto key_at = [&](int j) {
    return (static_cast<uint64_t>(ob[j]) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - (tid + kThreads * j));
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) s_bin[4 * tid + i] = 0u;
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) cnt += __popcll(__ballot(in >> j & 1u));
  if (lane == 0) s_cnt[wave] = cnt;
  __syncthreads();
  int n = 0, pos = 0;
  for (int w = 0; w < kThreads / kWave; ++w) {
    pos += w < wave ? s_cnt[w] : 0;
    n += s_cnt[w];
  }
  if (n > kTopM) {
    __syncthreads();  // s_cnt is reused by the caller
    return n;
  }
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) {
    const bool take = in >> j & 1u;
    const uint64_t m = __ballot(take);
    const int r = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
    if (take) keys[pos + r] = key_at(j);
    pos += __popcll(m);
  }
  for (int i = n + tid; i < kTopM; i += kThreads) keys[i] = 0ull;
  __syncthreads();  // also: every wave has read s_cnt
  uint64_t x[4];  // positions 4t .. 4t + 3
#pragma unroll
  for (int u = 0; u < 4; ++u) x[u] = keys[4 * tid + u];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (4 * tid + u < n) atomicAdd(&s_bin[fine(key_value(x[u]))], 1u);
  __syncthreads();
  // each bin's place: an exclusive prefix over the bins (four per thread, a wave per 256 bins, then
  // the waves in order), and the largest bin
  uint32_t c[4], tot = 0, cmax = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = s_bin[4 * tid + i];
    tot += c[i];
    cmax = max(cmax, c[i]);
  }
  uint32_t inc = tot;
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t v = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += v;
  }
  const uint32_t wmax = wave_max_u32_dpp(cmax);
  if (lane == kWave - 1) s_cnt[wave] = static_cast<int>(inc);
  if (lane == 0) s_start[kFineBins + 1 + wave] = wmax;  // scratch past the prefix: the waves' largest bins
  __syncthreads();
  uint32_t below = 0, big = 0;
  for (int w = 0; w < kThreads / kWave; ++w) {
    below += w < wave ? static_cast<uint32_t>(s_cnt[w]) : 0u;
    big = max(big, s_start[kFineBins + 1 + w]);
  }
  uint32_t st = below + inc - tot;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s_start[4 * tid + i] = st;
    s_bin[4 * tid + i] = st;  // the scatter's cursor
    st += c[i];
  }
  if (tid == 0) s_start[kFineBins] = static_cast<uint32_t>(n);
  __syncthreads();
  if (big > kFineMax) {  // the bitonic sort of the gathered keys (zeros after them)
    sort4096_desc(x, keys);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) keys[4 * tid + u] = x[u];
    __syncthreads();
    return n;
  }
  uint64_t* scat = keys + kTopM;  // the keys grouped by bin
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (4 * tid + u < n) scat[atomicAdd(&s_bin[fine(key_value(x[u]))], 1u)] = x[u];
  __syncthreads();
  for (int p = tid; p < n; p += kThreads) {  // consecutive threads on one bin: similar loop lengths
    const uint64_t k = scat[p];
    const int fb = fine(key_value(k));
    const int b0 = static_cast<int>(s_start[fb]), b1 = static_cast<int>(s_start[fb + 1]);
    int r = 0;
    for (int q = b0; q < b1; ++q) r += scat[q] > k ? 1 : 0;
    keys[b0 + r] = k;
  }
  __syncthreads();
  return n;
}

// The nucleus cut, its renormalisation, the draw and the walk (src/sampler.cpp:49-69) over the
// sorted head keys[0, M) with S the whole softmax sum; a cut past the head sets the flag for the
// full sort (no draw).  Thread t holds head terms kTopPer t .. kTopPer t + kTopPer - 1.
__device__ __forceinline__ void nucleus_finish(const SampleArgs& a, int b, const uint64_t* keys, int M, float mx, double S,
                               const uint64_t* etab, ScanShared& sh, int32_t* flag) {
  const int tid = threadIdx.x;
  double tm[kTopPer];
#pragma unroll
  for (int i = 0; i < kTopPer; ++i) {
    const int p = kTopPer * tid + i;
    tm[i] = p < M ? exp_libm(static_cast<double>(key_value(keys[p]) - mx), etab) / S : 0.0;
  }
  double cum;
  const int n = exact_scan<1, kTopPer, 32>(tm, M, static_cast<double>(a.top_p), sh, &cum);
  if (n >= M) {  // the nucleus reaches past the head
    if (tid == 0) *flag = 1;
    return;
  }
  const int kp = n + 1;
#pragma unroll
  for (int i = 0; i < kTopPer; ++i) tm[i] = tm[i] / cum;
  if (tid == 0) {
    MtState* st = reinterpret_cast<MtState*>(a.rng + static_cast<size_t>(b) * kRngStateBytes);
    sh.hit_sum = mt_uniform(st);
  }
  __syncthreads();
  const double r = sh.hit_sum;
  __syncthreads();
  double c2;
  const int i = exact_scan<2, kTopPer, 32>(tm, kp, r, sh, &c2);
  if (tid == 0) {
    a.out[b] = static_cast<int>(key_id(keys[i < kp ? i : kp - 1]));
    *flag = 0;
  }
}

__global__ __launch_bounds__(kThreads) void nucleus_kernel(SampleArgs a) {
  constexpr int kWaves = kThreads / kWave;
  __shared__ uint64_t s_keys[2 * kChunk];  // the head's keys, and the sort's exchange buffers
  __shared__ ScanShared sh;
  __shared__ uint32_t s_wmax[kWaves], s_bh[kWaves * 64];
  __shared__ int s_n[16];
  __shared__ uint32_t s_seen[kFineBins];  // the history marks (one word per thread), then the fine bins
  __shared__ uint32_t s_start[kFineBins + 1 + kWaves];
  __shared__ uint64_t s_exp[256];
  __shared__ double s_red[kWaves];
  __shared__ uint64_t s_redk[kWaves];
  __shared__ int s_bad;
  const int b = blockIdx.x, V = a.vocab, tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave),
            lane = tid & (kWave - 1);
  int32_t* flag = full_sort_flag(a, b);
  stage_exp_table(s_exp);
  __syncthreads();
  if (a.eos_p != nullptr) {
    const double pe = softmax_prob(a.logits + b * a.ld, V, a.eos_id, s_red, s_exp);
    if (tid == 0) a.eos_p[b] = pe;
  }
  uint32_t ob[kRegSlots];  // the keys' high halves: order bits of the tempered logits
  {
    float rv[kRegSlots];
    load_tempered(a, b, rv, s_seen);
#pragma unroll
    for (int j = 0; j < kRegSlots; ++j) ob[j] = tid + kThreads * j < V ? order_bits(rv[j]) : 0u;
  }
  // the maximum (a NaN or infinite one: the full sort's rule)
  uint32_t om = 0;
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) om = max(om, ob[j]);
  om = wave_max_u32_dpp(om);
  if (lane == 0) s_wmax[wave] = om;
  __syncthreads();
  om = 0;
  for (int w = 0; w < kWaves; ++w) om = max(om, s_wmax[w]);
  const float mx = ob_value(om);
  if (!isfinite(mx)) {
    if (tid == 0) *flag = 1;
    return;
  }
  // The head: the keys whose logit is within some distance of the maximum, at most kTopM of them.
  // One pass buckets the keys by floor(4 (max - v)) (clamped to 63; monotone in v, so a bucket
  // bound is a logit bound and the head is a prefix of the sorted order), per-wave histograms of
  // buckets 0..62 (bucket 63 is never part of the head or of the bounds below); the bound kept is
  // the largest whose buckets hold at most kTopM keys.
  auto bucket_of = [&](uint32_t u) {
    const float d = (mx - ob_value(u)) * 4.0f;
    return d < 63.0f ? static_cast<int>(d) : 63;
  };
  auto bucket = [&](int j, float m) {
    const float d = (m - ob_value(ob[j])) * 4.0f;
    return d < 63.0f ? static_cast<int>(d) : 63;
  };
  // The least order bits u with bucket_of(u) <= bk (bk < 63), by one wave: bucket_of does not rise
  // with u (u = 0, a NaN, is in bucket 63 and the maximum's om in bucket 0), so the answer lies in
  // (lo, hi] and each round splits the range into 64 parts, one per lane.  So a key is in buckets
  // <= bk exactly when its order bits are at least the answer.
  auto bucket_threshold = [&](int bk) {
    uint64_t lo = 0, hi = om;
    while (hi - lo > 1) {
      const uint64_t step = (hi - lo + kWave - 1) / kWave;
      const uint64_t c = min(lo + static_cast<uint64_t>(lane + 1) * step, hi);
      const uint64_t ok = __ballot(bucket_of(static_cast<uint32_t>(c)) <= bk);  // lane 63 (c = hi) holds
      const int f = __builtin_ctzll(ok);
      const uint64_t below = __shfl(c, f > 0 ? f - 1 : 0, kWave);
      hi = __shfl(c, f, kWave);
      lo = f > 0 ? below : lo;
    }
    return static_cast<uint32_t>(hi);
  };
  for (int i2 = tid; i2 < kWaves * 64; i2 += kThreads) s_bh[i2] = 0u;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j) {  // bucket 63 (the rest, never in the head) is not counted:
    const int bk = bucket(j, mx);        // ids past V have order bits 0, a NaN, so they fall there
    if (bk < 63) atomicAdd(&s_bh[wave * 64 + bk], 1u);
  }
  __syncthreads();
  if (wave == 0) {  // bucket `lane`: its count, the inclusive prefix over buckets <= lane
    uint32_t c = 0;
    for (int w = 0; w < kWaves; ++w) c += s_bh[w * 64 + lane];
    uint32_t pre = c;
    for (int o = 1; o < kWave; o <<= 1) {
      const uint32_t v = __shfl_up(pre, o, kWave);
      if (lane >= o) pre += v;
    }
    const uint64_t fits = __ballot(lane < 63 && pre <= static_cast<uint32_t>(kTopM));
    const int bm = fits == 0 ? -1 : 63 - __builtin_clzll(fits);  // prefix counts rise with the bucket
    // A nucleus that certainly reaches past the head goes to the full sort now: bucket b's terms
    // lie in (e^-(b+1)/4, e^-b/4], so the head holds at most the first sum of the mass and the
    // vocabulary at least the second (bucket 63 counted as 0); a 2% margin covers the float
    // arithmetic of the bounds.
    const float hi = lane <= bm ? static_cast<float>(c) * expf(-0.25f * static_cast<float>(lane)) : 0.0f;
    const float lo = lane < 63 ? static_cast<float>(c) * expf(-0.25f * static_cast<float>(lane + 1)) : 0.0f;
    const float head_hi = wave_sum(hi), all_lo = wave_sum(lo);
    const uint32_t thr = bm >= 0 ? bucket_threshold(bm) : 0u;
    if (lane == 0) {
      s_n[0] = bm >= 0 && head_hi < 0.98f * a.top_p * all_lo ? -2 : bm;
      s_n[1] = static_cast<int>(thr);
    }
  }
  __syncthreads();
  const int bmax = s_n[0];  // the head: buckets <= bmax
  const uint32_t thr = static_cast<uint32_t>(s_n[1]);
  if (bmax < 0) {  // more than kTopM keys within a quarter of the maximum, or a nucleus past the head
    if (tid == 0) *flag = 1;
    return;
  }
  uint32_t inh = 0;  // bit j: slot j is in the head (ids past V have order bits 0, below thr)
#pragma unroll
  for (int j = 0; j < kRegSlots; ++j)
    if (ob[j] >= thr) inh |= 1u << j;
  // The tail: the slots not yet summed.  One pass over the registers: 1 when the rest stays in
  // the sum's binade with no tie (the sum is then final), 2 when it leaves the binade, 0 for a tie
  // or a NaN term (the full sort's rule).
  auto tail = [&](uint32_t done, double& sum) {
    int ex;
    (void)frexp(sum, &ex);
    const int sc = 53 - ex;  // sum / u = sum 2^sc, an integer in [2^52, 2^53)
    const double M0 = ldexp(sum, sc);
    double T = 0.0;
    uint64_t tie = 0;
#pragma unroll
    for (int j = 0; j < kRegSlots; ++j) {
      if (tid + kThreads * j < V && !(done >> j & 1u)) {
        const double y = ldexp(exp_libm(static_cast<double>(ob_value(ob[j]) - mx), s_exp), sc), r = rint(y);
        T += r;
        if (fabs(y - r) == 0.5) tie = 1;
      }
    }
    T = block_sum_d(T, s_red);
    tie = block_max_u64(tie, s_redk);
    if (!(T == T) || tie != 0) return 0;
    if (M0 + T < 0x1p53) {
      sum = ldexp(M0 + T, -sc);
      return 1;
    }
    return 2;
  };
  // Chunk 0 is the head: sorted, summed from 0, then the tail checked.  When the sum leaves its
  // binade after the head, chunk 1 (the next buckets, at most kTopM keys) is sorted and added
  // in order from the head's sum and the rest checked again; the
  // head's keys wait in the workspace meanwhile.  (One loop, not two copies: the second copy made
  // the kernel spill.)
  int M = 0, st = 0;
  double s = 0.0;
  uint32_t done = 0, mask = inh;
  uint64_t* hk = keys_of(a, b);
#pragma unroll 1
  for (int c = 0; c < 2; ++c) {
    // keys, bins and terms are formed again in each chunk (hoisted out of the loop, they spill)
#pragma unroll
    for (int j = 0; j < kRegSlots; ++j) asm volatile("" : "+v"(ob[j]));
    const int n = gather_sort(ob, mask, mx, s_keys, s_seen, s_start, s_n);
    if (c == 0) M = n;
    if (n > kTopM || (c == 0 && n == 0)) {  // cannot happen: the buckets were chosen to fit
      st = 0;
      break;
    }
    double tm[kTopPer];
    bool finite = true;
#pragma unroll
    for (int i = 0; i < kTopPer; ++i) {
      const int p = kTopPer * tid + i;
      tm[i] = p < n ? exp_libm(static_cast<double>(key_value(s_keys[p]) - mx), s_exp) : 0.0;
      finite = finite && isfinite(tm[i]);
    }
    if (tid == 0) s_bad = 0;
    __syncthreads();
    if (!finite) s_bad = 1;
    __syncthreads();
    if (uniform_i(s_bad)) {  // NaN terms: the full sort's rule
      st = 0;
      break;
    }
    exact_scan<0, kTopPer, 32>(tm, n, 0.0, sh, &s, s);  // chunk 1 continues from the head's sum
    done |= mask;
    st = tail(done, s);
    if (st != 2 || c == 1) break;
    if (wave == 0) {  // chunk 1: the buckets after the head's whose keys fit
      uint32_t cb = 0;
      for (int w = 0; w < kWaves; ++w) cb += s_bh[w * 64 + lane];
      uint32_t pre = cb;
      for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t v = __shfl_up(pre, o, kWave);
        if (lane >= o) pre += v;
      }
      const uint64_t fits = __ballot(lane < 63 && lane > bmax && pre - static_cast<uint32_t>(M) <= kTopM);
      const int bm2 = fits == 0 ? -1 : 63 - __builtin_clzll(fits);
      const uint32_t thr2 = bm2 >= 0 ? bucket_threshold(bm2) : 0u;
      if (lane == 0) {
        s_n[0] = bm2;
        s_n[1] = static_cast<int>(thr2);
      }
    }
    __syncthreads();
    const int bmax2 = s_n[0];
    const uint32_t thr2 = static_cast<uint32_t>(s_n[1]);
    __syncthreads();
    if (bmax2 < 0) {
      st = 0;
      break;
    }
    for (int p = tid; p < M; p += kThreads) hk[p] = s_keys[p];
    mask = 0;  // buckets (bmax, bmax2]
#pragma unroll
    for (int j = 0; j < kRegSlots; ++j)
      if (ob[j] < thr && ob[j] >= thr2) mask |= 1u << j;
  }
  if (st != 1) {
    if (tid == 0) *flag = 1;
    return;
  }
  if (done != inh) {  // the head back from the workspace
    for (int p = tid; p < M; p += kThreads) s_keys[p] = hk[p];
    __syncthreads();
  }
  nucleus_finish(a, b, s_keys, M, mx, s, s_exp, sh, flag);
}

__device__ __forceinline__ int tail_keep(const SampleArgs& a) {
  return a.top_k > 0 && a.top_k < a.vocab ? a.top_k : a.vocab;
}

// The sampler after a split sort: the merged keys, every id kept unless top-k (above the LDS path)
// keeps k.  Up to kThreads * kScanPer kept ids (a kernel of its own: with the loops below in the
// same kernel, the registers spilled).
__global__ __launch_bounds__(kThreads) void sample_scan_kernel(SampleArgs a) {
  __shared__ ScanShared sh;
  __shared__ int s_flag;
  if (skip_full(a, blockIdx.x)) return;
  sample_tail_scan(a, blockIdx.x, merged_of(a, blockIdx.x), tail_keep(a), sh, s_flag);
}

// More kept ids: the loops one term at a time.
__global__ __launch_bounds__(kThreads) void sample_tail_kernel(SampleArgs a) {
  __shared__ double s_stage[2 * kStage];
  __shared__ int s_stop, s_keep;
  __shared__ double s_sum;
  __shared__ uint64_t s_exp[256];
  const int b = blockIdx.x, V = a.vocab;
  if (skip_full(a, b)) return;
  stage_exp_table(s_exp);
  __syncthreads();
  uint8_t* ws = a.ws + static_cast<size_t>(b) * a.ws_stride;
  double* prob = reinterpret_cast<double*>(ws + ((V * 4 + 255) & ~255));
  sample_tail(a, b, merged_of(a, b), tail_keep(a), false, prob, nullptr, s_stage, s_stop, s_sum, s_keep, s_exp);
}

// exp_libm over an array: the softmax-term call of the kernels above, for comparison with a host
// libm.
__global__ __launch_bounds__(256) void exp_kernel(const double* __restrict__ x, double* __restrict__ y, size_t n) {
  __shared__ uint64_t s_exp[256];
  stage_exp_table(s_exp);
  __syncthreads();
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = exp_libm(x[i], s_exp);
}

}  // namespace

size_t sample_workspace_stride(int vocab) {
  size_t n2 = 1;
  while (n2 < static_cast<size_t>(vocab)) n2 <<= 1;
  const size_t v = static_cast<size_t>(vocab);
  return ((v * 4 + 255) & ~size_t{255}) + prob_region_bytes(v) + 2 * ((n2 * 8 + 255) & ~size_t{255}) + 256;
}

int launch_rng_seed(void* rng, const uint64_t* seeds_dev, int batch, hipStream_t s) {
  hipLaunchKernelGGL(rng_seed_kernel, dim3((batch + 63) / 64), dim3(64), 0, s, static_cast<uint8_t*>(rng), seeds_dev,
                     batch);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_argmax(const float* x, int n, long ld, int batch, int32_t* out, hipStream_t s) {
  EFH_CHECK(n >= 1 && static_cast<size_t>(n) * 4 < (1ull << 32), "argmax: n must be in [1, 2^30)");
  hipLaunchKernelGGL(argmax_kernel, dim3(batch), dim3(kArgmaxThreads), 0, s, x, n, ld, out);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_exp(const double* x, double* y, size_t n, hipStream_t s) {
  if (n == 0) return EF_HIP_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(exp_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, x, y, n);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_argmax_finish(const float* x, int n, long ld, int batch, const StepArgs& f, hipStream_t s) {
  EFH_CHECK(n >= 1 && static_cast<size_t>(n) * 4 < (1ull << 32), "argmax: n must be in [1, 2^30)");
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(batch), dim3(kArgmaxThreads), 0, s, x, n, ld, f);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_rng_discard(void* rng, int batch, int k, hipStream_t s) {
  if (k <= 0) return EF_HIP_OK;
  hipLaunchKernelGGL(rng_discard_kernel, dim3((batch + 63) / 64), dim3(64), 0, s, static_cast<uint8_t*>(rng), batch, k);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_sample(const float* logits, int vocab, int batch, long ld, const ef_hip_sampler_config& cfg,
                  const int32_t* hist, const int32_t* hist_len, long hist_ld, void* rng, int32_t* out, void* ws,
                  hipStream_t s, int eos_id, double* eos_p) {
  SampleArgs a{};
  a.eos_id = eos_id;
  a.eos_p = eos_p;
  a.logits = logits;
  a.ld = ld;
  a.vocab = vocab;
  a.temperature = cfg.temperature;
  a.top_p = cfg.top_p;
  a.penalty = cfg.repetition_penalty;
  a.top_k = cfg.top_k;
  a.hist = hist;
  a.hist_len = hist_len;
  a.hist_ld = hist_ld;
  a.rng = static_cast<uint8_t*>(rng);
  a.out = out;
  a.ws = static_cast<uint8_t*>(ws);
  a.ws_stride = sample_workspace_stride(vocab);
  int n2 = 1;
  while (n2 < vocab) n2 <<= 1;
  a.npow2 = n2;
  // A full sort of 8K+ keys (sampling without a top-k on the LDS path) runs across workgroups:
  // the keys, each kChunk run sorted, the runs merged, then the rest of the sampler.
  const bool topk_lds = cfg.top_k > 0 && cfg.top_k < vocab && cfg.top_k <= kMaxTopK;
  if (cfg.temperature > 0.0f && !topk_lds && n2 >= 2 * kChunk) {
    a.phase = 1;
    // top-p without top-k over a vocabulary the registers hold: the nucleus from the sorted head
    // first; the full sort then runs only for the sequences it leaves
    a.fast = (cfg.top_k <= 0 || cfg.top_k >= vocab) && cfg.top_p < 1.0f && vocab <= kRegSlots * kThreads;
    if (a.fast) {
      hipLaunchKernelGGL(nucleus_kernel, dim3(batch), dim3(kThreads), 0, s, a);  // writes P(eos) too
      hipLaunchKernelGGL(key_sort_kernel, dim3(n2 / kChunk, batch), dim3(kThreads), 0, s, a);
    } else if (eos_p != nullptr) {  // P(eos) needs the whole vocabulary: the one-workgroup key launch
      hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL(chunk_sort_kernel, dim3(n2 / kChunk, batch), dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL(key_sort_kernel, dim3(n2 / kChunk, batch), dim3(kThreads), 0, s, a);
    }
    hipLaunchKernelGGL(rank_merge_kernel, dim3(n2 / kMergeThreads, batch), dim3(kMergeThreads), 0, s, a);
    const int keep = cfg.top_k > 0 && cfg.top_k < vocab ? cfg.top_k : vocab;
    if (keep <= kThreads * kScanPer) {
      hipLaunchKernelGGL(sample_scan_kernel, dim3(batch), dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL(sample_tail_kernel, dim3(batch), dim3(kThreads), 0, s, a);
    }
  } else {
    hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kThreads), 0, s, a);
  }
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

}  // namespace efh
