// The FP32 "glue" of one decode step that is not a packed GEMV (src/kernels.cpp, src/model.cpp):
// embedding row lookup at the current position, RoPE + GQA attention over the KV cache, the
// final RMSNorm output, and the bookkeeping that feeds a picked token back as the next input.
// Positions and token ids are read from device memory so one captured HIP graph serves every step.
//
// Arithmetic follows the reference's operation order with contraction off: the per-position dot
// product uses the 8-way partial sums of kern::dot_f32 (src/kernels.cpp:27-43), softmax subtracts
// the max, uses float exp and a double sum (:77-92), and each output dimension accumulates p * v
// over positions in order (:168-172).
#include <cmath>
#include <cstdlib>
#include <cstring>

#include <utility>

#include "glue.h"
#include "afrag.h"
#include "qdot.h"

#pragma clang fp contract(off)

namespace efh {
namespace {

constexpr int kAttnThreads = 256;

// x[b] = row hist[b][pos] of the embedding table (kern::row_f32 / embedding_bf16).  With rope_now,
// workgroup (0, 0) also copies RoPE's cos and sin rows at pos into rope_now[0, half) and
// [half, 2 half), so the step's attention launches read them without first reading the position.
// With em on, each row is also staged as the first product's tables (afrag.h): 32 consecutive
// threads hold one block of one sequence.
__global__ void embed_at_kernel(const uint8_t* __restrict__ W, int qtype, long rows, long cols, long rb,
                                const int32_t* __restrict__ hist, long hist_ld, const int32_t* __restrict__ pos_dev,
                                float* __restrict__ out, long ldo, const float* __restrict__ cos_t,
                                const float* __restrict__ sin_t, int half, float* __restrict__ rope_now, AEmit em) {
  const int b = blockIdx.y;
  if (rope_now != nullptr && blockIdx.x == 0 && b == 0) {
    const long base = static_cast<long>(*pos_dev) * half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      rope_now[i] = cos_t[base + i];
      rope_now[half + i] = sin_t[base + i];
    }
  }
  const int32_t id = hist[b * hist_ld + *pos_dev];
  const bool ok = id >= 0 && id < rows;
  const uint8_t* row = W + (ok ? id : 0) * rb;
  const long step = static_cast<long>(gridDim.x) * blockDim.x;
  for (long c0 = static_cast<long>(blockIdx.x) * blockDim.x; c0 < cols; c0 += step) {  // uniform trip count
    const long c = c0 + threadIdx.x;
    const bool in = c < cols;
    const float v = in ? (ok ? decode_elem(row, qtype, c) : __int_as_float(0x7FC00000)) : 0.0f;
    if (in) out[b * ldo + c] = v;
    if (em.on()) emit_block(em, b, static_cast<int>(c >> 5), static_cast<int>(c & 31), v, in);
  }
}

// One (query head h, sequence b) per workgroup: RoPE on q and on the new k (half-split pairs,
// src/kernels.cpp:133-146), the new k / v written into the cache at pos by the first head of each
// KV group, then causal attention over positions 0..pos (positions < pos from the cache, pos from
// LDS, so no head waits on another).  K and V rows are staged through LDS in chunks of kAttnChunk
// positions with coalesced float4 loads, each row at a stride of hd + 4 floats so that the lanes
// of a wave reading 16-byte pieces of different rows hit different banks.  A score is one thread's
// dot product with kern::dot_f32's eight partials (i % 8) and its pairwise tree.  P.V keeps the
// reference's order: one thread per output dimension accumulates positions in increasing order.
constexpr int kAttnChunk = 64;

__host__ __device__ constexpr int row_ld(int hd) { return hd + 4; }  // floats between staged rows
// Per-head kernel LDS after the scores: 4 reduction doubles, then (with the first-chunk prefetch)
// the first chunk's V rows at this float offset from the scores, a multiple of 4.
__host__ __device__ constexpr int vrows_offset(int max_seq) { return (((max_seq + 1) & ~1) + 8 + 3) & ~3; }
// Floats of the staging buffer: kAttnChunk padded rows, or `chunk` (a multiple of 4) rows in
// padded 4-row groups for the large-chunk path.
__host__ __device__ constexpr int stage_floats(int hd, int chunk) {
  return chunk > 64 ? (chunk / 4) * (4 * hd + 4) : 64 * (hd + 4);
}

// q . k over hd values (both in LDS, 16-byte aligned) in kern::dot_f32's order: partial j sums the
// products i = j mod 8 in increasing i, a tail joins partial 0, then
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)) (src/kernels.cpp:27-43).
__device__ __forceinline__ float dot_f32_lds(const float* qv, const float* kv, int hd) {
  float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f, p4 = 0.0f, p5 = 0.0f, p6 = 0.0f, p7 = 0.0f;
  int i = 0;
  for (; i + 8 <= hd; i += 8) {
    const float4 qa = *reinterpret_cast<const float4*>(qv + i), qb = *reinterpret_cast<const float4*>(qv + i + 4);
    const float4 ka = *reinterpret_cast<const float4*>(kv + i), kb = *reinterpret_cast<const float4*>(kv + i + 4);
    p0 += qa.x * ka.x;
    p1 += qa.y * ka.y;
    p2 += qa.z * ka.z;
    p3 += qa.w * ka.w;
    p4 += qb.x * kb.x;
    p5 += qb.y * kb.y;
    p6 += qb.z * kb.z;
    p7 += qb.w * kb.w;
  }
  for (; i < hd; ++i) p0 += qv[i] * kv[i];
  return ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7));
}

// dot_f32_lds for a compile-time length: the same partials and tree, every read issued first.
template <int HD>
__device__ __forceinline__ float dot_f32_lds_n(const float* qv, const float* kv) {
  static_assert(HD % 8 == 0, "whole groups of eight");
  float4 qa[HD / 8], qb[HD / 8], ka[HD / 8], kb[HD / 8];
#pragma unroll
  for (int i = 0; i < HD / 8; ++i) {
    qa[i] = *reinterpret_cast<const float4*>(qv + 8 * i);
    qb[i] = *reinterpret_cast<const float4*>(qv + 8 * i + 4);
    ka[i] = *reinterpret_cast<const float4*>(kv + 8 * i);
    kb[i] = *reinterpret_cast<const float4*>(kv + 8 * i + 4);
  }
  float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f, p4 = 0.0f, p5 = 0.0f, p6 = 0.0f, p7 = 0.0f;
#pragma unroll
  for (int i = 0; i < HD / 8; ++i) {
    p0 += qa[i].x * ka[i].x;
    p1 += qa[i].y * ka[i].y;
    p2 += qa[i].z * ka[i].z;
    p3 += qa[i].w * ka[i].w;
    p4 += qb[i].x * kb[i].x;
    p5 += qb[i].y * kb[i].y;
    p6 += qb[i].z * kb[i].z;
    p7 += qb[i].w * kb[i].w;
  }
  return ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7));
}

__device__ __forceinline__ void stage_rows(float* dst, const float* cache, long kvd, const float* cur, int pos,
                                           int c0, int n, int hd) {
  // rows c0 .. c0+n-1 (n <= kAttnChunk) of one KV head, row `pos` from `cur`
  const int q = hd / 4;  // float4 per row (hd % 4 == 0)
  for (int idx = threadIdx.x; idx < n * q; idx += blockDim.x) {
    const int r = idx / q, c = idx - r * q, tp = c0 + r;
    const float* src = tp == pos ? cur : cache + static_cast<long>(tp) * kvd;
    reinterpret_cast<float4*>(dst + r * row_ld(hd))[c] = reinterpret_cast<const float4*>(src)[c];
  }
}

// Large chunks (hd = 64 only): rows c0 .. c0+n-1 of one KV head by LDS-DMA, one full-wave
// buffer_load ... lds per 4 rows (lane l's 16 bytes land at the group's LDS address + 16 l, so a
// group of 4 rows is 1 KB contiguous), groups kGroupFloats apart (16 bytes of padding), every
// group issued before one wait; row `pos` is overwritten from `cur` after a barrier.  n rounded up to
// 4 must fit the buffer (rows past n read zeros).  The caller's barrier publishes them.
constexpr int kDmaHd = 64, kGroupFloats = 4 * kDmaHd + 4;
__device__ __forceinline__ int dma_row_off(int r) { return (r >> 2) * kGroupFloats + (r & 3) * kDmaHd; }
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void stage_rows_dma(float* dst, const float* cache, long kvd, const float* cur, int pos,
                                               int c0, int n) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(cache + static_cast<long>(c0) * kvd,
                                             static_cast<uint32_t>(n) * static_cast<uint32_t>(kvd) * 4u);
  const uint32_t lane_off = (static_cast<uint32_t>(lane >> 4) * static_cast<uint32_t>(kvd) + 4u * (lane & 15)) * 4u;
  for (int j = wave; j < (n + 3) / 4; j += nw)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + j * kGroupFloats), 16,
                                             static_cast<uint32_t>(4 * j) * static_cast<uint32_t>(kvd) * 4u + lane_off,
                                             0, 0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (pos >= c0 && pos < c0 + n) {
    __syncthreads();  // the group holding `pos` may come from another wave's load
    for (int i = threadIdx.x; i < kDmaHd; i += blockDim.x) dst[dma_row_off(pos - c0) + i] = cur[i];
  }
}

// The decode kernel requests the first chunk's cached K and V rows (thread t: float4 slots
// t + kAttnThreads j, row slot / (hd / 4)) before its q / k / v work, so their latency overlaps it,
// and stages them in LDS with the new row at `pos` once that is formed.  kPreSlots covers hd <= 128.
constexpr int kPreSlots = 8;
typedef float pre_f4 __attribute__((ext_vector_type(4)));
struct PreSlots {
  pre_f4 s0, s1, s2, s3, s4, s5, s6, s7;
  template <int J>
  __device__ __forceinline__ pre_f4& at() {
    if constexpr (J == 0) return s0;
    else if constexpr (J == 1) return s1;
    else if constexpr (J == 2) return s2;
    else if constexpr (J == 3) return s3;
    else if constexpr (J == 4) return s4;
    else if constexpr (J == 5) return s5;
    else if constexpr (J == 6) return s6;
    else return s7;
  }
};
template <typename F, int... J>
__device__ __forceinline__ void for_slots_impl(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <typename F>
__device__ __forceinline__ void for_slots(F&& f) {
  for_slots_impl(f, std::make_integer_sequence<int, kPreSlots>{});
}

// Causal attention of one (query head, row) over positions 0 .. n_pos-1 of one KV head: scores in
// kern::dot_f32's order, softmax_inplace, then p.v in position order (src/kernels.cpp:153-174).
// qs (roped query) is in LDS; K and V rows come from the cache except position `cur`, which is
// taken from kn / vn (the decode step's new row; cur = -1 when every row is in the cache).
// With USE_PRE the first chunk is already staged: its K rows in `rows`, its V rows in `vrows`.
template <bool USE_PRE, bool BIG = false>
__device__ __forceinline__ void attend(const float* qs, float* rows, float* sc, double* red, const float* kc,
                                       const float* vc, long kvd, const float* kn, const float* vn, int cur,
                                       int n_pos, int hd, float scale, float* out, const float* vrows,
                                       int big_chunk = kAttnChunk) {
  // With BIG, every chunk after the first (kAttnChunk rows, USE_PRE) has big_chunk rows (hd = 64)
  // staged by LDS-DMA in 4-row groups.  The chunking does not change any operation's order.
  const int t = threadIdx.x, ld = row_ld(hd);
  constexpr bool big = BIG;
  const int chunk = BIG ? big_chunk : kAttnChunk;
  auto step_at = [&](int c0) { return USE_PRE && c0 == 0 ? kAttnChunk : chunk; };
  auto grouped = [&](int c0) { return big && !(USE_PRE && c0 == 0); };  // layout of the chunk at c0
  auto stage = [&](const float* cache, const float* cur_row, int c0, int n) {
    if constexpr (big) {
      stage_rows_dma(rows, cache, kvd, cur_row, cur, c0, n);
    } else {
      stage_rows(rows, cache, kvd, cur_row, cur, c0, n, hd);
    }
  };
  // scores: one thread per position of the chunk; in a grouped chunk lane l of a wave takes row
  // 4 (l % 16) + l / 16 of its 64, so the 16 lanes of each LDS phase read 16 different groups
  for (int c0 = 0; c0 < n_pos; c0 += step_at(c0)) {
    const int n = min(step_at(c0), n_pos - c0);
    if (!USE_PRE || c0 > 0) stage(kc, kn, c0, n);
    __syncthreads();
    if (grouped(c0)) {
      const int l = t & (kWave - 1), lr = 4 * (l & 15) + (l >> 4);
      for (int r = (t - l) + lr; r < ((n + kWave - 1) & ~(kWave - 1)); r += blockDim.x)
        if (r < n) sc[c0 + r] = dot_f32_lds(qs, rows + dma_row_off(r), hd) * scale;
    } else if (t < n) {  // n <= kAttnChunk <= blockDim.x
      sc[c0 + t] = dot_f32_lds(qs, rows + t * ld, hd) * scale;
    }
    __syncthreads();
  }
  // softmax_inplace: max, float exp(x - max), double sum, scale by float(1 / sum)
  float mx = -INFINITY;
  for (int tp = t; tp < n_pos; tp += blockDim.x) mx = fmaxf(mx, sc[tp]);
  mx = wave_max_dpp(mx);
  if ((t & (kWave - 1)) == 0) red[t / kWave] = mx;
  __syncthreads();
  mx = static_cast<float>(red[0]);
  for (int w = 1; w < static_cast<int>(blockDim.x) / kWave; ++w) mx = fmaxf(mx, static_cast<float>(red[w]));
  __syncthreads();
  double s = 0.0;
  for (int tp = t; tp < n_pos; tp += blockDim.x) {
    const float e = expf(sc[tp] - mx);
    sc[tp] = e;
    s += static_cast<double>(e);
  }
  s = wave_sum_d_dpp(s);
  if ((t & (kWave - 1)) == 0) red[t / kWave] = s;
  __syncthreads();
  double tot = 0.0;
  for (int w = 0; w < static_cast<int>(blockDim.x) / kWave; ++w) tot += red[w];
  const float inv = static_cast<float>(1.0 / tot);
  // out[d] = sum_t p_t v_t[d], positions in order
  float o = 0.0f;
  for (int c0 = 0; c0 < n_pos; c0 += step_at(c0)) {
    const int n = min(step_at(c0), n_pos - c0);
    const float* vr = rows;
    if (USE_PRE && c0 == 0) {
      vr = vrows;
    } else {
      stage(vc, vn, c0, n);
    }
    __syncthreads();
    if (t < hd) {
      if (grouped(c0)) {
        for (int r = 0; r < n; ++r) {
          const float p = sc[c0 + r] * inv;
          o += p * vr[dma_row_off(r) + t];
        }
      } else {
        for (int r = 0; r < n; ++r) {
          const float p = sc[c0 + r] * inv;
          o += p * vr[r * ld + t];
        }
      }
    }
    __syncthreads();
  }
  if (t < hd) out[t] = o;
}


template <bool PRE, bool BIG>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int h = blockIdx.x, b = blockIdx.y, hd = a.hd, half = hd / 2;
  const int pos = *a.pos_dev, n_pos = pos + 1;
  const int g = h / (a.H / a.KV), kvd = a.KV * hd;
  float* qs = sm;              // [hd]
  float* kn = sm + hd;         // [hd] roped new k
  float* vn = sm + 2 * hd;     // [hd] new v
  float* rows = sm + 3 * hd;   // staged K or V rows: [kAttnChunk][row_ld(hd)], or a.chunk grouped rows
  float* sc = rows + (BIG ? stage_floats(hd, a.chunk) : kAttnChunk * row_ld(hd));  // [n_pos] scores / probabilities
  double* red = reinterpret_cast<double*>(sc + ((a.max_seq + 1) & ~1));
  const float* cr = a.cos_t + static_cast<long>(pos) * half;
  const float* sr = a.sin_t + static_cast<long>(pos) * half;
  const float* q = a.q + static_cast<long>(b) * a.ldq + h * hd;
  const float* k_new = a.knew + static_cast<long>(b) * kvd + g * hd;
  const float* v_new = a.vnew + static_cast<long>(b) * kvd + g * hd;
  const float* kc = a.kcache + (static_cast<long>(b) * a.max_seq) * kvd + g * hd;  // this layer, sequence, head
  const float* vc = a.vcache + (static_cast<long>(b) * a.max_seq) * kvd + g * hd;
  const int t = threadIdx.x;
  // the first chunk's cached K / V rows are requested before the q / k / v work below
  const bool pre = PRE && hd * kAttnChunk <= 4 * kPreSlots * kAttnThreads && a.pre_vrows;
  const int n0 = min(kAttnChunk, n_pos), q4n = hd / 4;
  // one register pair per slot (separate variables: an indexed array would live in scratch)
  PreSlots pk, pv;
  if (pre) {
    for_slots([&](auto J) {
      const int idx = t + kAttnThreads * decltype(J)::value, r = idx / q4n, c = idx - r * q4n;
      if (r < n0 && r != pos) {
        pk.template at<decltype(J)::value>() = reinterpret_cast<const pre_f4*>(kc + static_cast<long>(r) * kvd)[c];
        pv.template at<decltype(J)::value>() = reinterpret_cast<const pre_f4*>(vc + static_cast<long>(r) * kvd)[c];
      }
    });
  }
  if (t < half) {
    const float qa = q[t], qb = q[t + half], ka = k_new[t], kb = k_new[t + half];
    qs[t] = qa * cr[t] - qb * sr[t];
    qs[t + half] = qb * cr[t] + qa * sr[t];
    kn[t] = ka * cr[t] - kb * sr[t];
    kn[t + half] = kb * cr[t] + ka * sr[t];
  }
  for (int i = t; i < hd; i += blockDim.x) vn[i] = v_new[i];
  __syncthreads();
  if (h % (a.H / a.KV) == 0) {  // the group's first head publishes k / v at pos for later steps
    float* kw = a.kcache + (static_cast<long>(b) * a.max_seq + pos) * kvd + g * hd;
    float* vw = a.vcache + (static_cast<long>(b) * a.max_seq + pos) * kvd + g * hd;
    for (int i = t; i < hd; i += blockDim.x) {
      kw[i] = kn[i];
      vw[i] = vn[i];
    }
  }
  if (pre) {
    float* vrows = sc + vrows_offset(a.max_seq);  // after the reduction slots, 16-byte aligned
    for_slots([&](auto J) {
      const int idx = t + kAttnThreads * decltype(J)::value, r = idx / q4n, c = idx - r * q4n;
      if (r < n0) {
        reinterpret_cast<pre_f4*>(rows + r * row_ld(hd))[c] =
            r == pos ? reinterpret_cast<const pre_f4*>(kn)[c] : pk.template at<decltype(J)::value>();
        reinterpret_cast<pre_f4*>(vrows + r * row_ld(hd))[c] =
            r == pos ? reinterpret_cast<const pre_f4*>(vn)[c] : pv.template at<decltype(J)::value>();
      }
    });
    attend<true, BIG>(qs, rows, sc, red, kc, vc, kvd, kn, vn, pos, n_pos, hd, a.scale,
                      a.ctx + static_cast<long>(b) * a.ldq + h * hd, vrows, a.chunk);
  } else {
    attend<false>(qs, rows, sc, red, kc, vc, kvd, kn, vn, pos, n_pos, hd, a.scale,
                  a.ctx + static_cast<long>(b) * a.ldq + h * hd, nullptr);
  }
}

// One wave per (query head h, sequence b) for hd = 64 (the small-batch decode): lane l owns
// dimension l for RoPE and p.v, and position c0 + l of each 64-position chunk for the scores.
// Every load that does not need the position is issued at entry: this step's q / k / v, the
// step's RoPE row (rope_now, required), the first chunk's cached K
// rows (one row per lane) and V values (one column per lane).  The first 64 rows are in bounds
// whatever the position (rows past it are never used), so a single memory round trip precedes
// the arithmetic; softmax and p.v stay inside the wave (DPP reductions, p broadcast by readlane),
// with no workgroup barrier.  Operation order as attention_kernel: kern::dot_f32's partials and
// tree per score, float exp(s - max), a double sum, p = e * inv, and p * v accumulated per
// dimension over positions in increasing order (src/kernels.cpp:27-43,77-92,153-174); the double
// sum adds lane partials by a DPP tree, so its last bits can differ from the per-head kernel's.
constexpr int kWaveHd = 64;

__global__ __launch_bounds__(kWave) void attention_wave_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  float* qs = sm;                // [64] roped query
  float* kn = sm + kWaveHd;      // [64] roped new key
  float* sc = sm + 2 * kWaveHd;  // [max_seq]: scores, then exp, of positions >= 64
  const int h = blockIdx.x, b = blockIdx.y, l = threadIdx.x;
  const int hpg = a.H / a.KV, g = h / hpg, kvd = a.KV * kWaveHd;
  const float* qr = a.q + static_cast<long>(b) * a.ldq + h * kWaveHd;
  const float* knr = a.knew + static_cast<long>(b) * kvd + g * kWaveHd;
  const float* vnr = a.vnew + static_cast<long>(b) * kvd + g * kWaveHd;
  const long seq0 = static_cast<long>(b) * a.max_seq * kvd + g * kWaveHd;
  // one buffer resource over this (sequence, KV head)'s rows of the layer's cache
  const uint32_t span = static_cast<uint32_t>(a.max_seq - 1) * static_cast<uint32_t>(kvd) * 4u + kWaveHd * 4u;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kcache + seq0, span);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vcache + seq0, span);
  const uint32_t row_bytes = static_cast<uint32_t>(kvd) * 4u;
  const int n0 = min(kWaveHd, a.max_seq);

  // 1. loads, in the order they are consumed (vector-memory loads return in order).  The position
  //    is a vector load: as a scalar load its wait would also hold back the loads issued after it.
  const int pos_v = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.pos_dev, 4u), 0u, 0u, 0);
  const float q0 = qr[l], q1 = qr[l ^ 32], k0 = knr[l], k1 = knr[l ^ 32], vnew = vnr[l];
  const float cs = a.rope_now[l & 31], sn = a.rope_now[32 + (l & 31)];
  float4 kr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) kr[i] = buf_f4(rk, static_cast<uint32_t>(l) * row_bytes + 16u * i);
  __builtin_amdgcn_sched_barrier(0);  // the K rows (consumed first) are issued before the V values
  float vr[kWaveHd];
#pragma unroll
  for (int r = 0; r < kWaveHd; ++r)
    vr[r] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, static_cast<uint32_t>(l) * 4u,
                                                                static_cast<uint32_t>(r) * row_bytes, 0));

  // 2. RoPE on q and the new k (half-split pairs, src/kernels.cpp:133-146); the group's first head
  //    publishes k / v at pos for later steps
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);
  float qrot, krot;
  if (l < 32) {
    qrot = q0 * cs - q1 * sn;
    krot = k0 * cs - k1 * sn;
  } else {
    qrot = q0 * cs + q1 * sn;
    krot = k0 * cs + k1 * sn;
  }
  qs[l] = qrot;
  kn[l] = krot;
  if (h % hpg == 0) {
    a.kcache[seq0 + static_cast<long>(pos) * kvd + l] = krot;
    a.vcache[seq0 + static_cast<long>(pos) * kvd + l] = vnew;
  }
  __syncthreads();

  // 3. scores: the first chunk from registers (row pos from kn), later chunks loaded per chunk
  const int n_pos = pos + 1, c0n = min(n_pos, n0);
  float s0 = -INFINITY;
  if (l < c0n) {
    if (l == pos) {
#pragma unroll
      for (int i = 0; i < 16; ++i) kr[i] = reinterpret_cast<const float4*>(kn)[i];
    }
    s0 = dot64_regs(qs, kr) * a.scale;
  }
  float mx = s0;
  for (int c0 = kWaveHd; c0 < n_pos; c0 += kWaveHd) {
    const int r = c0 + l;
    if (r < n_pos) {
      float4 k4[16];
      if (r == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) k4[i] = reinterpret_cast<const float4*>(kn)[i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) k4[i] = buf_f4(rk, static_cast<uint32_t>(r) * row_bytes + 16u * i);
      }
      const float s = dot64_regs(qs, k4) * a.scale;
      sc[r] = s;
      mx = fmaxf(mx, s);
    }
  }

  // 4. softmax_inplace: max, float exp(s - max), double sum, inv = float(1 / sum)
  mx = wave_max_dpp(mx);
  const float e0 = l < c0n ? expf(s0 - mx) : 0.0f;
  double ssum = static_cast<double>(e0);
  for (int r = kWaveHd + l; r < n_pos; r += kWaveHd) {
    const float e = expf(sc[r] - mx);
    sc[r] = e;
    ssum += static_cast<double>(e);
  }
  const float inv = static_cast<float>(1.0 / wave_sum_d_dpp(ssum));
  __syncthreads();  // sc[] exps visible to every lane

  // 5. out[l] = sum_t p_t v_t[l], positions in increasing order
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < kWaveHd; ++r) {
    if (r < c0n) {
      const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), r)) * inv;
      o += p * (r == pos ? vnew : vr[r]);
    }
  }
  for (int c0 = kWaveHd; c0 < n_pos; c0 += kWaveHd) {
    const int n = min(kWaveHd, n_pos - c0);
#pragma unroll
    for (int r = 0; r < kWaveHd; ++r)
      if (r < n)
        vr[r] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            rv, static_cast<uint32_t>(l) * 4u, static_cast<uint32_t>(c0 + r) * row_bytes, 0));
#pragma unroll
    for (int r = 0; r < kWaveHd; ++r) {
      if (r < n) {
        const float p = sc[c0 + r] * inv;
        o += p * (c0 + r == pos ? vnew : vr[r]);
      }
    }
  }
  a.ctx[static_cast<long>(b) * a.ldq + h * kWaveHd + l] = o;
}

// One (KV group g, sequence b) per workgroup of kGroupThreads: the group's hpg query heads share
// each staged K / V chunk, so the cache is read once per group instead of once per head (the
// large-batch decode; launch_attention picks it).  Every head's arithmetic is the per-head
// kernel's, operation for operation: a quad of lanes per (head, position) score with the same
// partials and DPP tree, the softmax sums laid out as 256 threads (each half of the workgroup
// takes every other head: thread t % 256 sums positions t % 256 + 256 i, then the four waves in
// order), and one thread per (head, dimension) accumulating p * v over positions in order.
constexpr int kGroupThreads = 512;
constexpr int kGroupMaxOut = 4;  // (head, dimension) outputs per thread

// Slots of the first chunk's K and V rows held in registers by each thread of the group kernel:
// kAttnChunk rows of hd / 4 float4 over kGroupThreads threads (hd <= 128).
constexpr int kGroupPreSlots = 4;
struct GroupPre {
  pre_f4 s0, s1, s2, s3;
  template <int J>
  __device__ __forceinline__ pre_f4& at() {
    if constexpr (J == 0) return s0;
    else if constexpr (J == 1) return s1;
    else if constexpr (J == 2) return s2;
    else return s3;
  }
};
template <typename F>
__device__ __forceinline__ void for_group_slots(F&& f) {
  for_slots_impl(f, std::make_integer_sequence<int, kGroupPreSlots>{});
}

__global__ __launch_bounds__(kGroupThreads) void attention_group_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int g = blockIdx.x, b = blockIdx.y, hd = a.hd, half = hd / 2;
  const int hpg = a.H / a.KV, kvd = a.KV * hd, sp = (a.max_seq + 1) & ~1;
  float* qs = sm;                      // [hpg][hd] roped queries
  float* kn = qs + hpg * hd;           // [hd] roped new k
  float* vn = kn + hd;                 // [hd] new v
  const int ld = row_ld(hd);
  float* rows = vn + hd;                  // [kAttnChunk][ld] staged K rows (later chunks: K or V)
  float* vrows = rows + kAttnChunk * ld;  // [kAttnChunk][ld] the first chunk's V rows
  float* sc = vrows + kAttnChunk * ld;    // [hpg][sp] scores / probabilities
  float* invs = sc + hpg * sp;            // [hpg] 1 / sum of each head's exponentials
  const float* q = a.q + static_cast<long>(b) * a.ldq + g * hpg * hd;
  const float* k_new = a.knew + static_cast<long>(b) * kvd + g * hd;
  const float* v_new = a.vnew + static_cast<long>(b) * kvd + g * hd;
  const float* kc = a.kcache + (static_cast<long>(b) * a.max_seq) * kvd + g * hd;
  const float* vc = a.vcache + (static_cast<long>(b) * a.max_seq) * kvd + g * hd;
  const int t = threadIdx.x;
  // The first chunk's cached rows (every row below max_seq is in bounds; rows at or past the
  // position are replaced or unused) are requested with the position, q, k and v.
  const int q4n = hd / 4, n_pre = min(kAttnChunk, a.max_seq);
  GroupPre pk, pv;
  for_group_slots([&](auto J) {
    const int idx = t + kGroupThreads * decltype(J)::value, r = idx / q4n, c = idx - r * q4n;
    if (r < n_pre) {
      pk.template at<decltype(J)::value>() = reinterpret_cast<const pre_f4*>(kc + static_cast<long>(r) * kvd)[c];
      pv.template at<decltype(J)::value>() = reinterpret_cast<const pre_f4*>(vc + static_cast<long>(r) * kvd)[c];
    }
  });
  const int pos = *a.pos_dev, n_pos = pos + 1;
  // RoPE's rows at pos: the step's copy (no load waiting on the position) or the tables
  const float* cr = a.rope_now != nullptr ? a.rope_now : a.cos_t + static_cast<long>(pos) * half;
  const float* sr = a.rope_now != nullptr ? a.rope_now + half : a.sin_t + static_cast<long>(pos) * half;
  for (int idx = t; idx < hpg * half; idx += kGroupThreads) {
    const int hh = idx / half, j = idx - hh * half;
    const float qa = q[hh * hd + j], qb = q[hh * hd + j + half];
    qs[hh * hd + j] = qa * cr[j] - qb * sr[j];
    qs[hh * hd + j + half] = qb * cr[j] + qa * sr[j];
  }
  if (t < half) {
    const float ka = k_new[t], kb = k_new[t + half];
    kn[t] = ka * cr[t] - kb * sr[t];
    kn[t + half] = kb * cr[t] + ka * sr[t];
  }
  for (int i = t; i < hd; i += kGroupThreads) vn[i] = v_new[i];
  __syncthreads();
  {  // k / v at pos for later steps
    float* kw = a.kcache + (static_cast<long>(b) * a.max_seq + pos) * kvd + g * hd;
    float* vw = a.vcache + (static_cast<long>(b) * a.max_seq + pos) * kvd + g * hd;
    for (int i = t; i < hd; i += kGroupThreads) {
      kw[i] = kn[i];
      vw[i] = vn[i];
    }
  }
  const int n0 = min(kAttnChunk, n_pos);
  for_group_slots([&](auto J) {
    const int idx = t + kGroupThreads * decltype(J)::value, r = idx / q4n, c = idx - r * q4n;
    if (r < n0) {
      reinterpret_cast<pre_f4*>(rows + r * ld)[c] =
          r == pos ? reinterpret_cast<const pre_f4*>(kn)[c] : pk.template at<decltype(J)::value>();
      reinterpret_cast<pre_f4*>(vrows + r * ld)[c] =
          r == pos ? reinterpret_cast<const pre_f4*>(vn)[c] : pv.template at<decltype(J)::value>();
    }
  });
  // scores: thread -> (head, position) of the chunk, positions across the lanes of a wave (one
  // query row broadcast, distinct K rows)
  for (int c0 = 0; c0 < n_pos; c0 += kAttnChunk) {
    const int n = min(kAttnChunk, n_pos - c0);
    if (c0 > 0) stage_rows(rows, kc, kvd, kn, pos, c0, n, hd);
    __syncthreads();
    for (int pr = t; pr < hpg * kAttnChunk; pr += kGroupThreads) {
      const int hh = pr / kAttnChunk, r = pr - hh * kAttnChunk;
      if (r < n)
        sc[hh * sp + c0 + r] = (hd == 64 ? dot_f32_lds_n<64>(qs + hh * hd, rows + r * ld)
                                         : dot_f32_lds(qs + hh * hd, rows + r * ld, hd)) *
                               a.scale;
    }
    __syncthreads();
  }
  // softmax: one wave per head.  The per-head kernel's sums run over 256 threads (thread v takes
  // positions v + 256 i, then a DPP tree per wave, then the four waves in order); lane l here
  // keeps that layout's four threads l, 64 + l, 128 + l, 192 + l as four partial sums.
  {
    const int wave = t / kWave, lane = t & (kWave - 1);
    for (int hh = wave; hh < hpg; hh += kGroupThreads / kWave) {
      float* sh = sc + hh * sp;
      float mx = -INFINITY;
      for (int tp = lane; tp < n_pos; tp += kWave) mx = fmaxf(mx, sh[tp]);
      mx = wave_max_dpp(mx);
      double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
      for (int base = 0; base < n_pos; base += 4 * kWave) {
        auto take = [&](int tp, double& acc) {
          if (tp < n_pos) {
            const float e = expf(sh[tp] - mx);
            sh[tp] = e;
            acc += static_cast<double>(e);
          }
        };
        take(base + lane, s0);
        take(base + kWave + lane, s1);
        take(base + 2 * kWave + lane, s2);
        take(base + 3 * kWave + lane, s3);
      }
      // partials that took no position are exact zeros (adding them changes nothing): their
      // reductions are skipped (n_pos is uniform)
      s0 = wave_sum_d_dpp(s0);
      if (n_pos > kWave) s1 = wave_sum_d_dpp(s1);
      if (n_pos > 2 * kWave) s2 = wave_sum_d_dpp(s2);
      if (n_pos > 3 * kWave) s3 = wave_sum_d_dpp(s3);
      double tot = 0.0;
      tot += s0;
      tot += s1;
      tot += s2;
      tot += s3;
      if (lane == 0) invs[hh] = static_cast<float>(1.0 / tot);
    }
  }
  __syncthreads();
  // out[h][d] = sum_t p_t v_t[d], positions in order
  float o[kGroupMaxOut], inv[kGroupMaxOut];
#pragma unroll
  for (int u = 0; u < kGroupMaxOut; ++u) {
    o[u] = 0.0f;
    const int hh = (t + u * kGroupThreads) / hd;
    inv[u] = hh < hpg ? invs[hh] : 0.0f;
  }
  for (int c0 = 0; c0 < n_pos; c0 += kAttnChunk) {
    const int n = min(kAttnChunk, n_pos - c0);
    const float* vr = c0 == 0 ? vrows : rows;
    if (c0 > 0) {
      stage_rows(rows, vc, kvd, vn, pos, c0, n, hd);
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kGroupMaxOut; ++u) {
      const int idx = t + u * kGroupThreads, hh = idx / hd, d = idx - hh * hd;
      if (hh < hpg) {
        const float* ph = sc + hh * sp + c0;
        // eight positions' reads issued before their multiply-adds (the adds stay in order)
        int r = 0;
        for (; r + 8 <= n; r += 8) {
          float pp[8], vv[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            pp[k] = ph[r + k];
            vv[k] = vr[(r + k) * ld + d];
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float pv_ = pp[k] * inv[u];
            o[u] += pv_ * vv[k];
          }
        }
        for (; r < n; ++r) {
          const float pv_ = ph[r] * inv[u];
          o[u] += pv_ * vr[r * ld + d];
        }
      }
    }
    __syncthreads();
  }
  float* out = a.ctx + static_cast<long>(b) * a.ldq + g * hpg * hd;
#pragma unroll
  for (int u = 0; u < kGroupMaxOut; ++u) {
    const int idx = t + u * kGroupThreads;
    if (idx < hpg * hd) out[idx] = o[u];
    // staged as the o-projection's tables: 32 consecutive threads hold one block of this sequence
    if (a.em.on()) {
      const int e = g * hpg * hd + idx;
      emit_block(a.em, b, e >> 5, e & 31, o[u], idx < hpg * hd);
    }
  }
}

// Position-split decode attention (hd = 64, at most 8 query heads per KV head): workgroup
// (j, g, b) takes positions [j span, (j + 1) span) of KV group g of sequence b, up to the current
// position, for all of the group's query heads (the cache rows are read once per group).  Its
// scores follow kern::dot_f32's order (src/kernels.cpp:27-43); with several splits active each one
// keeps its own maximum m_j, float exp(s - m_j), their double sum l_j and the unnormalised
// o_j[d] = sum_t e_t v_t[d] (positions in order) in a record, and attention_combine_kernel adds the
// splits in index order: M = max m_j, w_j = exp(m_j - M), out[d] = (sum_j w_j o_j[d]) *
// float(1 / sum_j w_j l_j).  The order is fixed, so results are reproducible; they differ from the
// reference's single pass (src/kernels.cpp:153-174) by the rounding of the regrouped sums.  With
// one split active (positions < span) the workgroup runs the reference's softmax_inplace and p.v
// order itself and writes ctx directly.  Split 0 always has work and requests its rows before it
// reads the position; the others read it first and leave at once when they have none.
constexpr int kSplitThreads = 256;
constexpr int kSplitRows = 64;     // cache rows staged in LDS at a time (the span is a multiple)
constexpr int kSplitHd = 64;
constexpr int kSplitMaxHpg = 8;
constexpr int kSplitRec = kSplitMaxHpg * kSplitHd + kSplitMaxHpg + 2 * kSplitMaxHpg;  // o, m, l (doubles)
constexpr int kSplitLd = kSplitHd + 4;  // floats between staged rows
constexpr int kSplitPerThread = 16;  // splits whose o columns one thread holds in the combine
constexpr int kSplitMaxSplits = 64;  // splits of one (sequence, group): the combine's wave lanes
// Combine kernel LDS (one query head per workgroup): sums (doubles) and weights per split, tpc x
// cols float4 sub-sums, 1 / sum.
constexpr size_t kCombineLds = (2 * kSplitMaxSplits + kSplitMaxSplits + 4 * kSplitThreads + 1) * sizeof(float);
// The most splits the combine takes (one wave's lanes form the weights; each thread holds up to
// kSplitPerThread of them for its column).
__host__ __device__ constexpr int split_max(int) {
  return kSplitPerThread * (kSplitThreads / (kSplitHd / 4)) < kSplitMaxSplits ? kSplitPerThread * (kSplitThreads / (kSplitHd / 4))
                                                                               : kSplitMaxSplits;
}

size_t attention_split_lds_bytes(int hpg, int span) {
  return (static_cast<size_t>(hpg + 2) * kSplitHd + 2 * kSplitRows * kSplitLd + static_cast<size_t>(hpg) * span +
          3 * kSplitMaxHpg) *
         sizeof(float);
}

template <bool EAGER>
__global__ __launch_bounds__(kSplitThreads) void attention_split_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int hpg = a.split_hpw, parts = a.H / a.KV / hpg;  // this workgroup's query heads: h0 .. h0 + hpg - 1
  const int j = blockIdx.x, g = blockIdx.y / parts, h0 = (blockIdx.y - g * parts) * hpg, b = blockIdx.z, t = threadIdx.x;
  const int kvd = a.KV * kSplitHd, span = a.span;
  float* qs = sm;                                 // [hpg][64] roped queries
  float* kn = qs + hpg * kSplitHd;                // [64] roped new key
  float* vn = kn + kSplitHd;                      // [64] new value
  float* rows = vn + kSplitHd;                    // [64][kSplitLd] K rows (later sub-chunks: K or V)
  float* vrows = rows + kSplitRows * kSplitLd;    // [64][kSplitLd] the first sub-chunk's V rows
  float* sc = vrows + kSplitRows * kSplitLd;      // [hpg][span] scores, then exponentials
  double* s_l = reinterpret_cast<double*>(sc + hpg * span);  // [8] sums (span, hpg: even offset)
  float* s_m = reinterpret_cast<float*>(s_l + kSplitMaxHpg);  // [8] maxima
  const long seq0 = static_cast<long>(b) * a.max_seq * kvd + g * kSplitHd;
  const float* kc = a.kcache + seq0;
  const float* vc = a.vcache + seq0;
  const int c0 = j * span, n_first = min(kSplitRows, a.max_seq - c0);  // c0 < max_seq (host plan)

  // Loads that do not need the position go first, behind the position itself (a vector load, so
  // that waiting for it leaves the later ones in flight): the group's queries, RoPE's row at pos,
  // the new k / v, and (split 0 always, every split with EAGER) the first sub-chunk's cache rows.
  // Without EAGER, the other splits request their rows once the position shows they have work.
  const int pos_v = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.pos_dev, 4u), 0u, 0u, 0);
  const float* q = a.q + static_cast<long>(b) * a.ldq + (g * hpg * parts + h0) * kSplitHd;
  const float* k_new = a.knew + static_cast<long>(b) * kvd + g * kSplitHd;
  const int hq = t >> 5, iq = t & 31;
  float qa = 0.0f, qb = 0.0f, cq = 0.0f, sq = 0.0f, ka = 0.0f, kb = 0.0f, vnew = 0.0f;
  if (t < hpg * (kSplitHd / 2)) {
    qa = q[hq * kSplitHd + iq];
    qb = q[hq * kSplitHd + iq + 32];
  }
  if (t < hpg * (kSplitHd / 2) || t < kSplitHd) {
    cq = a.rope_now[iq];
    sq = a.rope_now[kSplitHd / 2 + iq];
  }
  if (t < kSplitHd) {
    ka = k_new[t & 31];
    kb = k_new[(t & 31) + 32];
    vnew = a.vnew[static_cast<long>(b) * kvd + g * kSplitHd + t];
  }
  float4 pk[4], pv[4];
  auto prefetch = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = t + kSplitThreads * i, r = idx >> 4, c = idx & 15;
      if (r < n_first) {
        pk[i] = reinterpret_cast<const float4*>(kc + static_cast<long>(c0 + r) * kvd)[c];
        pv[i] = reinterpret_cast<const float4*>(vc + static_cast<long>(c0 + r) * kvd)[c];
      }
    }
  };
  if (EAGER || j == 0) prefetch();
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);
  if (j * span > pos) return;  // no positions for this split
  if (!EAGER && j != 0) prefetch();
  const int n_pos = pos + 1, n_act = (n_pos + span - 1) / span;
  const bool last = j == n_act - 1;
  const int n_loc = min(span, n_pos - c0);

  // RoPE on the group's queries (one pair per thread) and, in the split holding pos, on the new
  // key; that split publishes k / v at pos for later steps (src/kernels.cpp:133-146)
  if (t < hpg * (kSplitHd / 2)) {
    qs[hq * kSplitHd + iq] = qa * cq - qb * sq;
    qs[hq * kSplitHd + iq + 32] = qb * cq + qa * sq;
  }
  if (last && t < kSplitHd) {
    const float k = t < 32 ? ka * cq - kb * sq : kb * cq + ka * sq;
    kn[t] = k;
    vn[t] = vnew;
    if (h0 == 0) {
      a.kcache[seq0 + static_cast<long>(pos) * kvd + t] = k;
      a.vcache[seq0 + static_cast<long>(pos) * kvd + t] = vnew;
    }
  }
  __syncthreads();
  // staged rows past the split's last position are zeros: p.v runs over whole 64-row sub-chunks
  // with p = 0 there (adding 0 * 0 leaves a sum unchanged)
  const int n0 = min(kSplitRows, n_loc);
  const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kSplitThreads * i, r = idx >> 4, c = idx & 15;
    float4 kv = zero4, vv = zero4;
    if (r < n0) {
      kv = pk[i];
      vv = pv[i];
      if (c0 + r == pos) {
        kv = reinterpret_cast<const float4*>(kn)[c];
        vv = reinterpret_cast<const float4*>(vn)[c];
      }
    }
    reinterpret_cast<float4*>(rows + r * kSplitLd)[c] = kv;
    reinterpret_cast<float4*>(vrows + r * kSplitLd)[c] = vv;
  }
  auto stage = [&](const float* cache, const float* cur_row, int s0, int n) {
    for (int idx = t; idx < kSplitRows * 16; idx += kSplitThreads) {
      const int r = idx >> 4, c = idx & 15, tp = c0 + s0 + r;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (r < n) v = reinterpret_cast<const float4*>(tp == pos ? cur_row : cache + static_cast<long>(tp) * kvd)[c];
      reinterpret_cast<float4*>(rows + r * kSplitLd)[c] = v;
    }
  };

  // scores: a wave per (head, 64 positions), positions across the lanes
  for (int s0 = 0; s0 < n_loc; s0 += kSplitRows) {
    const int n = min(kSplitRows, n_loc - s0);
    if (s0 > 0) stage(kc, kn, s0, n);
    __syncthreads();
    for (int pr = t; pr < hpg * kSplitRows; pr += kSplitThreads) {
      const int hh = pr >> 6, r = pr & 63;
      if (r < n) sc[hh * span + s0 + r] = dot_f32_lds(qs + hh * kSplitHd, rows + r * kSplitLd, kSplitHd) * a.scale;
    }
    __syncthreads();
  }
  // softmax over the split's positions: a wave per head (max, float exp, double sum)
  {
    const int wave = t / kWave, lane = t & (kWave - 1);
    for (int hh = wave; hh < hpg; hh += kSplitThreads / kWave) {
      float* sh = sc + hh * span;
      float mx = -INFINITY;
      for (int p = lane; p < n_loc; p += kWave) mx = fmaxf(mx, sh[p]);
      mx = wave_max_dpp(mx);
      double l = 0.0;
      for (int p = lane; p < n_loc; p += kWave) {
        const float e = expf(sh[p] - mx);
        sh[p] = e;
        l += static_cast<double>(e);
      }
      l = wave_sum_d_dpp(l);
      if (lane == 0) {
        s_m[hh] = mx;
        s_l[hh] = l;
      }
    }
  }
  __syncthreads();
  // p.v: thread -> (head, dimension) outputs, positions in order; one split: p = e * float(1 / l)
  // (softmax_inplace), several: the unnormalised e
  float o[2] = {0.0f, 0.0f}, inv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int hh = (t + u * kSplitThreads) >> 6;
    inv[u] = hh < hpg && n_act == 1 ? static_cast<float>(1.0 / s_l[hh]) : 1.0f;
  }
  // (a wave's outputs share one head: lane r holds p of row r, broadcast by readlane)
  for (int s0 = 0; s0 < n_loc; s0 += kSplitRows) {
    const int n = min(kSplitRows, n_loc - s0);
    const float* vr = s0 == 0 ? vrows : rows;
    if (s0 > 0) {
      stage(vc, vn, s0, n);
      __syncthreads();
    }
    const int lane = t & (kWave - 1);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + u * kSplitThreads, hh = idx >> 6, d = idx & 63;
      if (hh < hpg) {
        const int pl = __float_as_int(lane < n ? sc[hh * span + s0 + lane] * inv[u] : 0.0f);
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r) {
          const float p = __int_as_float(__builtin_amdgcn_readlane(pl, r));
          o[u] += p * vr[r * kSplitLd + d];
        }
      }
    }
    __syncthreads();
  }
  float* out = a.ctx + static_cast<long>(b) * a.ldq + (g * hpg * parts + h0) * kSplitHd;
  if (n_act == 1) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + u * kSplitThreads;
      if (idx < hpg * kSplitHd) out[idx] = o[u];
    }
    return;
  }
  float* recs = a.part + static_cast<long>(b * a.KV + g) * a.splits * kSplitRec;
  {
    float* rec = recs + static_cast<long>(j) * kSplitRec;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + u * kSplitThreads;
      if (idx < hpg * kSplitHd) rec[h0 * kSplitHd + idx] = o[u];
    }
    if (t < hpg) {
      rec[kSplitMaxHpg * kSplitHd + h0 + t] = s_m[t];
      reinterpret_cast<double*>(rec + kSplitMaxHpg * kSplitHd + kSplitMaxHpg)[h0 + t] = s_l[t];
    }
  }
}

// The combine of the position-split attention: one workgroup per (query head, sequence b), after
// the split kernel (the kernel boundary makes every split's record visible).  With one split
// active the split kernel has written ctx itself and this returns at once.
template <bool EAGER>
__global__ __launch_bounds__(kSplitThreads) void attention_combine_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int hpg = a.H / a.KV, g = blockIdx.x / hpg, hh = blockIdx.x - g * hpg, b = blockIdx.y, t = threadIdx.x;
  const float* recs = a.part + static_cast<long>(b * a.KV + g) * a.splits * kSplitRec;
  float* out = a.ctx + static_cast<long>(b) * a.ldq + (g * hpg + hh) * kSplitHd;
  // One query head per workgroup.  Thread (sub, col) holds float4 column col of the head's o for
  // splits sub * per .. sub * per + per - 1 (per from the split count, so the grouping does not
  // depend on the position), all requested at once; the splits' maxima and sums go to LDS, one
  // wave forms the weights (lanes = splits), each thread sums its splits in order, and the
  // sub-sums are added in sub order.  With EAGER the records are requested before the position is
  // known (every record is in bounds; those of inactive splits are never used).
  constexpr int cols = kSplitHd / 4, tpc = kSplitThreads / cols;
  const int per = (a.splits + tpc - 1) / tpc;
  const int col = t % cols, sub = t / cols;
  double* cl = reinterpret_cast<double*>(sm);                 // [splits] sums
  float* cw = reinterpret_cast<float*>(cl + kSplitMaxSplits);  // [splits] maxima, then weights
  float4* cred = reinterpret_cast<float4*>(cw + kSplitMaxSplits);  // [tpc][cols] sub-sums
  float* cinv = reinterpret_cast<float*>(cred + kSplitThreads);    // 1 / sum_j w_j l_j
  float4 ov[kSplitPerThread];
  auto fetch = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kSplitPerThread; ++q) {
      const int sj = sub * per + q;
      if (q < per && sj < a.splits)
        ov[q] = reinterpret_cast<const float4*>(recs + static_cast<long>(sj) * kSplitRec + hh * kSplitHd)[col];
    }
  };
  float mv = 0.0f;
  double lv = 0.0;
  auto fetch_ml = [&]() __attribute__((always_inline)) {
    if (t < a.splits) {
      const float* rec = recs + static_cast<long>(t) * kSplitRec;
      mv = rec[kSplitMaxHpg * kSplitHd + hh];
      lv = reinterpret_cast<const double*>(rec + kSplitMaxHpg * kSplitHd + kSplitMaxHpg)[hh];
    }
  };
  const int pos_v = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.pos_dev, 4u), 0u, 0u, 0);
  if (EAGER) {
    fetch_ml();
    fetch();
  }
  const int n_act = (__builtin_amdgcn_readfirstlane(pos_v) + a.span) / a.span;  // ceil((pos + 1) / span)
  if (n_act == 1) return;  // the split kernel wrote ctx
  if (!EAGER) {
    fetch_ml();
    fetch();
  }
  if (t < kWave) {  // the weights: lane = split
    const float m = t < n_act ? mv : -INFINITY;
    const float M = wave_max_dpp(m);
    const float w = t < n_act ? expf(m - M) : 0.0f;
    const double L = wave_sum_d_dpp(t < n_act ? lv * static_cast<double>(w) : 0.0);
    cw[t] = w;
    if (t == 0) cinv[0] = static_cast<float>(1.0 / L);
  }
  __syncthreads();
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int q = 0; q < kSplitPerThread; ++q) {
    const int sj = sub * per + q;
    if (q < per && sj < n_act) {
      const float w = cw[sj];
      acc.x += ov[q].x * w;
      acc.y += ov[q].y * w;
      acc.z += ov[q].z * w;
      acc.w += ov[q].w * w;
    }
  }
  cred[sub * cols + col] = acc;
  __syncthreads();
  if (sub == 0) {
    float4 r = cred[col];
    for (int k = 1; k < tpc; ++k) {
      const float4 v = cred[k * cols + col];
      r.x += v.x;
      r.y += v.y;
      r.z += v.z;
      r.w += v.w;
    }
    const float iv = cinv[0];
    r.x *= iv;
    r.y *= iv;
    r.z *= iv;
    r.w *= iv;
    reinterpret_cast<float4*>(out)[col] = r;
  }
}

// Prefill, step 1: every row r = (sequence b, chunk index i) at position p = *pos_dev + i gets RoPE
// on each query head in place and on each key head, and its roped key and its value row are
// written into the cache at p (the decode kernel's rotation, operation for operation).
__global__ __launch_bounds__(kAttnThreads) void rope_store_kernel(PrefillArgs a) {
  const int r = blockIdx.x, b = r / a.n, p = *a.a.pos_dev + r % a.n;
  const int hd = a.a.hd, half = hd / 2, kvd = a.a.KV * hd;
  const float* cr = a.a.cos_t + static_cast<long>(p) * half;
  const float* sr = a.a.sin_t + static_cast<long>(p) * half;
  float* q = const_cast<float*>(a.a.q) + static_cast<long>(r) * a.a.ldq;
  for (int idx = threadIdx.x; idx < a.a.H * half; idx += blockDim.x) {
    const int j = idx % half;
    float* qh = q + (idx / half) * hd;
    const float qa = qh[j], qb = qh[j + half];
    qh[j] = qa * cr[j] - qb * sr[j];
    qh[j + half] = qb * cr[j] + qa * sr[j];
  }
  const float* k = a.a.knew + static_cast<long>(r) * kvd;
  const float* v = a.a.vnew + static_cast<long>(r) * kvd;
  float* kw = a.a.kcache + (static_cast<long>(b) * a.a.max_seq + p) * kvd;
  float* vw = a.a.vcache + (static_cast<long>(b) * a.a.max_seq + p) * kvd;
  for (int idx = threadIdx.x; idx < a.a.KV * half; idx += blockDim.x) {
    const int j = idx % half, o = (idx / half) * hd;
    const float ka = k[o + j], kb = k[o + j + half];
    kw[o + j] = ka * cr[j] - kb * sr[j];
    kw[o + j + half] = kb * cr[j] + ka * sr[j];
  }
  for (int idx = threadIdx.x; idx < kvd; idx += blockDim.x) vw[idx] = v[idx];
}

// Prefill, step 2: one (query head, row) per workgroup over positions 0 .. p, all from the cache.
__global__ __launch_bounds__(kAttnThreads) void prefill_attention_kernel(PrefillArgs a) {
  extern __shared__ float sm[];
  const int h = blockIdx.x, r = blockIdx.y, b = r / a.n, p = *a.a.pos_dev + r % a.n;
  const int hd = a.a.hd, g = h / (a.a.H / a.a.KV), kvd = a.a.KV * hd;
  float* qs = sm;
  float* rows = sm + 3 * hd;
  float* sc = rows + kAttnChunk * row_ld(hd);
  double* red = reinterpret_cast<double*>(sc + ((a.a.max_seq + 1) & ~1));
  const float* q = a.a.q + static_cast<long>(r) * a.a.ldq + h * hd;
  for (int i = threadIdx.x; i < hd; i += blockDim.x) qs[i] = q[i];
  __syncthreads();
  const float* kc = a.a.kcache + (static_cast<long>(b) * a.a.max_seq) * kvd + g * hd;
  const float* vc = a.a.vcache + (static_cast<long>(b) * a.a.max_seq) * kvd + g * hd;
  attend<false>(qs, rows, sc, red, kc, vc, kvd, nullptr, nullptr, -1, p + 1, hd, a.a.scale,
                a.a.ctx + static_cast<long>(r) * a.a.ldq + h * hd, nullptr);
}

// Prefill, step 2 for long prompts (hd = 64, at most 8 query heads per KV head): workgroup (x, g)
// takes kPfRows consecutive rows of one sequence and KV group g, so each staged 64-position chunk of
// K / V serves every (row, head) pair of the block instead of one.  Thread t owns pair t % 128
// (row t % 128 / hpg, head t % 128 % hpg) with its roped query in registers, and half t / 128 of
// each chunk's positions.  Scores follow kern::dot_f32's order (src/kernels.cpp:27-43).  Two passes
// over the chunks: the row's maximum, then e = float exp(s - max), their double sum (each half in
// position order, then the two halves) and o[d] = sum_t e_t v_t[d] over positions in increasing
// order (thread: its pair, dimensions 32 (t / 128) ..); out = o * float(1 / sum).  The reference
// scales each e by 1 / sum before the p.v sum (src/kernels.cpp:77-92,153-174): the results differ
// by that rounding.  Rows, chunk rows past the block's last position and positions past a row's
// own take no part (zero K / V rows, e = 0).
constexpr int kPfRows = 16, kPfChunk = 64, kPfLd = 68, kPfPairs = 128, kPfPsLd = 65;
constexpr int kPfTileFrom = 128;  // positions per sequence in a launch from which the tiled kernel runs

size_t prefill_tile_lds_bytes() {
  return (2 * kPfChunk * kPfLd + kPfPairs * kPfPsLd + 2 * kPfPairs) * sizeof(float) + 2 * kPfPairs * sizeof(double);
}

__global__ __launch_bounds__(256) void prefill_tile_kernel(PrefillArgs pa) {
#pragma clang fp contract(off)
  const AttnArgs& a = pa.a;
  extern __shared__ float sm[];
  float* ks = sm;                                           // [64][kPfLd] K rows of the chunk
  float* vs = ks + kPfChunk * kPfLd;                        // [64][kPfLd] V rows
  float* ps = vs + kPfChunk * kPfLd;                        // [128][kPfPsLd] exponentials of the chunk
  float* mx2 = ps + kPfPairs * kPfPsLd;                     // [2][128] maxima per half
  double* l2 = reinterpret_cast<double*>(mx2 + 2 * kPfPairs);  // [2][128] sums per half
  const int nb = (pa.n + kPfRows - 1) / kPfRows;
  const int b = blockIdx.x / nb, i0 = (blockIdx.x % nb) * kPfRows, g = blockIdx.y, t = threadIdx.x;
  const int hpg = a.H / a.KV, kvd = a.KV * 64;
  const int pair = t & (kPfPairs - 1), half = t >> 7;
  const int il = pair / hpg, hh = pair - il * hpg, i = i0 + il;
  const bool active = il < kPfRows && i < pa.n;
  const int pos0 = *a.pos_dev;
  const int prow = pos0 + i, plast = pos0 + min(i0 + kPfRows, pa.n) - 1;
  const long r = static_cast<long>(b) * pa.n + i;
  float q[64];
  if (active) {
    const float4* qp = reinterpret_cast<const float4*>(a.q + r * a.ldq + (g * hpg + hh) * 64);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float4 v = qp[k];
      q[4 * k] = v.x;
      q[4 * k + 1] = v.y;
      q[4 * k + 2] = v.z;
      q[4 * k + 3] = v.w;
    }
  }
  const float* kc = a.kcache + static_cast<long>(b) * a.max_seq * kvd + g * 64;
  const float* vc = a.vcache + static_cast<long>(b) * a.max_seq * kvd + g * 64;
  auto stage = [&](float* dst, const float* src, int c0) {
    for (int idx = t; idx < kPfChunk * 16; idx += 256) {
      const int rr = idx >> 4, cc = idx & 15;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (c0 + rr <= plast) v = reinterpret_cast<const float4*>(src + static_cast<long>(c0 + rr) * kvd)[cc];
      reinterpret_cast<float4*>(dst + rr * kPfLd)[cc] = v;
    }
  };
  auto score = [&](int rr) -> float {
    const float* kr = ks + rr * kPfLd;
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f, p4 = 0.0f, p5 = 0.0f, p6 = 0.0f, p7 = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float4 ka = *reinterpret_cast<const float4*>(kr + 8 * m);
      const float4 kb = *reinterpret_cast<const float4*>(kr + 8 * m + 4);
      p0 += q[8 * m] * ka.x;
      p1 += q[8 * m + 1] * ka.y;
      p2 += q[8 * m + 2] * ka.z;
      p3 += q[8 * m + 3] * ka.w;
      p4 += q[8 * m + 4] * kb.x;
      p5 += q[8 * m + 5] * kb.y;
      p6 += q[8 * m + 6] * kb.z;
      p7 += q[8 * m + 7] * kb.w;
    }
    return (((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7))) * a.scale;
  };
  const int nchunks = plast / kPfChunk + 1;
  // pass 1: each row's maximum
  float m = -INFINITY;
  for (int c = 0; c < nchunks; ++c) {
    stage(ks, kc, c * kPfChunk);
    __syncthreads();
    if (active) {
      for (int j = 0; j < 32; ++j) {
        const int rr = 32 * half + j;
        if (c * kPfChunk + rr <= prow) m = fmaxf(m, score(rr));
      }
    }
    __syncthreads();
  }
  mx2[half * kPfPairs + pair] = m;
  __syncthreads();
  const float M = fmaxf(mx2[pair], mx2[kPfPairs + pair]);
  // pass 2: exponentials, their sum and the unnormalised p.v
  double l = 0.0;
  float o[32];
#pragma unroll
  for (int d = 0; d < 32; ++d) o[d] = 0.0f;
  for (int c = 0; c < nchunks; ++c) {
    stage(ks, kc, c * kPfChunk);
    stage(vs, vc, c * kPfChunk);
    __syncthreads();
    for (int j = 0; j < 32; ++j) {
      const int rr = 32 * half + j;
      float e = 0.0f;
      if (active && c * kPfChunk + rr <= prow) {
        e = expf(score(rr) - M);
        l += static_cast<double>(e);
      }
      ps[pair * kPfPsLd + rr] = e;
    }
    __syncthreads();
    if (active) {
      for (int rr = 0; rr < kPfChunk; ++rr) {
        const float e = ps[pair * kPfPsLd + rr];
        const float* vr = vs + rr * kPfLd + 32 * half;
#pragma unroll
        for (int d = 0; d < 32; d += 4) {
          const float4 v = *reinterpret_cast<const float4*>(vr + d);
          o[d] += e * v.x;
          o[d + 1] += e * v.y;
          o[d + 2] += e * v.z;
          o[d + 3] += e * v.w;
        }
      }
    }
    __syncthreads();
  }
  l2[half * kPfPairs + pair] = l;
  __syncthreads();
  if (!active) return;
  const float inv = static_cast<float>(1.0 / (l2[pair] + l2[kPfPairs + pair]));
  float* out = a.ctx + r * a.ldq + (g * hpg + hh) * 64 + 32 * half;
#pragma unroll
  for (int d = 0; d < 32; d += 4) {
    float4 v;
    v.x = o[d] * inv;
    v.y = o[d + 1] * inv;
    v.z = o[d + 2] * inv;
    v.w = o[d + 3] * inv;
    reinterpret_cast<float4*>(out + d)[0] = v;
  }
}

// x[r] = row hist[b][*pos_dev + i] of the embedding table for every prefill row r = (b, i).
__global__ void embed_rows_kernel(const uint8_t* __restrict__ W, int qtype, long rows, long cols, long rb,
                                  const int32_t* __restrict__ hist, long hist_ld, const int32_t* __restrict__ pos_dev,
                                  int n, float* __restrict__ out, long ldo) {
  const int r = blockIdx.y, b = r / n, p = *pos_dev + r % n;
  const int32_t id = hist[b * hist_ld + p];
  const bool ok = id >= 0 && id < rows;
  const uint8_t* row = W + (ok ? id : 0) * rb;
  for (long c = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; c < cols;
       c += static_cast<long>(gridDim.x) * blockDim.x) {
    out[r * ldo + c] = ok ? decode_elem(row, qtype, c) : __int_as_float(0x7FC00000);
  }
}

__global__ void advance_by_kernel(int32_t* pos_dev, int n) { *pos_dev += n; }

// out[b] = w * (x[b] * rsqrt(mean(x[b]^2) + eps)) (kern::rmsnorm).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float eps, int n, long ld, float* __restrict__ out) {
  __shared__ double red[4];
  const float* xb = x + blockIdx.x * ld;
  double ss = 0.0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ss += static_cast<double>(xb[i]) * static_cast<double>(xb[i]);
  ss = wave_sum_d_dpp(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const double tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(n) + static_cast<double>(eps)));
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[blockIdx.x * ld + i] = w[i] * (xb[i] * inv);
}

// After a token is picked at position p for every sequence: it becomes the input at p + 1, joins
// the history, lands in the output list at p - (n_prompt - 1), and the position advances.
__global__ void finish_step_kernel(const int32_t* __restrict__ next, int batch, int32_t* hist, long hist_ld,
                                   int32_t* hist_len, int32_t* out, long out_ld, const int32_t* n_prompt_dev,
                                   int32_t* pos_dev, const double* eos_p, double* out_eos) {
  const int p = *pos_dev;
  const int k = p - (*n_prompt_dev - 1);
  for (int b = threadIdx.x; b < batch; b += blockDim.x) {
    const int32_t tok = next[b];
    if (p + 1 < hist_ld) hist[b * hist_ld + p + 1] = tok;
    hist_len[b] = p + 2 < hist_ld ? p + 2 : static_cast<int32_t>(hist_ld);
    if (k >= 0 && k < out_ld) {
      out[b * out_ld + k] = tok;
      if (out_eos != nullptr) out_eos[b * out_ld + k] = eos_p[b];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *pos_dev = p + 1;
}

__global__ void advance_kernel(int32_t* pos_dev) { *pos_dev += 1; }

// dst[r][c] = src[r][c] for r < rows, c < n (4-byte words, row strides lds / ldd): touches exactly
// the rows' n words, nothing of the stride gaps.
__global__ __launch_bounds__(256) void copy_rows_kernel(const uint32_t* __restrict__ src, long lds,
                                                        uint32_t* __restrict__ dst, long ldd, int n, int rows) {
  const int r = blockIdx.y;
  if (r >= rows) return;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < n; c += gridDim.x * blockDim.x)
    dst[r * ldd + c] = src[r * lds + c];
}

}  // namespace

int launch_embed_at(const ef_hip_weight_s* W, const int32_t* hist, long hist_ld, const int32_t* pos_dev, int batch,
                    float* out, long ldo, hipStream_t s, const float* cos_t, const float* sin_t, int half,
                    float* rope_now, const AEmit* em) {
  EFH_CHECK(em == nullptr || !em->on() || (W->cols % 32 == 0 && static_cast<int>(W->cols / 32) == em->nb),
            "embed_at: staging needs cols % 32 == 0 and the product's K");
  const unsigned gx = static_cast<unsigned>(std::min<size_t>((W->cols + 255) / 256, 16));
  const AEmit e = em != nullptr ? *em : AEmit{};
  hipLaunchKernelGGL(embed_at_kernel, dim3(gx, batch), dim3(256), 0, s, W->dev, W->qtype, static_cast<long>(W->rows),
                     static_cast<long>(W->cols), static_cast<long>(W->row_bytes), hist, hist_ld, pos_dev, out, ldo,
                     cos_t, sin_t, half, rope_now, e);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

size_t attention_lds_bytes(int hd, int max_seq) {
  return (3 * static_cast<size_t>(hd) + static_cast<size_t>(kAttnChunk) * row_ld(hd) + vrows_offset(max_seq)) *
         sizeof(float);
}

int launch_prefill_attention(const PrefillArgs& a, int rows, hipStream_t s) {
  hipLaunchKernelGGL(rope_store_kernel, dim3(rows), dim3(kAttnThreads), 0, s, a);
  EFH_HIP(hipGetLastError());
  // long prompts (a launch of kPfTileFrom or more positions per sequence): the tiled kernel
  const int hpg = a.a.KV > 0 ? a.a.H / a.a.KV : 0;
  const char* forced = std::getenv("EF_HIP_PREFILL_ATTENTION");
  const bool tiled_ok = a.a.hd == 64 && a.a.H % a.a.KV == 0 && hpg >= 1 && hpg * kPfRows <= kPfPairs &&
                        a.a.ldq % 4 == 0;
  // EF_HIP_PREFILL_ATTENTION=tiled / rows forces either kernel (tests)
  const bool force_rows = forced != nullptr && std::strcmp(forced, "rows") == 0;
  const bool force_tiled = forced != nullptr && std::strcmp(forced, "tiled") == 0;
  if (tiled_ok && !force_rows && (force_tiled || a.n >= kPfTileFrom)) {
    EFH_CHECK(rows % a.n == 0, "prefill attention: rows must be sequences x positions");
    const int nb = (a.n + kPfRows - 1) / kPfRows;
    hipLaunchKernelGGL(prefill_tile_kernel, dim3((rows / a.n) * nb, a.a.KV), dim3(256), prefill_tile_lds_bytes(), s,
                       a);
    EFH_HIP(hipGetLastError());
    return EF_HIP_OK;
  }
  const size_t lds = attention_lds_bytes(a.a.hd, a.a.max_seq);
  hipLaunchKernelGGL(prefill_attention_kernel, dim3(a.a.H, rows), dim3(kAttnThreads), lds, s, a);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_embed_rows(const ef_hip_weight_s* W, const int32_t* hist, long hist_ld, const int32_t* pos_dev, int n,
                      int rows, float* out, long ldo, hipStream_t s) {
  const unsigned gx = static_cast<unsigned>(std::min<size_t>((W->cols + 255) / 256, 16));
  hipLaunchKernelGGL(embed_rows_kernel, dim3(gx, rows), dim3(256), 0, s, W->dev, W->qtype, static_cast<long>(W->rows),
                     static_cast<long>(W->cols), static_cast<long>(W->row_bytes), hist, hist_ld, pos_dev, n, out, ldo);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_advance_by(int32_t* pos_dev, int n, hipStream_t s) {
  hipLaunchKernelGGL(advance_by_kernel, dim3(1), dim3(1), 0, s, pos_dev, n);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

size_t attention_group_lds_bytes(int hpg, int hd, int max_seq) {
  return (static_cast<size_t>(hpg + 2) * hd + 2 * static_cast<size_t>(kAttnChunk) * row_ld(hd) +
          static_cast<size_t>(hpg) * ((max_seq + 1) & ~1) + hpg) *
         sizeof(float);
}

// EF_HIP_ATTENTION=head / group forces a decode attention kernel (where the group kernel applies);
// read at every launch, so an engine created after a change captures the new choice.
int attention_choice() {
  const char* v = std::getenv("EF_HIP_ATTENTION");
  if (v == nullptr) return 0;
  if (std::strcmp(v, "head") == 0) return 1;
  if (std::strcmp(v, "split") == 0) return 4;
  if (std::strcmp(v, "group") == 0) return 2;
  if (std::strcmp(v, "wave") == 0) return 3;
  return 0;
}

bool attention_split_plan(int H, int KV, int hd, int max_seq, int batch, int* splits, int* span, size_t* part_floats) {
  *splits = 1;
  *span = max_seq;
  *part_floats = 0;
  if (hd != kSplitHd || KV < 1 || H % KV != 0 || H / KV > kSplitMaxHpg || max_seq <= kSplitRows ||
      attention_choice() == 1 || attention_choice() == 2 || attention_choice() == 3)
    return false;
  const long cap = static_cast<long>(kSplitRows) * split_max(H / KV);
  const int sp = static_cast<int>(((max_seq + cap - 1) / cap) * kSplitRows);
  const size_t lim = std::max<size_t>(ctx().lds_per_block, 65536);
  if (attention_split_lds_bytes(H / KV, sp) > lim) return false;
  *span = sp;
  *splits = (max_seq + sp - 1) / sp;
  *part_floats = static_cast<size_t>(batch) * KV * *splits * kSplitRec;
  return true;
}

// Many sequences: one workgroup per (KV group, sequence) when that fills the chip (or is forced)
// and the group's scores fit in LDS.
bool attention_uses_group(const AttnArgs& a, int batch) {
  const size_t lim = std::max<size_t>(ctx().lds_per_block, 65536);
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  const int hpg = a.H / a.KV, choice = attention_choice();
  const size_t glds = attention_group_lds_bytes(hpg, a.hd, a.max_seq);
  const bool group_ok = hpg >= 2 && a.hd % 8 == 0 && a.hd * kAttnChunk <= 4 * kGroupPreSlots * kGroupThreads &&
                        hpg * a.hd <= kGroupMaxOut * kGroupThreads && glds <= lim;
  return group_ok && (choice == 2 || (choice == 0 && static_cast<long>(a.KV) * batch >= cus / 2));
}

int launch_attention(const AttnArgs& a, int batch, hipStream_t s) {
  const size_t lim = std::max<size_t>(ctx().lds_per_block, 65536);
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  const int choice = attention_choice();
  if (attention_uses_group(a, batch)) {
    const int hpg = a.H / a.KV;
    EFH_CHECK(!a.em.on() || (hpg * a.hd) % 32 == 0, "attention: staging needs H / KV * hd % 32 == 0");
    const size_t glds = attention_group_lds_bytes(hpg, a.hd, a.max_seq);
    hipLaunchKernelGGL(attention_group_kernel, dim3(a.KV, batch), dim3(kGroupThreads), glds, s, a);
    EFH_HIP(hipGetLastError());
    return EF_HIP_OK;
  }
  EFH_CHECK(!a.em.on(), "attention: only the KV-group kernel stages its output as tables");
  if (a.part != nullptr && a.rope_now != nullptr) {
    EFH_CHECK(a.hd == kSplitHd && a.H % a.KV == 0 && a.H / a.KV <= kSplitMaxHpg && a.span % kSplitRows == 0 &&
                  static_cast<long>(a.splits) * a.span >= a.max_seq && (a.splits - 1) * a.span < a.max_seq &&
                  a.splits <= split_max(a.H / a.KV),
              "attention: position split does not fit the shape");
    // the rows of every split requested before the position is known when that costs at most
    // 128 workgroups' worth (about 4 MB) of reads at short positions; then each (split, group)
    // also splits its query heads over two workgroups (both stage the same rows) so that the
    // launch reaches every CU
    const bool eager = static_cast<long>(a.splits) * a.KV * batch <= 128;
    AttnArgs sa = a;
    const int hpg = a.H / a.KV, parts = eager && hpg % 2 == 0 ? 2 : 1;
    sa.split_hpw = hpg / parts;
    const size_t lds = attention_split_lds_bytes(sa.split_hpw, a.span);
    if (eager) {
      hipLaunchKernelGGL(attention_split_kernel<true>, dim3(a.splits, a.KV * parts, batch), dim3(kSplitThreads), lds, s,
                         sa);
    } else {
      hipLaunchKernelGGL(attention_split_kernel<false>, dim3(a.splits, a.KV * parts, batch), dim3(kSplitThreads), lds,
                         s, sa);
    }
    EFH_HIP(hipGetLastError());
    if (eager) {
      hipLaunchKernelGGL(attention_combine_kernel<true>, dim3(a.H, batch), dim3(kSplitThreads), kCombineLds, s, a);
    } else {
      hipLaunchKernelGGL(attention_combine_kernel<false>, dim3(a.H, batch), dim3(kSplitThreads), kCombineLds, s, a);
    }
    EFH_HIP(hipGetLastError());
    return EF_HIP_OK;
  }
  // hd = 64 with the step's RoPE row: one wave per (head, sequence), unless another kernel is forced
  if (a.hd == kWaveHd && a.rope_now != nullptr && a.H % a.KV == 0 && choice != 1 && choice != 2) {
    const size_t wlds = (2 * static_cast<size_t>(kWaveHd) + static_cast<size_t>(a.max_seq)) * sizeof(float);
    if (wlds <= lim) {
      hipLaunchKernelGGL(attention_wave_kernel, dim3(a.H, batch), dim3(kWave), wlds, s, a);
      EFH_HIP(hipGetLastError());
      return EF_HIP_OK;
    }
  }
  // With few workgroups (latency-bound: a small batch) the decode kernel prefetches the first
  // chunk's K / V rows, stages the V rows in a second LDS buffer and stages every later chunk with
  // as many rows as the LDS holds (one round trip per chunk); with many, the lighter kernel keeps
  // more workgroups resident.
  AttnArgs b = a;
  b.chunk = kAttnChunk;
  size_t lds = attention_lds_bytes(a.hd, a.max_seq);
  const size_t ld = row_ld(a.hd), vrows = static_cast<size_t>(kAttnChunk) * ld * sizeof(float);
  b.pre_vrows = lds + vrows <= lim && static_cast<long>(a.H) * batch <= 2L * cus ? 1 : 0;
  if (b.pre_vrows) {
    lds += vrows;
    // large chunks only when every workgroup runs in one round (they cost occupancy)
    const size_t base = lds - static_cast<size_t>(stage_floats(a.hd, kAttnChunk)) * sizeof(float);
    const size_t group_bytes = static_cast<size_t>(4 * a.hd + 4) * sizeof(float);
    const long want = std::min<long>(a.max_seq - kAttnChunk, static_cast<long>((lim - base) / group_bytes) * 4);
    if (a.hd == kDmaHd && static_cast<long>(a.H) * batch <= cus && want >= 2 * kAttnChunk) {
      b.chunk = static_cast<int>((want + 3) & ~3L);
      if (base + static_cast<size_t>(stage_floats(a.hd, b.chunk)) * sizeof(float) > lim) b.chunk -= 4;
      lds = base + static_cast<size_t>(stage_floats(a.hd, b.chunk)) * sizeof(float);
      hipLaunchKernelGGL((attention_kernel<true, true>), dim3(a.H, batch), dim3(kAttnThreads), lds, s, b);
    } else {
      hipLaunchKernelGGL((attention_kernel<true, false>), dim3(a.H, batch), dim3(kAttnThreads), lds, s, b);
    }
  } else {
    hipLaunchKernelGGL((attention_kernel<false, false>), dim3(a.H, batch), dim3(kAttnThreads), lds, s, b);
  }
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_rmsnorm(const float* x, const float* w, float eps, int n, long ld, int batch, float* out, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(batch), dim3(256), 0, s, x, w, eps, n, ld, out);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_finish_step(const int32_t* next, int batch, int32_t* hist, long hist_ld, int32_t* hist_len, int32_t* out,
                       long out_ld, const int32_t* n_prompt_dev, int32_t* pos_dev, hipStream_t s, const double* eos_p,
                       double* out_eos) {
  hipLaunchKernelGGL(finish_step_kernel, dim3(1), dim3(256), 0, s, next, batch, hist, hist_ld, hist_len, out, out_ld,
                     n_prompt_dev, pos_dev, eos_p, out_eos);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_copy_rows(const void* src, long lds, void* dst, long ldd, int n, int rows, hipStream_t s) {
  if (n <= 0 || rows <= 0) return EF_HIP_OK;
  const unsigned gx = static_cast<unsigned>(std::min(16, (n + 255) / 256));
  hipLaunchKernelGGL(copy_rows_kernel, dim3(gx, rows), dim3(256), 0, s, static_cast<const uint32_t*>(src), lds,
                     static_cast<uint32_t*>(dst), ldd, n, rows);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_advance(int32_t* pos_dev, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, pos_dev);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

}  // namespace efh
