// Packed Q4_0 / Q8_0 GEMV for decode (batch of independent FP32 activation vectors).
//
// Layout in HBM: the reference's row-major [rows][cols/32] array of 18-byte (Q4_0) or 34-byte
// (Q8_0) blocks, read in place (include/ef/quant.h:22-35).  When cols % 64 == 0 every row is a
// whole number of 36 / 68-byte block PAIRS starting 4-byte aligned, so a lane owns one pair and
// reads it with dword-aligned vector loads; the 2-byte misalignment of the first block's codes is
// undone in registers with v_alignbyte.  Other widths take a generic one-block-per-lane path.
//
// A workgroup (4 waves) stages the activation vector (optionally RMS-normalised, kern::rmsnorm
// order) in LDS once, in 64-float slots padded to 68 floats so lanes reading different pairs hit
// different banks, plus per-block sums of x.  Lanes form groups of G (8/16/32) that share a row;
// each lane walks the row's pairs with stride G, keeps R rows in flight (x read from LDS once per
// pair for R rows), and the group reduces with cross-lane shuffles.
//
// Numerics: codes are converted unsigned (v_cvt_f32_ubyteN) and the bias folded per block:
// sum_j (c_j - 8) x_j = sum_j c_j x_j - 8 * sum_j x_j (Q4_0); Q8_0 codes convert signed.  Each
// block's partial sum is scaled by its fp16 d (exact widening) and accumulated in FP32.  The
// order differs from the reference's CPU kernels (src/qkernels.cpp:39-65, 131-180) only by
// rounding; the result is deterministic for a given shape.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>

#include "gemv.h"
#include "qdot.h"

namespace efh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxJobs = 4;
constexpr size_t kMaxCols = 14336;  // staged x + block sums stay under 64 KB of LDS

struct JobDev {
  const uint8_t* W;
  const uint8_t* W2;
  const float* x;
  float* y;
  int rows;
  int qtype;
  int rows_per_tile;
  int tile_begin;
  int row_bytes;
  long ldx, ldy;
};

struct Args {
  JobDev job[kMaxJobs];
  int n_jobs;
  int K;
  const float* norm_w;
  float eps;
  // LDS layout of the DMA path (byte offsets from the dynamic LDS base)
  uint32_t raw_x_off, raw_nw_off, w_off, w_stride;
};

// ---- staging of x in LDS ------------------------------------------------------------------------
// lds_x: K/64 slots of kSlot floats (a partial last slot for K % 64 == 32); lds_xs: K/32 block sums.
// Thread t owns the float4s at 4t + 1024k.  The first kXRegs of them (and their norm weights) are
// requested by xload_issue() before the caller issues its weight loads: vector-memory loads retire
// in order on CDNA, so loads requested after the weights could only be consumed once every weight
// load had landed.  xload_finish() then forms the RMSNorm, writes LDS and the block sums (formed in
// registers: the 8 consecutive threads that store a 32-float block add their partials with lane
// shuffles).  One barrier without a norm, two with it.
constexpr int kXRegs = 6;  // K <= 6144 staged from registers; the rest is loaded during staging

struct XLoad {
  float4 x[kXRegs];
  float4 w[kXRegs];
};

// x (and the norm weights: a zero-length resource when there is no norm) for K <= kXRegs*1024.
__device__ __forceinline__ void xload_issue(const float* __restrict__ x, const float* __restrict__ nw, int K,
                                            XLoad& r) {
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(K) * 4u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(nw != nullptr ? nw : x, nw != nullptr ? static_cast<uint32_t>(K) * 4u : 0u);
#pragma unroll
  for (int k = 0; k < kXRegs; ++k) r.x[k] = buf_f4(rx, (threadIdx.x * 4u + k * kThreads * 4u) * 4u);
#pragma unroll
  for (int k = 0; k < kXRegs; ++k) r.w[k] = buf_f4(rw, (threadIdx.x * 4u + k * kThreads * 4u) * 4u);
}

__device__ __forceinline__ void store_x4(float4 v, int i, float* lds_x, float* lds_xs) {
  *reinterpret_cast<float4*>(lds_x + (i >> 6) * kSlot + (i & 63)) = v;
  // K % 32 == 0, so the 8 threads of a block are active together and the xor partners stay
  // inside the aligned group of 8.
  const float s = group_sum_dpp<8>((v.x + v.y) + (v.z + v.w));
  if ((threadIdx.x & 7) == 0) lds_xs[i >> 5] = s;
}


__device__ void xload_finish(const float* __restrict__ x, const float* __restrict__ nw, float eps, int K,
                             const XLoad& r, float* lds_x, float* lds_xs, double* red) {
  constexpr int kReg = kXRegs * kThreads * 4;
  float inv = 1.0f;
  if (nw != nullptr) {  // kern::rmsnorm: double sum of squares, inv = float(1 / sqrt(mean + eps))
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < kXRegs; ++k) {
      const int i = threadIdx.x * 4 + k * kThreads * 4;
      if (i < K) ss += sq_d(r.x[k]);
    }
    for (int i = threadIdx.x * 4 + kReg; i < K; i += kThreads * 4) ss += sq_d(*reinterpret_cast<const float4*>(x + i));
    ss = wave_sum_d_dpp(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    inv = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(eps)));
  }
#pragma unroll
  for (int k = 0; k < kXRegs; ++k) {
    const int i = threadIdx.x * 4 + k * kThreads * 4;
    if (i < K) store_x4(nw != nullptr ? norm4(r.x[k], r.w[k], inv) : r.x[k], i, lds_x, lds_xs);
  }
  for (int i = threadIdx.x * 4 + kReg; i < K; i += kThreads * 4) {
    float4 v = *reinterpret_cast<const float4*>(x + i);
    if (nw != nullptr) v = norm4(v, *reinterpret_cast<const float4*>(nw + i), inv);
    store_x4(v, i, lds_x, lds_xs);
  }
  __syncthreads();
}

__device__ void stage_x(const float* __restrict__ x, const float* __restrict__ nw, float eps, int K, float* lds_x,
                        float* lds_xs, double* red) {
  XLoad r;
  xload_issue(x, nw, K, r);
  xload_finish(x, nw, eps, K, r, lds_x, lds_xs, red);
}


// The job owning `tile`, selected with constant indices so the kernel arguments stay in SGPRs.
__device__ __forceinline__ JobDev find_job(const Args& a, int tile) {
  JobDev j = a.job[0];
#pragma unroll
  for (int i = 1; i < kMaxJobs; ++i)
    if (i < a.n_jobs && tile >= a.job[i].tile_begin) j = a.job[i];
  return j;
}

// Body of the fast path for one weight type.  A lane group of G lanes owns R output rows; with the
// SwiGLU epilogue it also owns the matching R up-projection rows, so RR = 2R weight rows share each
// x read from LDS.  Pairs are processed in chunks of G * NPL: lane t holds pairs t, t + G, ...,
// t + (NPL-1) G of the chunk for all RR rows in registers.  The first chunk is requested before x
// is staged, so its HBM latency overlaps the staging.
template <int QT, int EPI, int G, int R, int NPL>
__device__ __forceinline__ void pairs_body(const Args& a, const JobDev& jb, int b, int row0, int nvalid, int t,
                                           float* lds_x, float* lds_xs, double* red) {
  constexpr int PD = PairOf<QT>::PD, PB = PD * 4;
  constexpr int RR = EPI == kEpiSwiglu ? 2 * R : R;
  const int K = a.K, np = K >> 6;
  const size_t rb = static_cast<size_t>(jb.row_bytes);
  // One resource per matrix: rows at or past jb.rows read as zeros.  Pairs past np of a valid row
  // would read the next row, so they are skipped in the dot loop.
  const uint32_t mat_bytes = static_cast<uint32_t>(jb.rows) * static_cast<uint32_t>(rb);
  const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(jb.W, mat_bytes);
  const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(EPI == kEpiSwiglu ? jb.W2 : jb.W, mat_bytes);
  uint32_t buf[NPL][RR][PD];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const uint32_t p = static_cast<uint32_t>(c * (G * NPL) + i * G + t);
#pragma unroll
      for (int r = 0; r < RR; ++r) {
        const __amdgpu_buffer_rsrc_t rs = r < R ? rw1 : rw2;
        const uint32_t off = static_cast<uint32_t>(row0 + r % R) * static_cast<uint32_t>(rb) + p * PB;
#pragma unroll
        for (int k = 0; k + 4 <= PD; k += 4) {
          const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4u * k, 0, kNonTemporal);
          buf[i][r][k] = v.x;
          buf[i][r][k + 1] = v.y;
          buf[i][r][k + 2] = v.z;
          buf[i][r][k + 3] = v.w;
        }
        buf[i][r][PD - 1] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4u * (PD - 1), 0, kNonTemporal);
      }
    }
  };
  const float* xb = jb.x + b * jb.ldx;
  XLoad xr;
  xload_issue(xb, a.norm_w, K, xr);
  load_chunk(0);
  xload_finish(xb, a.norm_w, a.eps, K, xr, lds_x, lds_xs, red);
  float acc[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = 0.0f;
  const int nch = (np + G * NPL - 1) / (G * NPL);
  for (int c = 0; c < nch; ++c) {
    if (c > 0) load_chunk(c);
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int p = c * (G * NPL) + i * G + t;
      if (p < np) pair_dot<QT, RR>(buf[i], lds_x + p * kSlot, lds_xs[2 * p], lds_xs[2 * p + 1], acc);
    }
  }
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = group_sum_dpp<G>(acc[r]);
  if (t != G - 1 || nvalid <= 0) return;  // lane G - 1 holds the group's sums
  float* y = jb.y + b * jb.ldy + row0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nvalid) break;
    if (EPI == kEpiResidual) {
      y[r] = y[r] + acc[r];
    } else if (EPI == kEpiSwiglu) {
      y[r] = silu_f(acc[r]) * acc[R + r];
    } else {
      y[r] = acc[r];
    }
  }
}

// Fast path: cols % 64 == 0.  grid = (tiles, batch).
template <int EPI, int G, int R, int NPL>
__global__ __launch_bounds__(kThreads) void gemv_pairs_kernel(Args a) {
  extern __shared__ float lds[];
  __shared__ double red[kWaves];
  const int np = a.K >> 6;
  float* lds_x = lds;
  float* lds_xs = lds + np * kSlot;
  const int tile = blockIdx.x, b = blockIdx.y;
  const JobDev jb = find_job(a, tile);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int grp = lane / G, t = lane % G;
  const int row0 = (tile - jb.tile_begin) * jb.rows_per_tile + (wave * (kWave / G) + grp) * R;
  const int nvalid = max(0, min(R, jb.rows - row0));
  // Every thread stays to the end: stage_x has block-wide barriers.
  if (jb.qtype == EF_QTYPE_Q4_0) {
    pairs_body<EF_QTYPE_Q4_0, EPI, G, R, NPL>(a, jb, b, row0, nvalid, t, lds_x, lds_xs, red);
  } else {
    pairs_body<EF_QTYPE_Q8_0, EPI, G, R, NPL>(a, jb, b, row0, nvalid, t, lds_x, lds_xs, red);
  }
}

// ---- DMA path: whole rows fetched with coalesced LDS-DMA loads ----------------------------------
// A wave owns RW = (64/G) R consecutive rows of each matrix (gate and up for SwiGLU): RW * row_bytes
// contiguous bytes, fetched as 1 KB buffer_load ... lds instructions (lane l's 16 bytes land at
// base + 16 l), so every HBM request is a fully used, contiguous 1 KB.  The raw activations and
// the norm weights are fetched the same way.  All fetches are issued before anything waits; after
// one wait and a barrier, x is normalised into the padded slots, and each lane reads its block
// pairs from LDS (row stride row_bytes: lanes of a group read pairs 36 / 68 bytes apart, a stride
// co-prime with the bank count).

template <int QT, int EPI, int G, int R>
__device__ __forceinline__ void dma_body(const float* lds_x, const float* lds_xs, const uint8_t* wl, uint32_t wstride,
                                         int np, int rb, int t, int grp, float (&acc)[EPI == kEpiSwiglu ? 2 * R : R]) {
  constexpr int PD = PairOf<QT>::PD, PB = PD * 4;
  constexpr int RR = EPI == kEpiSwiglu ? 2 * R : R;
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = 0.0f;
  for (int p = t; p < np; p += G) {
    uint32_t d[RR][PD];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      const int m = r < R ? 0 : 1;
      lds_pair<QT, RR>(wl + m * wstride + (grp * R + r % R) * rb + p * PB, d, r);
    }
    pair_dot<QT, RR>(d, lds_x + p * kSlot, lds_xs[2 * p], lds_xs[2 * p + 1], acc);
  }
}

template <int EPI, int G, int R, int NW>
__global__ __launch_bounds__(NW * kWave) void gemv_dma_kernel(Args a) {
  constexpr int NT = NW * kWave;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ double red[NW];
  constexpr int RW = (kWave / G) * R;
  constexpr int RR = EPI == kEpiSwiglu ? 2 * R : R;
  const int K = a.K, np = K >> 6;
  uint8_t* lb = reinterpret_cast<uint8_t*>(lds);
  float* lds_x = lds;
  float* lds_xs = lds + np * kSlot;
  const float* raw_x = reinterpret_cast<const float*>(lb + a.raw_x_off);
  const float* raw_nw = reinterpret_cast<const float*>(lb + a.raw_nw_off);
  const int tile = blockIdx.x, b = blockIdx.y;
  const JobDev jb = find_job(a, tile);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x & (kWave - 1);
  const uint32_t rb = static_cast<uint32_t>(jb.row_bytes);
  const int wrow0 = (tile - jb.tile_begin) * jb.rows_per_tile + wave * RW;
  uint8_t* wl = lb + a.w_off + static_cast<uint32_t>(wave) * (EPI == kEpiSwiglu ? 2u : 1u) * a.w_stride;

  // 1. every fetch of the workgroup: this wave's quarter of x (and of the norm weights), then its
  //    weight rows; the staging below waits for x only, the dot products for the rows
  int n_rows_ops;
  {
    const uint32_t xq = static_cast<uint32_t>(K) * 4u / NW;  // bytes of x per wave (a multiple of 16)
    const float* xb = jb.x + b * jb.ldx;
    dma_span<0>(make_rsrc(xb, static_cast<uint32_t>(K) * 4u), wave * xq, lb + a.raw_x_off + wave * xq, xq, lane);
    if (a.norm_w != nullptr)
      dma_span<0>(make_rsrc(a.norm_w, static_cast<uint32_t>(K) * 4u), wave * xq, lb + a.raw_nw_off + wave * xq, xq,
                  lane);
    const uint32_t mat_bytes = static_cast<uint32_t>(jb.rows) * rb;
    const uint32_t region = (static_cast<uint32_t>(RW) * rb + 15u) & ~15u;
    const uint32_t src = static_cast<uint32_t>(wrow0) * rb;  // rows past the end read as zeros
    dma_span<kNonTemporal>(make_rsrc(jb.W, mat_bytes), src, wl, region, lane);
    if (EPI == kEpiSwiglu) dma_span<kNonTemporal>(make_rsrc(jb.W2, mat_bytes), src, wl + a.w_stride, region, lane);
    n_rows_ops = static_cast<int>((region + 1023u) / 1024u) * (EPI == kEpiSwiglu ? 2 : 1);
  }
  wait_vmcnt_at_most(n_rows_ops);
  // every wave's part of x is in LDS: a bare barrier (a __syncthreads fence would wait for the
  // weight rows too)
  asm volatile("s_barrier" ::: "memory");

  // 2. normalise x into the padded slots (+ block sums), while the weight rows are in flight.
  //    K <= 8 NT (every float4 of x in two per thread, read once): x and the norm weights come in
  //    one batch of LDS reads and stay in registers; longer rows loop.
  {
    // K % 32 == 0: the 8 threads of a block are active together, the group sum stays inside
    auto put = [&](int i, float4 v) {
      lds_write4(lds_x + (i >> 6) * kSlot + (i & 63), v);
      const float bs = group_sum_dpp<8>((v.x + v.y) + (v.z + v.w));
      if ((threadIdx.x & 7) == 0) lds_write1(lds_xs + (i >> 5), bs);
    };
    auto norm_inv = [&](double ss) -> float {
      ss = wave_sum_d_dpp(ss);
      if (lane == 0) red[wave] = ss;
      lds_barrier();
      double tot = 0.0;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += red[w];  // waves in order
      return static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(a.eps)));
    };
    if (K <= 2 * NT * 4) {
      const int i0 = threadIdx.x * 4, i1 = i0 + NT * 4;
      const bool h0 = i0 < K, h1 = i1 < K;
      const int j0 = h0 ? i0 : 0, j1 = h1 ? i1 : 0;  // in-range addresses for idle threads
      float4 x0, x1;
      if (a.norm_w != nullptr) {
        float4 w0, w1;
        lds_read4x4(raw_x + j0, raw_x + j1, raw_nw + j0, raw_nw + j1, x0, x1, w0, w1);
        const float inv = norm_inv((h0 ? sq_d(x0) : 0.0) + (h1 ? sq_d(x1) : 0.0));
        x0 = norm4(x0, w0, inv);
        x1 = norm4(x1, w1, inv);
      } else {
        lds_read4x2(raw_x + j0, raw_x + j1, x0, x1);
      }
      if (h0) put(i0, x0);
      if (h1) put(i1, x1);
    } else {
      float inv = 1.0f;
      if (a.norm_w != nullptr) {
        double ss = 0.0;
        for (int i = threadIdx.x * 4; i < K; i += NT * 4) ss += sq_d(lds_read4(raw_x + i));
        inv = norm_inv(ss);
      }
      for (int i = threadIdx.x * 4; i < K; i += NT * 4) {
        float4 v = lds_read4(raw_x + i);
        if (a.norm_w != nullptr) v = norm4(v, lds_read4(raw_nw + i), inv);
        put(i, v);
      }
    }
    __syncthreads();
  }

  // 3. dot products, once this wave's rows have landed (only this wave reads them)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const int grp = lane / G, t = lane % G;
  const int row0 = wrow0 + grp * R;
  const int nvalid = max(0, min(R, jb.rows - row0));
  float acc[RR];
  if (jb.qtype == EF_QTYPE_Q4_0) {
    dma_body<EF_QTYPE_Q4_0, EPI, G, R>(lds_x, lds_xs, wl, a.w_stride, np, static_cast<int>(rb), t, grp, acc);
  } else {
    dma_body<EF_QTYPE_Q8_0, EPI, G, R>(lds_x, lds_xs, wl, a.w_stride, np, static_cast<int>(rb), t, grp, acc);
  }
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = group_sum_dpp<G>(acc[r]);
  if (t != G - 1 || nvalid <= 0) return;  // lane G - 1 holds the group's sums
  float* y = jb.y + b * jb.ldy + row0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nvalid) break;
    if (EPI == kEpiResidual) {
      y[r] = y[r] + acc[r];
    } else if (EPI == kEpiSwiglu) {
      y[r] = silu_f(acc[r]) * acc[R + r];
    } else {
      y[r] = acc[r];
    }
  }
}

// Generic path (any cols % 32 == 0): one wave per row, one block per lane per step, 16-bit
// loads (rows may start 2-byte aligned).  x staged unpadded-in-slots as in the fast path.
__device__ float row_dot_generic(const uint8_t* __restrict__ row, int qtype, int nb, const float* lds_x,
                                 const float* lds_xs, int lane) {
  const int bs = qtype == EF_QTYPE_Q4_0 ? 18 : 34;
  float acc = 0.0f;
  for (int blk = lane; blk < nb; blk += kWave) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(row + static_cast<size_t>(blk) * bs);
    const float d = half_bits_to_float(h[0]);
    const float* xb = lds_x + (blk >> 1) * kSlot + (blk & 1) * 32;
    float s = 0.0f;
    if (qtype == EF_QTYPE_Q4_0) {
      for (int j = 0; j < 8; ++j) {
        const uint32_t v = h[1 + j];
        const uint32_t b0 = v & 0xFFu, b1 = v >> 8;
        s = fmaf(static_cast<float>(b0 & 15u), xb[2 * j], s);
        s = fmaf(static_cast<float>(b0 >> 4), xb[16 + 2 * j], s);
        s = fmaf(static_cast<float>(b1 & 15u), xb[2 * j + 1], s);
        s = fmaf(static_cast<float>(b1 >> 4), xb[16 + 2 * j + 1], s);
      }
      s = fmaf(-8.0f, lds_xs[blk], s);
    } else {
      for (int j = 0; j < 16; ++j) {
        const uint32_t v = h[1 + j];
        s = fmaf(static_cast<float>(static_cast<int8_t>(v & 0xFFu)), xb[2 * j], s);
        s = fmaf(static_cast<float>(static_cast<int8_t>(v >> 8)), xb[2 * j + 1], s);
      }
    }
    acc = fmaf(d, s, acc);
  }
  return wave_sum(acc);
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemv_generic_kernel(Args a) {
  extern __shared__ float lds[];
  __shared__ double red[kWaves];
  const int K = a.K, nb = K >> 5, nslot = (K + 63) >> 6;
  float* lds_x = lds;
  float* lds_xs = lds + nslot * kSlot;
  const int tile = blockIdx.x, b = blockIdx.y;
  const JobDev jb = find_job(a, tile);
  stage_x(jb.x + b * jb.ldx, a.norm_w, a.eps, K, lds_x, lds_xs, red);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int row = (tile - jb.tile_begin) * jb.rows_per_tile + wave;
  if (row >= jb.rows) return;
  const size_t rb = static_cast<size_t>(jb.row_bytes);
  const float v = row_dot_generic(jb.W + row * rb, jb.qtype, nb, lds_x, lds_xs, lane);
  float v2 = 0.0f;
  if (EPI == kEpiSwiglu) v2 = row_dot_generic(jb.W2 + row * rb, jb.qtype, nb, lds_x, lds_xs, lane);
  if (lane != 0) return;
  float* y = jb.y + b * jb.ldy + row;
  if (EPI == kEpiResidual) {
    *y = *y + v;
  } else if (EPI == kEpiSwiglu) {
    *y = silu_f(v) * v2;
  } else {
    *y = v;
  }
}

// ---- launch ---------------------------------------------------------------------------------------
// Pairs per lane per chunk are capped so that RR rows x NPL pairs of Q8_0 data (17 dwords each)
// stay within about 136 VGPRs; larger rows run in several chunks.
template <int EPI, int G, int R>
void* pick_pairs_kernel_n(int npl) {
  constexpr int RR = EPI == kEpiSwiglu ? 2 * R : R;
  constexpr int cap = RR >= 8 ? 1 : (RR >= 4 ? 2 : 4);
  if constexpr (cap >= 4) {
    if (npl >= 4) return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, R, 4>);
  }
  if constexpr (cap >= 2) {
    if (npl >= 2) return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, R, 2>);
  }
  return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, R, 1>);
}

template <int EPI, int G>
void* pick_pairs_kernel_r(int R, int npl) {
  if (R == 4) return pick_pairs_kernel_n<EPI, G, 4>(npl);
  if (R == 2) return pick_pairs_kernel_n<EPI, G, 2>(npl);
  return pick_pairs_kernel_n<EPI, G, 1>(npl);
}

template <int EPI>
void* pick_pairs_kernel(int G, int R, int npl) {
  if (G == 32) return pick_pairs_kernel_r<EPI, 32>(R, npl);
  if (G == 16) return pick_pairs_kernel_r<EPI, 16>(R, npl);
  return pick_pairs_kernel_r<EPI, 8>(R, npl);
}

template <int EPI, int G, int NW>
void* pick_dma_kernel_r(int R) {
  if (R == 4) return reinterpret_cast<void*>(&gemv_dma_kernel<EPI, G, 4, NW>);
  if (R == 2) return reinterpret_cast<void*>(&gemv_dma_kernel<EPI, G, 2, NW>);
  return reinterpret_cast<void*>(&gemv_dma_kernel<EPI, G, 1, NW>);
}

template <int EPI, int NW>
void* pick_dma_kernel_g(int G, int R) {
  if (G == 32) return pick_dma_kernel_r<EPI, 32, NW>(R);
  if (G == 16) return pick_dma_kernel_r<EPI, 16, NW>(R);
  return pick_dma_kernel_r<EPI, 8, NW>(R);
}

template <int EPI>
void* pick_dma_kernel(int G, int R) {
  return pick_dma_kernel_g<EPI, 4>(G, R);
}

}  // namespace


int launch_gemv(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                size_t ldy, hipStream_t stream, void* ws, size_t ws_bytes) {
  EFH_CHECK(n_jobs >= 1 && n_jobs <= kMaxJobs, "gemv: 1..4 jobs per launch");
  EFH_CHECK(batch >= 1 && batch <= 65535, "gemv: batch must be in [1, 65535]");
  EFH_CHECK(epi >= kEpiStore && epi <= kEpiSwiglu, "gemv: unknown epilogue");
  int n_dense = 0;
  for (int j = 0; j < n_jobs; ++j) {
    EFH_CHECK(jobs[j].W && jobs[j].x && jobs[j].y, "gemv: null weight / x / y");
    n_dense += is_dense_qtype(jobs[j].W->qtype) ? 1 : 0;
  }
  if (n_dense > 0) {
    for (int j = 0; j < n_jobs; ++j)
      EFH_CHECK(jobs[j].W->cols == jobs[0].W->cols, "gemv: all jobs of one launch need the same cols");
    if (batch > 1) {
      for (int j = 0; j < n_jobs; ++j) {
        EFH_CHECK((jobs[j].ldx ? jobs[j].ldx : ldx) >= jobs[j].W->cols, "gemv: ldx smaller than cols");
        EFH_CHECK((jobs[j].ldy ? jobs[j].ldy : ldy) >= jobs[j].W->rows, "gemv: ldy smaller than rows");
      }
    }
    // one launch per unquantized type, then one for the packed jobs
    GemvJob group[kMaxJobs];
    for (int qt : {EF_QTYPE_F32, EF_QTYPE_F16, EF_QTYPE_BF16}) {
      int n = 0;
      for (int j = 0; j < n_jobs; ++j)
        if (jobs[j].W->qtype == qt) group[n++] = jobs[j];
      if (n > 0) EFH_RC(launch_gemv_dense(group, n, epi, norm_w, eps, batch, ldx, ldy, stream));
    }
    int n = 0;
    for (int j = 0; j < n_jobs; ++j)
      if (!is_dense_qtype(jobs[j].W->qtype)) group[n++] = jobs[j];
    if (n == 0) return EF_HIP_OK;
    return launch_gemv(group, n, epi, norm_w, eps, batch, ldx, ldy, stream, ws, ws_bytes);
  }
  const size_t K = jobs[0].W ? jobs[0].W->cols : 0;
  EFH_CHECK(K >= 32 && K % 32 == 0 && K <= kMaxCols, "gemv: cols must be a multiple of 32 in [32, 14336]");
  for (int j = 0; j < n_jobs; ++j) {
    const GemvJob& g = jobs[j];
    EFH_CHECK(g.W && g.x && g.y, "gemv: null weight / x / y");
    EFH_CHECK(g.W->qtype == EF_QTYPE_Q4_0 || g.W->qtype == EF_QTYPE_Q8_0, "gemv: weights must be Q4_0 or Q8_0");
    EFH_CHECK(g.W->cols == K, "gemv: all jobs of one launch need the same cols");
    EFH_CHECK(g.W->rows >= 1 && g.W->rows <= (1u << 24), "gemv: rows must be in [1, 2^24]");
    // buffer resources address a matrix with 32-bit byte offsets
    EFH_CHECK(g.W->rows * g.W->row_bytes < (1ull << 32) - (1ull << 20), "gemv: a matrix must be under 4 GiB");
    if (epi == kEpiSwiglu) {
      EFH_CHECK(g.W2 && g.W2->qtype == g.W->qtype && g.W2->rows == g.W->rows && g.W2->cols == K,
                "gemv: swiglu needs gate and up of the same type and shape");
    }
  }
  if (batch > 1) {
    for (int j = 0; j < n_jobs; ++j) {
      EFH_CHECK((jobs[j].ldx ? jobs[j].ldx : ldx) >= K, "gemv: ldx smaller than cols");
      EFH_CHECK((jobs[j].ldy ? jobs[j].ldy : ldy) >= jobs[j].W->rows, "gemv: ldy smaller than rows");
    }
  }
  bool taken = false;
  EFH_RC(launch_gemv_batch(jobs, n_jobs, epi, norm_w, eps, batch, ldx, ldy, stream, &taken));
  if (taken) return EF_HIP_OK;
  EFH_RC(launch_gemv_mfma(jobs, n_jobs, epi, norm_w, eps, batch, ldx, ldy, ws, ws_bytes, stream, &taken));
  if (taken) return EF_HIP_OK;
  Args a{};
  a.n_jobs = n_jobs;
  a.K = static_cast<int>(K);
  a.norm_w = norm_w;
  a.eps = eps;
  const bool fast = K % 64 == 0;
  const int np = static_cast<int>(K / 64);
  int G = np >= 32 ? 32 : (np >= 16 ? 16 : 8);
  const int nmat = epi == kEpiSwiglu ? 2 : 1;
  // LDS of the DMA path for R rows per lane group: x slots + block sums, raw x (+ raw norm
  // weights), then per wave and matrix the wave's RW rows.
  auto dma_layout = [&](int g, int r, int nw, Args* out) -> size_t {
    const size_t rw = static_cast<size_t>(kWave / g) * r;
    size_t wstride = 0;
    for (int j = 0; j < n_jobs; ++j) wstride = std::max(wstride, (rw * jobs[j].W->row_bytes + 15) & ~size_t(15));
    size_t off = ((static_cast<size_t>(np) * kSlot + K / 32) * sizeof(float) + 15) & ~size_t(15);
    const size_t raw_x = off;
    off += K * 4;
    const size_t raw_nw = off;
    if (norm_w != nullptr) off += K * 4;
    const size_t w_off = off;
    off += static_cast<size_t>(nw) * nmat * wstride;
    if (out != nullptr) {
      out->raw_x_off = static_cast<uint32_t>(raw_x);
      out->raw_nw_off = static_cast<uint32_t>(raw_nw);
      out->w_off = static_cast<uint32_t>(w_off);
      out->w_stride = static_cast<uint32_t>(wstride);
    }
    return off;
  };
  constexpr size_t kDmaLdsTarget = 80 * 1024;  // two workgroups per CU
  // Waves per workgroup of the DMA kernel: four.  Eight waves spread the per-workgroup staging over
  // twice the rows but measured slower on MI355X (gate/up 5632x2048: 8.99 us against 8.30 us).
  int nw = 4;
  bool use_dma = fast && dma_layout(G, 1, nw, nullptr) <= kDmaLdsTarget;
  if (!use_dma) nw = kWaves;
  // rows per tile: nw waves x (64/G) groups x R rows.  Register path: R as large as keeps >= 2
  // tiles per CU.  DMA path: the R that gives the busiest CU the fewest rows (rounds of tiles over
  // the CUs x rows per tile), the larger R on a tie (fewer workgroups re-stage x).  q/k/v (2560
  // rows) takes R = 2, 160 tiles of 16 rows, instead of 320 tiles of 8 (64 CUs with two): 90.1 ->
  // 86 us per B = 1 step; lm_head keeps R = 2 (R = 1: 17.8 -> 20.5 us).
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  int R = 1;
  if (fast) {
    size_t best = 0;
    for (int cand : {1, 2, 4}) {
      const size_t per_tile = static_cast<size_t>(nw * (kWave / G) * cand);
      size_t tiles = 0;
      for (int j = 0; j < n_jobs; ++j) tiles += (jobs[j].W->rows + per_tile - 1) / per_tile;
      tiles *= static_cast<size_t>(batch);
      if (!use_dma) {
        if (cand == 1 || tiles >= static_cast<size_t>(2 * cus)) R = cand;
        continue;
      }
      if (cand > 1 && dma_layout(G, cand, nw, nullptr) > kDmaLdsTarget) continue;
      const size_t busiest = (tiles + cus - 1) / cus * per_tile;
      if (best == 0 || busiest <= best) {
        best = busiest;
        R = cand;
      }
    }
  }
  size_t dma_lds = 0;
  if (use_dma) {
    dma_lds = dma_layout(G, R, nw, &a);
    const size_t lim = ctx().lds_per_block > 0 ? ctx().lds_per_block : 65536;
    if (dma_lds > lim) use_dma = false;
  }
  if (!use_dma) nw = kWaves;
  // pairs per lane and chunk of the register path: all of a row's pairs when they fit in four
  int npl = (np + G - 1) / G;
  npl = npl >= 3 ? 4 : npl;
  int tiles = 0;
  for (int j = 0; j < n_jobs; ++j) {
    JobDev& d = a.job[j];
    const ef_hip_weight_s* W = jobs[j].W;
    d.W = W->dev;
    d.W2 = jobs[j].W2 ? jobs[j].W2->dev : nullptr;
    d.x = jobs[j].x;
    d.y = jobs[j].y;
    d.rows = static_cast<int>(W->rows);
    d.qtype = W->qtype;
    d.row_bytes = static_cast<int>(W->row_bytes);
    d.ldx = static_cast<long>(jobs[j].ldx ? jobs[j].ldx : ldx);
    d.ldy = static_cast<long>(jobs[j].ldy ? jobs[j].ldy : ldy);
    d.rows_per_tile = fast ? nw * (kWave / G) * R : kWaves;
    d.tile_begin = tiles;
    tiles += (d.rows + d.rows_per_tile - 1) / d.rows_per_tile;
  }
  const int nslot = static_cast<int>((K + 63) / 64);
  size_t lds_bytes = (static_cast<size_t>(nslot) * kSlot + K / 32) * sizeof(float);
  void* fn = nullptr;
  if (fast && use_dma) {
    fn = epi == kEpiStore ? pick_dma_kernel<kEpiStore>(G, R)
                          : (epi == kEpiResidual ? pick_dma_kernel<kEpiResidual>(G, R)
                                                 : pick_dma_kernel<kEpiSwiglu>(G, R));
    lds_bytes = dma_lds;
  } else if (fast) {
    fn = epi == kEpiStore ? pick_pairs_kernel<kEpiStore>(G, R, npl)
                          : (epi == kEpiResidual ? pick_pairs_kernel<kEpiResidual>(G, R, npl)
                                                 : pick_pairs_kernel<kEpiSwiglu>(G, R, npl));
  } else {
    fn = epi == kEpiStore ? reinterpret_cast<void*>(&gemv_generic_kernel<kEpiStore>)
                          : (epi == kEpiResidual ? reinterpret_cast<void*>(&gemv_generic_kernel<kEpiResidual>)
                                                 : reinterpret_cast<void*>(&gemv_generic_kernel<kEpiSwiglu>));
  }
  void* params[] = {&a};
  EFH_HIP(hipLaunchKernel(fn, dim3(tiles, batch), dim3(nw * kWave), params, lds_bytes, stream));
  return EF_HIP_OK;
}

}  // namespace efh
