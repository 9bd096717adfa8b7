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

#include "gemv.h"

namespace efh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxJobs = 4;
constexpr int kSlot = 68;  // 64 floats of a block pair + 4 floats of bank padding
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
};

// ---- staging of x in LDS ------------------------------------------------------------------------
// lds_x: K/64 slots of kSlot floats (a partial last slot for K % 64 == 32); lds_xs: K/32 block sums.
__device__ void stage_x(const float* __restrict__ x, const float* __restrict__ nw, float eps, int K, float* lds_x,
                        float* lds_xs, double* red) {
  float inv = 1.0f;
  if (nw != nullptr) {  // kern::rmsnorm: double sum of squares, inv = float(1 / sqrt(mean + eps))
    double ss = 0.0;
    for (int i = threadIdx.x * 4; i < K; i += kThreads * 4) {
      const float4 v = *reinterpret_cast<const float4*>(x + i);
      ss += static_cast<double>(v.x) * static_cast<double>(v.x);
      ss += static_cast<double>(v.y) * static_cast<double>(v.y);
      ss += static_cast<double>(v.z) * static_cast<double>(v.z);
      ss += static_cast<double>(v.w) * static_cast<double>(v.w);
    }
    ss = wave_sum_d(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    inv = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(eps)));
  }
  for (int i = threadIdx.x * 4; i < K; i += kThreads * 4) {
    float4 v = *reinterpret_cast<const float4*>(x + i);
    if (nw != nullptr) {  // HF order: w * (x * inv)
      const float4 w = *reinterpret_cast<const float4*>(nw + i);
      v.x = w.x * (v.x * inv);
      v.y = w.y * (v.y * inv);
      v.z = w.z * (v.z * inv);
      v.w = w.w * (v.w * inv);
    }
    *reinterpret_cast<float4*>(lds_x + (i >> 6) * kSlot + (i & 63)) = v;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < K / 32; b += kThreads) {
    const float* s = lds_x + (b >> 1) * kSlot + (b & 1) * 32;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) acc += s[j];
    lds_xs[b] = acc;
  }
  __syncthreads();
}

__device__ __forceinline__ float byte_f(uint32_t v, int k) { return static_cast<float>((v >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sbyte_f(uint32_t v, int k) {
  return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(v >> (8 * k))));
}

// sum_j c_j x_j over one Q4_0 block: q[k] holds codes 4k..4k+3 (low nibbles) and 16+4k.. (high).
__device__ __forceinline__ float q4_codes_dot(const uint32_t (&q)[4], const float4 (&xv)[8]) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
    // Hide the nibble masks from the optimizer so each byte converts with one v_cvt_f32_ubyteN
    // (otherwise the masks fold into a v_bfe per code).
    asm volatile("" : "+v"(lo), "+v"(hi));
    const float4 a = xv[k], b = xv[4 + k];
    s0 = fmaf(byte_f(lo, 0), a.x, s0);
    s1 = fmaf(byte_f(hi, 0), b.x, s1);
    s0 = fmaf(byte_f(lo, 1), a.y, s0);
    s1 = fmaf(byte_f(hi, 1), b.y, s1);
    s0 = fmaf(byte_f(lo, 2), a.z, s0);
    s1 = fmaf(byte_f(hi, 2), b.z, s1);
    s0 = fmaf(byte_f(lo, 3), a.w, s0);
    s1 = fmaf(byte_f(hi, 3), b.w, s1);
  }
  return s0 + s1;
}

// sum_j q_j x_j over one Q8_0 block: q[k] holds codes 4k..4k+3.
__device__ __forceinline__ float q8_codes_dot(const uint32_t (&q)[8], const float4 (&xv)[8]) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; k += 2) {
    const float4 a = xv[k], b = xv[k + 1];
    s0 = fmaf(sbyte_f(q[k], 0), a.x, s0);
    s1 = fmaf(sbyte_f(q[k + 1], 0), b.x, s1);
    s0 = fmaf(sbyte_f(q[k], 1), a.y, s0);
    s1 = fmaf(sbyte_f(q[k + 1], 1), b.y, s1);
    s0 = fmaf(sbyte_f(q[k], 2), a.z, s0);
    s1 = fmaf(sbyte_f(q[k + 1], 2), b.z, s1);
    s0 = fmaf(sbyte_f(q[k], 3), a.w, s0);
    s1 = fmaf(sbyte_f(q[k + 1], 3), b.w, s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ void load_x_block(const float* slot, float4 (&xv)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) xv[k] = *reinterpret_cast<const float4*>(slot + 4 * k);
}

template <int N>
__device__ __forceinline__ void load_dwords(const uint8_t* p, uint32_t (&d)[N]) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) d[i] = __builtin_nontemporal_load(q + i);
}

// Dot of R rows (stride rb bytes, starting at W) with x over the pairs p = t, t+G, ... of a row.
template <int QT, int G, int R>
__device__ __forceinline__ void rows_dot_pairs(const uint8_t* __restrict__ W, int rb, int np, int t, int nvalid,
                                               const float* lds_x, const float* lds_xs, float (&acc)[R]) {
  constexpr int PD = QT == EF_QTYPE_Q4_0 ? 9 : 17;  // dwords per block pair
  constexpr int PB = PD * 4;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int p = t; p < np; p += G) {
    uint32_t d[R][PD];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < nvalid) {
        load_dwords<PD>(W + static_cast<size_t>(r) * rb + static_cast<size_t>(p) * PB, d[r]);
      } else {
#pragma unroll
        for (int i = 0; i < PD; ++i) d[r][i] = 0u;
      }
    }
    const float* slot = lds_x + p * kSlot;
    float4 xv[8];
    // block A of the pair: scale in bytes 0-1, codes from byte 2 (realigned by 2 bytes)
    load_x_block(slot, xv);
    const float xsA = lds_xs[2 * p];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float dA = half_bits_to_float(d[r][0] & 0xFFFFu);
      if (QT == EF_QTYPE_Q4_0) {
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = __builtin_amdgcn_alignbyte(d[r][k + 1], d[r][k], 2);
        acc[r] = fmaf(dA, fmaf(-8.0f, xsA, q4_codes_dot(q, xv)), acc[r]);
      } else {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = __builtin_amdgcn_alignbyte(d[r][k + 1], d[r][k], 2);
        acc[r] = fmaf(dA, q8_codes_dot(q, xv), acc[r]);
      }
    }
    // block B: scale in the high half of the dword that ends block A's codes, codes aligned
    load_x_block(slot + 32, xv);
    const float xsB = lds_xs[2 * p + 1];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (QT == EF_QTYPE_Q4_0) {
        const float dB = half_bits_to_float(d[r][4] >> 16);
        const uint32_t q[4] = {d[r][5], d[r][6], d[r][7], d[r][8]};
        acc[r] = fmaf(dB, fmaf(-8.0f, xsB, q4_codes_dot(q, xv)), acc[r]);
      } else {
        const float dB = half_bits_to_float(d[r][8] >> 16);
        const uint32_t q[8] = {d[r][9], d[r][10], d[r][11], d[r][12], d[r][13], d[r][14], d[r][15], d[r][16]};
        acc[r] = fmaf(dB, q8_codes_dot(q, xv), acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) acc[r] += __shfl_xor(acc[r], o, kWave);
  }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }  // src/kernels.cpp:94

// The job owning `tile`, selected with constant indices so the kernel arguments stay in SGPRs.
__device__ __forceinline__ JobDev find_job(const Args& a, int tile) {
  JobDev j = a.job[0];
#pragma unroll
  for (int i = 1; i < kMaxJobs; ++i)
    if (i < a.n_jobs && tile >= a.job[i].tile_begin) j = a.job[i];
  return j;
}

// Fast path: cols % 64 == 0.  grid = (tiles, batch).
template <int EPI, int G, int R>
__global__ __launch_bounds__(kThreads) void gemv_pairs_kernel(Args a) {
  extern __shared__ float lds[];
  __shared__ double red[kWaves];
  const int K = a.K, np = K >> 6;
  float* lds_x = lds;
  float* lds_xs = lds + np * kSlot;
  const int tile = blockIdx.x, b = blockIdx.y;
  const JobDev jb = find_job(a, tile);
  stage_x(jb.x + b * jb.ldx, a.norm_w, a.eps, K, lds_x, lds_xs, red);

  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int grp = lane / G, t = lane % G;
  const int row0 = (tile - jb.tile_begin) * jb.rows_per_tile + (wave * (kWave / G) + grp) * R;
  if (row0 >= jb.rows) return;
  const int nvalid = min(R, jb.rows - row0);
  const size_t rb = static_cast<size_t>(jb.row_bytes);
  float acc[R], acc2[R];
  if (jb.qtype == EF_QTYPE_Q4_0) {
    rows_dot_pairs<EF_QTYPE_Q4_0, G, R>(jb.W + row0 * rb, jb.row_bytes, np, t, nvalid, lds_x, lds_xs, acc);
    if (EPI == kEpiSwiglu)
      rows_dot_pairs<EF_QTYPE_Q4_0, G, R>(jb.W2 + row0 * rb, jb.row_bytes, np, t, nvalid, lds_x, lds_xs, acc2);
  } else {
    rows_dot_pairs<EF_QTYPE_Q8_0, G, R>(jb.W + row0 * rb, jb.row_bytes, np, t, nvalid, lds_x, lds_xs, acc);
    if (EPI == kEpiSwiglu)
      rows_dot_pairs<EF_QTYPE_Q8_0, G, R>(jb.W2 + row0 * rb, jb.row_bytes, np, t, nvalid, lds_x, lds_xs, acc2);
  }
  if (t != 0) return;
  float* y = jb.y + b * jb.ldy + row0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nvalid) break;
    if (EPI == kEpiResidual) {
      y[r] = y[r] + acc[r];
    } else if (EPI == kEpiSwiglu) {
      y[r] = silu_f(acc[r]) * acc2[r];
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
template <int EPI, int G>
void* pick_pairs_kernel(int R) {
  if (R == 4) return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, 4>);
  if (R == 2) return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, 2>);
  return reinterpret_cast<void*>(&gemv_pairs_kernel<EPI, G, 1>);
}

template <int EPI>
void* pick_pairs_kernel(int G, int R) {
  if (G == 32) return pick_pairs_kernel<EPI, 32>(R);
  if (G == 16) return pick_pairs_kernel<EPI, 16>(R);
  return pick_pairs_kernel<EPI, 8>(R);
}

}  // namespace

int launch_gemv(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                size_t ldy, hipStream_t stream) {
  EFH_CHECK(n_jobs >= 1 && n_jobs <= kMaxJobs, "gemv: 1..4 jobs per launch");
  EFH_CHECK(batch >= 1 && batch <= 65535, "gemv: batch must be in [1, 65535]");
  EFH_CHECK(epi >= kEpiStore && epi <= kEpiSwiglu, "gemv: unknown epilogue");
  const size_t K = jobs[0].W ? jobs[0].W->cols : 0;
  EFH_CHECK(K >= 32 && K % 32 == 0 && K <= kMaxCols, "gemv: cols must be a multiple of 32 in [32, 14336]");
  for (int j = 0; j < n_jobs; ++j) {
    const GemvJob& g = jobs[j];
    EFH_CHECK(g.W && g.x && g.y, "gemv: null weight / x / y");
    EFH_CHECK(g.W->qtype == EF_QTYPE_Q4_0 || g.W->qtype == EF_QTYPE_Q8_0, "gemv: weights must be Q4_0 or Q8_0");
    EFH_CHECK(g.W->cols == K, "gemv: all jobs of one launch need the same cols");
    EFH_CHECK(g.W->rows >= 1 && g.W->rows <= (1u << 24), "gemv: rows must be in [1, 2^24]");
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
  Args a{};
  a.n_jobs = n_jobs;
  a.K = static_cast<int>(K);
  a.norm_w = norm_w;
  a.eps = eps;
  const bool fast = K % 64 == 0;
  const int np = static_cast<int>(K / 64);
  const int G = np >= 32 ? 32 : (np >= 16 ? 16 : 8);
  // rows per tile: 4 waves x (64/G) groups x R rows; R as large as keeps >= 2 tiles per CU
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  int R = 1;
  if (fast) {
    for (int cand : {4, 2}) {
      const size_t per_tile = static_cast<size_t>(kWaves * (kWave / G) * cand);
      size_t tiles = 0;
      for (int j = 0; j < n_jobs; ++j) tiles += (jobs[j].W->rows + per_tile - 1) / per_tile;
      if (tiles * static_cast<size_t>(batch) >= static_cast<size_t>(2 * cus)) {
        R = cand;
        break;
      }
    }
  }
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
    d.rows_per_tile = fast ? kWaves * (kWave / G) * R : kWaves;
    d.tile_begin = tiles;
    tiles += (d.rows + d.rows_per_tile - 1) / d.rows_per_tile;
  }
  const int nslot = static_cast<int>((K + 63) / 64);
  const size_t lds_bytes = (static_cast<size_t>(nslot) * kSlot + K / 32) * sizeof(float);
  void* fn = nullptr;
  if (fast) {
    fn = epi == kEpiStore ? pick_pairs_kernel<kEpiStore>(G, R)
                          : (epi == kEpiResidual ? pick_pairs_kernel<kEpiResidual>(G, R)
                                                 : pick_pairs_kernel<kEpiSwiglu>(G, R));
  } else {
    fn = epi == kEpiStore ? reinterpret_cast<void*>(&gemv_generic_kernel<kEpiStore>)
                          : (epi == kEpiResidual ? reinterpret_cast<void*>(&gemv_generic_kernel<kEpiResidual>)
                                                 : reinterpret_cast<void*>(&gemv_generic_kernel<kEpiSwiglu>));
  }
  void* params[] = {&a};
  EFH_HIP(hipLaunchKernel(fn, dim3(tiles, batch), dim3(kThreads), params, lds_bytes, stream));
  return EF_HIP_OK;
}

}  // namespace efh
