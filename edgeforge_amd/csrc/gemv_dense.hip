// GEMV over unquantized weights: F32, F16 and BF16 rows (kern::matvec_rows' non-block cases,
// src/qkernels.cpp:213-269: dot_bf16_avx2 :182-194, dot_f32_avx2 :196-207, the F16 loop :226-234).
//
// These types reach the decode path through lossless .efq files (layers = BF16), tied embeddings
// (lm_head is the BF16 embedding table, src/model.cpp:86) and the quantizer's BF16 fallback for row
// lengths that are not a multiple of 32 (src/qfile.cpp:71).  The kernel streams each row once:
// a wave owns kRowsPerWave rows, each lane loads 16 bytes of every row per step (a coalesced
// 1 KiB per row per wave), and x (optionally RMS-normalised, kern::rmsnorm order) sits in LDS.
// Rows whose byte length or base is not 16-byte aligned take a per-element path.  Any cols in
// [1, kMaxDenseCols] (x is held in LDS).
#include "gemv.h"

namespace efh {
namespace {

constexpr int kThreadsD = 256;
constexpr int kWavesD = kThreadsD / kWave;
constexpr int kRowsPerWave = 4;
constexpr int kRowsPerTile = kWavesD * kRowsPerWave;
constexpr int kMaxJobsD = 4;

struct DenseJob {
  const uint8_t* W;
  const uint8_t* W2;
  const float* x;
  float* y;
  long ldx, ldy;
  long row_bytes;
  int rows, tile_begin;
};

struct DenseArgs {
  DenseJob job[kMaxJobsD];
  int n_jobs;
  int K;
  const float* norm_w;
  float eps;
};

template <int QT>
struct Elem;
template <>
struct Elem<EF_QTYPE_F32> {
  static constexpr int kPer16 = 4;
  __device__ static float at(const uint8_t* row, int c) { return reinterpret_cast<const float*>(row)[c]; }
  __device__ static void unpack(uint4 v, float* f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
};
template <>
struct Elem<EF_QTYPE_BF16> {  // bf16 -> f32 is the top half of the f32 bits (include/ef/fp16.h:28)
  static constexpr int kPer16 = 8;
  __device__ static float at(const uint8_t* row, int c) {
    return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(row)[c]) << 16);
  }
  __device__ static void unpack(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};
template <>
struct Elem<EF_QTYPE_F16> {  // exact fp16 -> f32 (include/ef/fp16.h:44-67)
  static constexpr int kPer16 = 8;
  __device__ static float at(const uint8_t* row, int c) {
    return half_bits_to_float(reinterpret_cast<const uint16_t*>(row)[c]);
  }
  __device__ static void unpack(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = half_bits_to_float(w[i] & 0xFFFFu);
      f[2 * i + 1] = half_bits_to_float(w[i] >> 16);
    }
  }
};

__device__ __forceinline__ float silu_d(float g) { return g / (1.0f + expf(-g)); }  // src/kernels.cpp:94

// Dot products of up to kRowsPerWave rows (row pointers clamped in range by the caller) with x.
template <int QT, bool VEC>
__device__ __forceinline__ void rows_dot(const uint8_t* const* rows, const float* xs, int K, int lane,
                                         float* acc) {
  if constexpr (VEC) {
    constexpr int E = Elem<QT>::kPer16;
#pragma unroll 2
    for (int c = lane * E; c < K; c += kWave * E) {
      float xv[E];
#pragma unroll
      for (int i = 0; i < E; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(xs + c + i);
        xv[i] = t.x;
        xv[i + 1] = t.y;
        xv[i + 2] = t.z;
        xv[i + 3] = t.w;
      }
      v4i v[kRowsPerWave];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r)
        v[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(rows[r] + static_cast<size_t>(c) * (16 / E)));
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) {
        float w[E];
        Elem<QT>::unpack(make_uint4(v[r].x, v[r].y, v[r].z, v[r].w), w);
#pragma unroll
        for (int i = 0; i < E; ++i) acc[r] = fmaf(w[i], xv[i], acc[r]);
      }
    }
  } else {
    for (int c = lane; c < K; c += kWave) {
      const float xv = xs[c];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) acc[r] = fmaf(Elem<QT>::at(rows[r], c), xv, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) acc[r] = wave_sum(acc[r]);
}

template <int EPI, int QT, bool VEC>
__global__ __launch_bounds__(kThreadsD) void gemv_dense_kernel(DenseArgs a) {
  extern __shared__ float xs[];
  __shared__ double red[kWavesD];
  const int K = a.K, tile = blockIdx.x, b = blockIdx.y;
  int j = 0;
  for (int i = 1; i < a.n_jobs; ++i) j = tile >= a.job[i].tile_begin ? i : j;
  DenseJob jb = a.job[0];
  for (int i = 1; i < a.n_jobs; ++i)
    if (i == j) jb = a.job[i];
  const float* x = jb.x + b * jb.ldx;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  if (a.norm_w != nullptr) {  // kern::rmsnorm: sum of squares in double, then w * (x * inv)
    double ss = 0.0;
    for (int i = tid; i < K; i += kThreadsD) ss += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    ss = wave_sum_d(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(a.eps)));
    for (int i = tid; i < K; i += kThreadsD) xs[i] = a.norm_w[i] * (x[i] * inv);
  } else {
    for (int i = tid; i < K; i += kThreadsD) xs[i] = x[i];
  }
  __syncthreads();
  const int r0 = (tile - jb.tile_begin) * kRowsPerTile + wave * kRowsPerWave;
  if (r0 >= jb.rows) return;
  const uint8_t* rows[kRowsPerWave];
  float acc[kRowsPerWave] = {};
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) rows[r] = jb.W + static_cast<size_t>(min(r0 + r, jb.rows - 1)) * jb.row_bytes;
  rows_dot<QT, VEC>(rows, xs, K, lane, acc);
  float acc2[kRowsPerWave] = {};
  if (EPI == kEpiSwiglu) {
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      rows[r] = jb.W2 + static_cast<size_t>(min(r0 + r, jb.rows - 1)) * jb.row_bytes;
    rows_dot<QT, VEC>(rows, xs, K, lane, acc2);
  }
  float* y = jb.y + b * jb.ldy + r0;
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    if (lane != r || r0 + r >= jb.rows) continue;
    if (EPI == kEpiResidual) {
      y[r] = y[r] + acc[r];
    } else if (EPI == kEpiSwiglu) {
      y[r] = silu_d(acc[r]) * acc2[r];
    } else {
      y[r] = acc[r];
    }
  }
}

template <int EPI, int QT>
void* pick_vec(bool vec) {
  return vec ? reinterpret_cast<void*>(&gemv_dense_kernel<EPI, QT, true>)
             : reinterpret_cast<void*>(&gemv_dense_kernel<EPI, QT, false>);
}

template <int EPI>
void* pick_dense(int qt, bool vec) {
  if (qt == EF_QTYPE_F32) return pick_vec<EPI, EF_QTYPE_F32>(vec);
  if (qt == EF_QTYPE_F16) return pick_vec<EPI, EF_QTYPE_F16>(vec);
  return pick_vec<EPI, EF_QTYPE_BF16>(vec);
}

}  // namespace

bool is_dense_qtype(int qtype) {
  return qtype == EF_QTYPE_F32 || qtype == EF_QTYPE_F16 || qtype == EF_QTYPE_BF16;
}

int launch_gemv_dense(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch,
                      size_t ldx, size_t ldy, hipStream_t stream) {
  EFH_CHECK(n_jobs >= 1 && n_jobs <= kMaxJobsD, "gemv: 1..4 jobs per launch");
  const size_t K = jobs[0].W->cols;
  const int qt = jobs[0].W->qtype;
  EFH_CHECK(K >= 1 && K <= kMaxDenseCols, "gemv: cols of an F32 / F16 / BF16 matrix must be in [1, 16320]");
  DenseArgs a{};
  a.n_jobs = n_jobs;
  a.K = static_cast<int>(K);
  a.norm_w = norm_w;
  a.eps = eps;
  bool vec = true;
  int tiles = 0;
  for (int j = 0; j < n_jobs; ++j) {
    const GemvJob& g = jobs[j];
    EFH_CHECK(g.W->qtype == qt && g.W->cols == K, "gemv: the F32 / F16 / BF16 jobs of one launch need one type and cols");
    EFH_CHECK(g.W->rows >= 1 && g.W->rows <= (1u << 24), "gemv: rows must be in [1, 2^24]");
    if (epi == kEpiSwiglu) {
      EFH_CHECK(g.W2 && g.W2->qtype == qt && g.W2->rows == g.W->rows && g.W2->cols == K,
                "gemv: swiglu needs gate and up of the same type and shape");
    }
    DenseJob& d = a.job[j];
    d.W = static_cast<const uint8_t*>(g.W->dev);
    d.W2 = g.W2 ? static_cast<const uint8_t*>(g.W2->dev) : nullptr;
    d.x = g.x;
    d.y = g.y;
    d.ldx = static_cast<long>(g.ldx ? g.ldx : ldx);
    d.ldy = static_cast<long>(g.ldy ? g.ldy : ldy);
    d.row_bytes = static_cast<long>(g.W->row_bytes);
    d.rows = static_cast<int>(g.W->rows);
    d.tile_begin = tiles;
    tiles += (d.rows + kRowsPerTile - 1) / kRowsPerTile;
    vec = vec && d.row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(d.W) % 16 == 0 &&
          (d.W2 == nullptr || reinterpret_cast<uintptr_t>(d.W2) % 16 == 0);
  }
  void* fn = epi == kEpiStore ? pick_dense<kEpiStore>(qt, vec)
                              : (epi == kEpiResidual ? pick_dense<kEpiResidual>(qt, vec) : pick_dense<kEpiSwiglu>(qt, vec));
  void* params[] = {&a};
  EFH_HIP(hipLaunchKernel(fn, dim3(tiles, batch), dim3(kThreadsD), params, K * sizeof(float), stream));
  return EF_HIP_OK;
}

}  // namespace efh
