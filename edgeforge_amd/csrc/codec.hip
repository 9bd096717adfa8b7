// Block codec on the device: the reference quantizer (Q4_0 scale search, Q8_0), 16-bit float
// packing, and row lookup (dequantization / widening) for embeddings.
//
// The quantizer is the reference's per-block algorithm (src/quant.cpp:26-99, 151-175), one thread
// per 32-weight block, written so every float and double operation is the same IEEE operation in
// the same order (correctly rounded divides, no contraction), so the packed bytes are identical.
#include <climits>
#include <cmath>

#include "codec.h"

#pragma clang fp contract(off)

namespace efh {
namespace {

// binary32 -> binary16, round to nearest even (include/ef/fp16.h:69-91).
__device__ uint16_t f32_to_fp16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return static_cast<uint16_t>(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
  if (a >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);
  if (a < 0x38800000u) {
    if (a <= 0x33000000u) return sign;
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t sh = 126u - (a >> 23);
    uint32_t r = m >> sh;
    const uint32_t rest = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rest > half || (rest == half && (r & 1u))) ++r;
    return static_cast<uint16_t>(sign | r);
  }
  const uint32_t x = a - 0x38000000u;
  return static_cast<uint16_t>(sign | ((x + 0xFFFu + ((x >> 13) & 1u)) >> 13));
}

// binary32 -> bfloat16, round to nearest even, NaN kept quiet (include/ef/fp16.h:32-40).
__device__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ float fp16_round(float d) { return half_bits_to_float(f32_to_fp16_bits(d)); }

__device__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// static_cast<int>(float) as the reference's x86-64 build executes it (cvttss2si): NaN and
// out-of-range values give INT_MIN ("integer indefinite"); v_cvt_i32_f32 would saturate instead.
__device__ int to_int_x86(float v) { return fabsf(v) < 2147483648.0f ? static_cast<int>(v) : INT_MIN; }

__device__ double q4_try(const float* x, float d, uint8_t* codes) {
  const float inv = __fdiv_rn(1.0f, d);
  double sse = 0.0;
  for (int j = 0; j < 32; ++j) {
    const int c = clampi(to_int_x86(rintf(x[j] * inv)) + 8, 0, 15);
    codes[j] = static_cast<uint8_t>(c);
    const double e = static_cast<double>(x[j]) - static_cast<double>(static_cast<float>(c - 8) * d);
    sse += e * e;
  }
  return sse;
}

// q4_group for one 32-weight block (src/quant.cpp:26-99).
__device__ float q4_block(const float* x, bool search, uint8_t* q) {
  float amax = 0.0f, smax = 0.0f;
  for (int j = 0; j < 32; ++j) {
    const float a = fabsf(x[j]);
    if (a > amax) {
      amax = a;
      smax = x[j];
    }
  }
  if (!(amax > 0.0f) || !isfinite(amax)) {
    for (int j = 0; j < 32; ++j) q[j] = 8;
    return 0.0f;
  }
  float cand[6];
  int nc = 0;
  cand[nc++] = __fdiv_rn(smax, -8.0f);
  if (search) {
    cand[nc++] = __fdiv_rn(amax, 7.0f);
    cand[nc++] = __fdiv_rn(amax, 7.25f);
    cand[nc++] = __fdiv_rn(amax, 7.5f);
    cand[nc++] = __fdiv_rn(amax, 7.75f);
    cand[nc++] = __fdiv_rn(amax, 8.0f);
  }
  uint8_t trial[32];
  float best = 0.0f;
  double best_sse = -1.0;
  for (int c = 0; c < nc; ++c) {
    const float v = fminf(fmaxf(cand[c], -65504.0f), 65504.0f);
    const float d = fp16_round(v);
    if (d == 0.0f) continue;
    const double sse = q4_try(x, d, trial);
    if (best_sse < 0.0 || sse < best_sse) {
      best_sse = sse;
      best = d;
      for (int j = 0; j < 32; ++j) q[j] = trial[j];
    }
  }
  if (best_sse < 0.0) {
    for (int j = 0; j < 32; ++j) q[j] = 8;
    return 0.0f;
  }
  if (!search) return best;
  for (int round = 0; round < 2; ++round) {
    double num = 0.0, den = 0.0;
    for (int j = 0; j < 32; ++j) {
      const double c = static_cast<double>(static_cast<int>(q[j]) - 8);
      num += static_cast<double>(x[j]) * c;
      den += c * c;
    }
    if (den == 0.0) break;
    double ls = num / den;
    ls = ls < -65504.0 ? -65504.0 : (ls > 65504.0 ? 65504.0 : ls);
    const float d = fp16_round(static_cast<float>(ls));
    if (d == 0.0f || d == best) break;
    const double sse = q4_try(x, d, trial);
    if (!(sse < best_sse)) break;
    best_sse = sse;
    best = d;
    for (int j = 0; j < 32; ++j) q[j] = trial[j];
  }
  return best;
}

__global__ void quantize_blocks_kernel(int qtype, const float* __restrict__ w, long rows, long cols, int search,
                                       uint8_t* __restrict__ out) {
  const long nbr = cols / 32;
  const long g = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= rows * nbr) return;
  const long r = g / nbr, blk = g % nbr;
  float x[32];
  const float* src = w + r * cols + blk * 32;
  for (int j = 0; j < 32; ++j) x[j] = src[j];
  if (qtype == EF_QTYPE_Q4_0) {
    uint8_t q[32];
    const uint16_t d = f32_to_fp16_bits(q4_block(x, search != 0, q));
    uint8_t* o = out + r * nbr * 18 + blk * 18;
    o[0] = static_cast<uint8_t>(d & 0xFF);
    o[1] = static_cast<uint8_t>(d >> 8);
    for (int j = 0; j < 16; ++j) o[2 + j] = static_cast<uint8_t>(q[j] | (q[j + 16] << 4));
  } else {  // Q8_0 (src/quant.cpp:166-175)
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    float d = 0.0f;
    if (amax > 0.0f && isfinite(amax)) d = fp16_round(fminf(__fdiv_rn(amax, 127.0f), 65504.0f));
    const uint16_t h = f32_to_fp16_bits(d);
    uint8_t* o = out + r * nbr * 34 + blk * 34;
    o[0] = static_cast<uint8_t>(h & 0xFF);
    o[1] = static_cast<uint8_t>(h >> 8);
    const float inv = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    for (int j = 0; j < 32; ++j) {
      o[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(clampi(to_int_x86(rintf(x[j] * inv)), -127, 127)));
    }
  }
}

__global__ void pack16_kernel(int qtype, const float* __restrict__ w, size_t n, uint16_t* __restrict__ out) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    out[i] = qtype == EF_QTYPE_BF16 ? f32_to_bf16_bits(w[i]) : f32_to_fp16_bits(w[i]);
  }
}

// Row lookup: out[b][:] = row ids[b] of W as FP32 (kern::row_f32, src/qkernels.cpp:299-305).
__global__ void rows_f32_kernel(const uint8_t* __restrict__ W, int qtype, long rows, long cols, long rb,
                                const int32_t* __restrict__ ids, float* __restrict__ out, long ldo) {
  const int b = blockIdx.y;
  const int32_t id = ids[b];
  float* o = out + b * ldo;
  const bool ok = id >= 0 && id < rows;
  const uint8_t* row = W + (ok ? id : 0) * rb;
  for (long c = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; c < cols;
       c += static_cast<long>(gridDim.x) * blockDim.x) {
    float v = 0.0f;
    if (!ok) {
      v = __int_as_float(0x7FC00000);  // an out-of-range id yields NaN rows (callers validate ids first)
    } else if (qtype == EF_QTYPE_F32) {
      v = reinterpret_cast<const float*>(row)[c];
    } else if (qtype == EF_QTYPE_BF16) {
      v = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(row)[c]) << 16);
    } else if (qtype == EF_QTYPE_F16) {
      v = half_bits_to_float(reinterpret_cast<const uint16_t*>(row)[c]);
    } else {
      const long blk = c >> 5, j = c & 31;
      if (qtype == EF_QTYPE_Q4_0) {
        const uint8_t* p = row + blk * 18;
        const float d = half_bits_to_float(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
        const int code = j < 16 ? (p[2 + j] & 15) : (p[2 + j - 16] >> 4);
        v = static_cast<float>(code - 8) * d;
      } else {
        const uint8_t* p = row + blk * 34;
        const float d = half_bits_to_float(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
        v = static_cast<float>(static_cast<int8_t>(p[2 + j])) * d;
      }
    }
    o[c] = v;
  }
}

}  // namespace

int launch_quantize(int qtype, const float* w, size_t rows, size_t cols, int search, void* out, hipStream_t s) {
  if (qtype == EF_QTYPE_Q4_0 || qtype == EF_QTYPE_Q8_0) {
    const size_t blocks = rows * (cols / 32);
    const unsigned grid = static_cast<unsigned>((blocks + 255) / 256);
    hipLaunchKernelGGL(quantize_blocks_kernel, dim3(grid), dim3(256), 0, s, qtype, w, static_cast<long>(rows),
                       static_cast<long>(cols), search, static_cast<uint8_t*>(out));
  } else if (qtype == EF_QTYPE_BF16 || qtype == EF_QTYPE_F16) {
    const size_t n = rows * cols;
    const unsigned grid = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 65536));
    hipLaunchKernelGGL(pack16_kernel, dim3(grid), dim3(256), 0, s, qtype, w, n, static_cast<uint16_t*>(out));
  } else {
    EFH_HIP(hipMemcpyAsync(out, w, rows * cols * 4, hipMemcpyDeviceToDevice, s));
  }
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_rows_f32(const ef_hip_weight_s* W, const int32_t* ids, int batch, float* out, size_t ldo, hipStream_t s) {
  const unsigned gx = static_cast<unsigned>(std::min<size_t>((W->cols + 255) / 256, 64));
  hipLaunchKernelGGL(rows_f32_kernel, dim3(gx, batch), dim3(256), 0, s, W->dev, W->qtype, static_cast<long>(W->rows),
                     static_cast<long>(W->cols), static_cast<long>(W->row_bytes), ids, out, static_cast<long>(ldo));
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

}  // namespace efh

// ---- synthetic inputs -----------------------------------------------------------------------------------
// N(mean, scale^2) floats from Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as
// 1, 2, 3", SC'11) and the Box-Muller transform: element i uses counter (i / 4, offset), key seed.
// Deterministic for (seed, offset, i) on every run; used to build synthetic weights and inputs.
namespace efh {
namespace {

__device__ __forceinline__ void philox_round(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c[0];
  const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c[2];
  const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c[1] ^ k0;
  const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c[3] ^ k1;
  c[1] = static_cast<uint32_t>(p1);
  c[3] = static_cast<uint32_t>(p0);
  c[0] = n0;
  c[2] = n2;
}

__global__ void fill_normal_kernel(float* __restrict__ out, size_t n, uint64_t seed, uint64_t offset, float mean,
                                   float scale) {
  const size_t q = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q * 4 >= n) return;
  uint32_t c[4] = {static_cast<uint32_t>(q), static_cast<uint32_t>(q >> 32), static_cast<uint32_t>(offset),
                   static_cast<uint32_t>(offset >> 32)};
  uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
  for (int r = 0; r < 10; ++r) {
    philox_round(c, k0, k1);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  float z[4];
  for (int h = 0; h < 2; ++h) {
    const float u1 = (static_cast<float>(c[2 * h] >> 8) + 0.5f) * 0x1p-24f;  // (0, 1)
    const float u2 = static_cast<float>(c[2 * h + 1] >> 8) * 0x1p-24f;       // [0, 1)
    const float r = sqrtf(-2.0f * logf(u1));
    z[2 * h] = r * cosf(6.28318530717958647692f * u2);
    z[2 * h + 1] = r * sinf(6.28318530717958647692f * u2);
  }
  for (int j = 0; j < 4; ++j)
    if (q * 4 + j < n) out[q * 4 + j] = mean + scale * z[j];
}

}  // namespace

int launch_fill_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float mean, float scale,
                       hipStream_t s) {
  const size_t quads = (n + 3) / 4;
  hipLaunchKernelGGL(fill_normal_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0, s, out, n,
                     seed, offset, mean, scale);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

}  // namespace efh
