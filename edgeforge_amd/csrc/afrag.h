// Producer-side staging of the matrix-core GEMV's block-scaled A tables (gemv_mfma.hip): a kernel
// whose output is the next batched product's input writes that input straight into the tables, so
// the product needs no preparation launch.  Shared by the GEMV epilogues, the KV-group attention
// and the embedding lookup.
//
// Table layout (one per column order): for sequence tile T (16 sequences), block kb (32 values of
// the product's K), part (hi, lo) and lane 16 g + i (sequence i of the tile), 8 fp16 values:
//   Q4_0 order: the block's values 4g + {0, 2, 16, 18, 1, 3, 17, 19} (the high-nibble slots 2, 3,
//               6, 7 divided by 16),
//   Q8_0 order: 8g + {0, 2, 1, 3, 4, 6, 5, 7};
// at byte ((T * nb + kb) * 2 * 64 + 16 g + i) * 16, the lo part 1024 bytes after the hi part.
// Every (sequence, block) has a power-of-two scale 2^e (max |v| 2^-e < 2^15) at
// bscale[kb * bpad + sequence]; the tables hold v 2^-e split exactly into fp16 hi + lo, with
// v = norm_w * x for a product with an input RMSNorm (else x), and ssp[kb * bpad + sequence] the
// block's double sum of x^2 (the norm's statistic, one partial per block).
#pragma once

#include "common.h"

namespace efh {

struct AEmit {
  uint8_t* t4 = nullptr;  // the consuming product's column orders (null: not needed)
  uint8_t* t8 = nullptr;
  float* bscale = nullptr;
  double* ssp = nullptr;      // null: the consumer has no RMSNorm
  const float* nw = nullptr;  // the consumer's norm weights (null: none)
  int nb = 0;                 // the consumer's K / 32
  int bpad = 0;
  __host__ __device__ bool on() const { return bscale != nullptr; }
};

namespace {

// Max over the 32 lanes of each half-wave, returned on every lane of that half (DPP within rows of
// 16, then row 1 <- row 0 and row 3 <- row 2; lanes 31 and 63 hold the halves' maxima).
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, dpp_self_f<0xB1>(v));
  v = fmaxf(v, dpp_self_f<0x4E>(v));
  v = fmaxf(v, dpp_self_f<0x141>(v));
  v = fmaxf(v, dpp_self_f<0x140>(v));
  v = fmaxf(v, dpp_self_f<0x142, 0xA>(v));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return (threadIdx.x & 32) ? hi : lo;
}

// Element kk of block kb of sequence seq, already divided by the block's scale.
__device__ __forceinline__ void afrag_store(const AEmit& em, int seq, int kb, int kk, float v) {
  const int tile = seq >> 4, i = seq & 15;
  const _Float16 hh = static_cast<_Float16>(v);
  const _Float16 ll = static_cast<_Float16>(v - static_cast<float>(hh));
  const size_t frag = (static_cast<size_t>(tile) * em.nb + kb) * 2 * 64;
  if (em.t4 != nullptr) {
    const int half = kk >> 4, m = kk & 15, g = m >> 2, r = m & 3;
    const int u = (r & 1) * 4 + half * 2 + (r >> 1);
    const _Float16 qs = static_cast<_Float16>((u & 2) ? 0.0625f : 1.0f);  // exact powers of two
    _Float16* p = reinterpret_cast<_Float16*>(em.t4 + (frag + 16 * g + i) * 16) + u;
    p[0] = hh * qs;
    p[512] = ll * qs;  // 1024 bytes on: the lo part
  }
  if (em.t8 != nullptr) {
    const int g = kk >> 3, o = kk & 7;
    const int u = (o & 4) + ((o & 1) << 1) + ((o >> 1) & 1);
    _Float16* p = reinterpret_cast<_Float16*>(em.t8 + (frag + 16 * g + i) * 16) + u;
    p[0] = hh;
    p[512] = ll;
  }
}

// One (sequence, block) per half-wave: lane kk of the half holds element kk (x, the un-normed
// value).  All 64 lanes of the wave take part; `live` (uniform over a half) says whether the
// half's unit is a real one.
__device__ __forceinline__ void emit_block(const AEmit& em, int seq, int kb, int kk, float x, bool live) {
  const float v = (em.nw != nullptr && live) ? em.nw[kb * 32 + kk] * x : x;
  const float m = half_wave_max(live ? fabsf(v) : 0.0f);
  const float bound = m * 1.0001f;
  int ex = 0;
  if (bound > 0.0f && bound <= 3.0e38f) ex = ilogbf(bound) - 14;  // bound * 2^-ex < 2^15
  if (em.ssp != nullptr) {
    double q = live ? static_cast<double>(x) * static_cast<double>(x) : 0.0;
    q = group_sum_dpp<32>(q);  // lane 31 of each half holds the block's sum
    if (live && kk == 31) em.ssp[static_cast<size_t>(kb) * em.bpad + seq] = q;
  }
  if (!live) return;
  if (kk == 0) em.bscale[static_cast<size_t>(kb) * em.bpad + seq] = ldexpf(1.0f, ex);
  afrag_store(em, seq, kb, kk, v * ldexpf(1.0f, -ex));
}

}  // namespace
}  // namespace efh
