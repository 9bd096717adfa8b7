// Packed Q4_0 / Q8_0 GEMV on the matrix cores for batches of sequences (2..64 per launch).
//
// Two kernels per launch:
//  1. xfrag_kernel turns the activations [B][K] (optionally RMS-normalised, kern::rmsnorm order)
//     into the A operands of v_mfma_f32_16x16x32_f16, in global memory, laid out exactly as a wave
//     loads them: for each tile of 8 sequences and each 32-weight block, 64 lanes x 16 bytes (one
//     coalesced 1 KB load).  A row i = 2s + p of a tile holds sequence s's hi (p = 0) or lo (p = 1)
//     part: x' = x * 2^-e_s (a per-sequence power of two keeping |x'| < 2^15) split exactly into
//     fp16 hi + lo (x' - hi - lo is below 2^-22 |x'|).  Columns follow the codes' k order below.
//  2. gemv_mfma_kernel: a workgroup (8 waves) owns 16 or 32 rows (x2 matrices for SwiGLU); its
//     rows' packed blocks are fetched with coalesced 1 KB LDS-DMA loads into LDS rows an odd number
//     of 16-byte units apart (the 16 rows one B fragment reads fall in distinct banks).  The waves
//     split the block pairs (pair m to wave m % 8).  Per pair, each matrix's codes are converted
//     once into B operands and reused for every sequence tile:
//       B = the row's codes minus their bias as exact fp16, straight out of the packed bytes: one
//           AND-OR of a Q4_0 dword with the fp16 pattern of 1024 yields two codes as 1024 + c
//           ((q & 0x000F000F) | 0x64006400: codes 0 and 2 of the dword's low nibbles; the high
//           nibbles through 0x00F000F0 come out as 1024 + 16 c), and one packed fp16 add removes
//           1024 + 8 (resp. 1024 + 128) exactly.  Q8_0 codes are offset to unsigned (q ^ 0x80) and
//           taken two per AND-OR the same way, minus 1024 + 128.  The A columns are permuted to
//           match, and divided by 16 where the code is a scaled high nibble;
//       D = A x B gives, for each sequence of the tile, hi and lo parts of sum_k (c_k - bias) x'_k;
//           the block adds d * (D[2s][j] + D[2s+1][j]) to an FP32 accumulator.
//     Partial sums of the eight waves are combined in LDS in a fixed order; the scale 2^e_s is
//     undone and the epilogue (store / residual / SwiGLU) applied.
// (Codes as fp16 subnormals would save the add, but the matrix core does not sum products of
// subnormal operands exactly: measured errors of thousands of ulps, biased; normal operands give
// a few ulps, unbiased.)  Products are exact (fp16 x fp16 in FP32), so results match an FP32 dot
// product to rounding; the order differs from the reference CPU kernels (src/qkernels.cpp:39-65,
// 131-180) and is fixed for a given shape.  Single sequences use the vector-ALU kernels (gemv.hip),
// which are faster when nothing amortises the activation preparation.
#include <cmath>

#include "gemv.h"

namespace efh {
namespace {

constexpr int kT = 512;                         // GEMV workgroup: 8 waves split the block pairs
constexpr int kWavesM = kT / kWave;
constexpr int kTP = 1024;                       // prep workgroup
constexpr int kWavesP = kTP / kWave;
constexpr int kTileRows = 16;
constexpr int kSeqTile = 8;                     // sequences per A operand (hi + lo rows)
constexpr int kMaxTiles = 8;                    // sequence tiles per launch: 64 sequences
constexpr int kMaxJobsM = 4;
constexpr int kPrepSplit = 4;                   // workgroups per sequence tile in xfrag_kernel

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

struct MJob {
  const uint8_t* W;
  const uint8_t* W2;
  float* y;
  int rows, qtype, row_bytes, tile_begin;
  long ldy;
};

struct MArgs {
  MJob job[kMaxJobsM];
  int n_jobs, K, B, n_tiles;
  const uint8_t* t4;    // A tables (Q4_0 and Q8_0 column orders), [tile][block][64 lanes][16 bytes]
  const uint8_t* t8;
  const float* post;    // [B] 2^e_s
  uint32_t row_stride, w_stride;  // LDS: weight rows rs bytes apart, w_stride bytes per matrix
  int ksplit, pairs_per_split;    // split-K: workgroups per row group and block pairs each
  float* part;          // [group][split][B][rows of the group][matrices] partial sums (ksplit > 1)
};

struct PrepArgs {
  const float* x;       // [B][ldx]
  long ldx;
  int K, B;
  const float* norm_w;
  float eps;
  uint8_t* t4;
  uint8_t* t8;
  float* post;
};

__device__ __forceinline__ MJob find_mjob(const MArgs& a, int tile) {
  MJob j = a.job[0];
#pragma unroll
  for (int i = 1; i < kMaxJobsM; ++i)
    if (i < a.n_jobs && tile >= a.job[i].tile_begin) j = a.job[i];
  return j;
}

template <int AUX>
__device__ __forceinline__ void dma_copy(__amdgpu_buffer_rsrc_t r, uint32_t src_off, uint8_t* dst, uint32_t bytes,
                                         int lane) {
  // bytes % 16 == 0; lane l's 16 bytes of each 1 KB instruction land at dst + o + 16 l
  for (uint32_t o = 0; o < bytes; o += 1024u) {
    if (o + 16u * lane < bytes)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + o), 16, src_off + o + 16u * lane, 0, 0, AUX);
  }
}

__device__ __forceinline__ float f16lo(uint32_t v) { return half_bits_to_float(v & 0xFFFFu); }
__device__ __forceinline__ float f16hi(uint32_t v) { return half_bits_to_float(v >> 16); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// (v & mask) | fp16(1024) pattern in both halves, minus (1024 + bias) in both halves: exact.
__device__ __forceinline__ uint32_t codes2(uint32_t v, uint32_t mask, _Float16 minus) {
  const uint32_t m = (v & mask) | 0x64006400u;
  h2 h;
  __builtin_memcpy(&h, &m, 4);
  const h2 c = {minus, minus};
  h = h + c;
  uint32_t r;
  __builtin_memcpy(&r, &h, 4);
  return r;
}

__device__ __forceinline__ h8 q4_operand(uint32_t q) {
  const uint32_t s = q >> 8;
  const _Float16 lo = static_cast<_Float16>(-1032.0f), hi = static_cast<_Float16>(-1152.0f);
  const uint32_t w[4] = {codes2(q, 0x000F000Fu, lo), codes2(q, 0x00F000F0u, hi), codes2(s, 0x000F000Fu, lo),
                         codes2(s, 0x00F000F0u, hi)};
  h8 r;
  __builtin_memcpy(&r, w, 16);
  return r;
}

__device__ __forceinline__ h8 q8_operand(uint32_t q0, uint32_t q1) {
  const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
  const _Float16 m = static_cast<_Float16>(-1152.0f);
  const uint32_t w[4] = {codes2(u0, 0x00FF00FFu, m), codes2(u0 >> 8, 0x00FF00FFu, m), codes2(u1, 0x00FF00FFu, m),
                         codes2(u1 >> 8, 0x00FF00FFu, m)};
  h8 r;
  __builtin_memcpy(&r, w, 16);
  return r;
}

__device__ __forceinline__ float silu_m(float g) { return g / (1.0f + expf(-g)); }  // src/kernels.cpp:94

// grid (kPrepSplit, tiles): every workgroup of a tile recomputes the tile's per-sequence factors
// (a read of 8 x K floats from L2), then writes the fragments of its share of the blocks.
__global__ __launch_bounds__(kTP) void xfrag_kernel(PrepArgs a) {
  __shared__ double s_ss[kWavesP];
  __shared__ float s_ax[kWavesP];
  __shared__ float s_aw[kWavesP];
  __shared__ float s_mul[kSeqTile], s_pre[kSeqTile];
  const int K = a.K, tile = blockIdx.y, nb = K >> 5;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const bool has_norm = a.norm_w != nullptr;
  // 1. per-sequence sum of squares (double, kern::rmsnorm) and max |x|, and max |norm weight|.
  //    Threads are sequence-major (128 per sequence), so each thread reduces one sequence and the
  //    cross-lane reductions are one chain per wave rather than one per sequence.
  {
    constexpr int kPer = kTP / kSeqTile;  // threads per sequence: two waves
    const int s = threadIdx.x / kPer, r = threadIdx.x % kPer, sq = tile * kSeqTile + s;
    double ss = 0.0;
    float ax = 0.0f, aw = 0.0f;
    if (sq < a.B) {
      const float* xr = a.x + sq * a.ldx;
      for (int k = r * 4; k < K; k += kPer * 4) {
        const float4 v = *reinterpret_cast<const float4*>(xr + k);
        ss += static_cast<double>(v.x) * static_cast<double>(v.x);
        ss += static_cast<double>(v.y) * static_cast<double>(v.y);
        ss += static_cast<double>(v.z) * static_cast<double>(v.z);
        ss += static_cast<double>(v.w) * static_cast<double>(v.w);
        ax = fmaxf(ax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
      }
    }
    if (has_norm) {
      for (int k = threadIdx.x * 4; k < K; k += kTP * 4) {
        const float4 w = *reinterpret_cast<const float4*>(a.norm_w + k);
        aw = fmaxf(aw, fmaxf(fmaxf(fabsf(w.x), fabsf(w.y)), fmaxf(fabsf(w.z), fabsf(w.w))));
      }
    }
    ss = wave_sum_d(ss);
    for (int o = kWave / 2; o > 0; o >>= 1) {
      ax = fmaxf(ax, __shfl_xor(ax, o, kWave));
      aw = fmaxf(aw, __shfl_xor(aw, o, kWave));
    }
    if (lane == 0) {
      s_ss[wave] = ss;
      s_ax[wave] = ax;
      s_aw[wave] = aw;
    }
  }
  __syncthreads();
  if (threadIdx.x < kSeqTile) {
    const int s = threadIdx.x, sq = tile * kSeqTile + s;
    float aw = 0.0f;
    for (int w = 0; w < kWavesP; ++w) aw = fmaxf(aw, s_aw[w]);
    if (!has_norm) aw = 1.0f;
    const double tot = s_ss[2 * s] + s_ss[2 * s + 1];  // the sequence's two waves
    const float ax = fmaxf(s_ax[2 * s], s_ax[2 * s + 1]);
    const float inv = has_norm ? static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(a.eps)))
                               : 1.0f;
    const float bound = ax * inv * aw * 1.0001f;  // >= max |w * (x * inv)|
    int e = 0;
    if (bound > 0.0f && bound <= 3.0e38f) e = ilogbf(bound) - 14;  // bound * 2^-e < 2^15
    s_mul[s] = inv;
    s_pre[s] = ldexpf(1.0f, -e);
    if (blockIdx.x == 0 && sq < a.B) a.post[sq] = ldexpf(1.0f, e);
  }
  __syncthreads();
  // 2. fragments: one (block, lane) per thread, 16 bytes each.  The 8 values of a Q4_0 fragment are
  //    weights 4g..4g+3 and 4g+16..4g+19 of the block, of a Q8_0 fragment 8g..8g+7: two float4 each.
  const int i = lane & 15, g = lane >> 4, s = i >> 1, part = i & 1, sq = tile * kSeqTile + s;
  const bool live = sq < a.B;
  const float inv = s_mul[s], pre = s_pre[s];
  const float* xr = a.x + (live ? sq : 0) * a.ldx;
  const int per = (nb + kPrepSplit - 1) / kPrepSplit;
  const int kb0 = blockIdx.x * per, kb1 = min(nb, kb0 + per);
  auto frag = [&](const int (&k0)[2], float (&out)[8]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float4 v = live ? *reinterpret_cast<const float4*>(xr + k0[h]) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (has_norm) {  // HF order: w * (x * inv)
        const float4 w = *reinterpret_cast<const float4*>(a.norm_w + k0[h]);
        v.x = w.x * (v.x * inv);
        v.y = w.y * (v.y * inv);
        v.z = w.z * (v.z * inv);
        v.w = w.w * (v.w * inv);
      }
      out[4 * h + 0] = v.x * pre;
      out[4 * h + 1] = v.y * pre;
      out[4 * h + 2] = v.z * pre;
      out[4 * h + 3] = v.w * pre;
    }
  };
  auto split = [&](float xp) -> _Float16 {
    const _Float16 hi = static_cast<_Float16>(xp);
    return part == 0 ? hi : static_cast<_Float16>(xp - static_cast<float>(hi));
  };
  for (int kb = kb0 + wave; kb < kb1; kb += kWavesP) {
    if (a.t4 != nullptr) {  // slots 0..7 = weights 4g + {0, 2, 16, 18, 1, 3, 17, 19}
      const int k0[2] = {kb * 32 + 4 * g, kb * 32 + 16 + 4 * g};
      float xv[8];
      frag(k0, xv);
      const _Float16 q = static_cast<_Float16>(0.0625f);  // pairs a code scaled by 16
      const h8 f = {split(xv[0]), split(xv[2]), split(xv[4]) * q, split(xv[6]) * q,
                    split(xv[1]), split(xv[3]), split(xv[5]) * q, split(xv[7]) * q};
      *reinterpret_cast<h8*>(a.t4 + ((static_cast<size_t>(tile) * nb + kb) * kWave + lane) * 16) = f;
    }
    if (a.t8 != nullptr) {  // slots 0..7 = weights 8g + {0, 2, 1, 3, 4, 6, 5, 7}
      const int k0[2] = {kb * 32 + 8 * g, kb * 32 + 8 * g + 4};
      float xv[8];
      frag(k0, xv);
      const h8 f = {split(xv[0]), split(xv[2]), split(xv[1]), split(xv[3]),
                    split(xv[4]), split(xv[6]), split(xv[5]), split(xv[7])};
      *reinterpret_cast<h8*>(a.t8 + ((static_cast<size_t>(tile) * nb + kb) * kWave + lane) * 16) = f;
    }
  }
}

// B operands and block scales of one 16-row tile, one block pair, one matrix.
struct PairOps {
  h8 b0, b1;
  float d0, d1;
};

__device__ __forceinline__ PairOps pair_ops(const uint8_t* row, bool q4, int m, int g) {
  PairOps o;
  const uint32_t* P = reinterpret_cast<const uint32_t*>(row);
  if (q4) {
    const uint32_t* pp = P + m * 9;
    o.d0 = f16lo(pp[0]);
    o.d1 = f16hi(pp[4]);
    o.b0 = q4_operand(__builtin_amdgcn_alignbyte(pp[g + 1], pp[g], 2));
    o.b1 = q4_operand(pp[5 + g]);
  } else {
    const uint32_t* pp = P + m * 17;
    o.d0 = f16lo(pp[0]);
    o.d1 = f16hi(pp[8]);
    o.b0 = q8_operand(__builtin_amdgcn_alignbyte(pp[2 * g + 1], pp[2 * g], 2),
                      __builtin_amdgcn_alignbyte(pp[2 * g + 2], pp[2 * g + 1], 2));
    o.b1 = q8_operand(pp[9 + 2 * g], pp[10 + 2 * g]);
  }
  return o;
}

// Phase 3 of both batched kernels: the eight waves' partial sums combined in LDS in a fixed order
// (the operand LDS is reused), the scale undone, then the epilogue (one K split) or the split's sums
// to the workspace for finalize_kernel.
template <int EPI, int RT, int NT>
__device__ __forceinline__ void combine_and_store(const MArgs& a, const MJob& jb, uint8_t* lb,
                                                  float (&acc)[NT][RT][EPI == kEpiSwiglu ? 2 : 1][2], int wave,
                                                  int lane, int row0, int tile, int ks, int s0) {
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int ROWS = RT * kTileRows;
  const int S = a.ksplit;
  const int nloc = min(NT * kSeqTile, a.B - s0);  // this workgroup's sequences s0 .. s0 + nloc - 1
  __syncthreads();
  float* red = reinterpret_cast<float*>(lb);  // [wave][t][r][mt][lane][2]
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) {
        float* p = red + ((((wave * NT + t) * RT + r) * NM + mt) * kWave + lane) * 2;
        p[0] = acc[t][r][mt][0];
        p[1] = acc[t][r][mt][1];
      }
  __syncthreads();
  constexpr int wstep = NT * RT * NM * kWave * 2;  // floats per wave
  // the workgroup's sums for output o = (sequence, row) of matrix mt, waves in order
  auto wg_sum = [&](int o, int mt) {
    const int sq = o / ROWS, jr = o % ROWS;
    const int t = sq / kSeqTile, s = sq % kSeqTile, r = jr / kTileRows, jj = jr % kTileRows;
    const int src = (jj + 16 * (s >> 1)) * 2 + (s & 1);  // lane holding D rows 4(l/16).., slot
    const float* p = red + (((t * RT + r) * NM + mt) * kWave) * 2 + src;
    float sum = p[0];
#pragma unroll
    for (int w = 1; w < kWavesM; ++w) sum += p[w * wstep];
    return sum;
  };
  auto epilogue = [&](int o, const float (&v)[NM]) {
    const int sq = s0 + o / ROWS, row = row0 + o % ROWS;
    float* y = jb.y + sq * jb.ldy + row;
    if (EPI == kEpiResidual) {
      *y = *y + v[0];
    } else if (EPI == kEpiSwiglu) {
      *y = silu_m(v[0]) * v[NM - 1];
    } else {
      *y = v[0];
    }
  };
  if (S == 1) {
    for (int o = threadIdx.x; o < ROWS * nloc; o += kT) {
      if (row0 + o % ROWS >= jb.rows) continue;
      float v[NM];
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) v[mt] = wg_sum(o, mt) * a.post[s0 + o / ROWS];
      epilogue(o, v);
    }
    return;
  }
  // split-K: this split's sums go to the workspace; finalize_kernel adds the splits in index order
  // and applies the epilogue (the kernel boundary makes every split visible, no fences needed).
  const size_t gsz = static_cast<size_t>(a.B) * ROWS * NM;
  float* mine = a.part + (static_cast<size_t>(tile) * S + ks) * gsz + static_cast<size_t>(s0) * ROWS * NM;
  for (int o = threadIdx.x; o < ROWS * nloc; o += kT) {
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) mine[o * NM + mt] = wg_sum(o, mt);
  }
}

// RT row tiles of 16 rows per workgroup, NT sequence tiles of 8 sequences per launch.
template <int EPI, int RT, int NT>
__global__ __launch_bounds__(kT) void gemv_mfma_kernel(MArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lb[];
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int ROWS = RT * kTileRows;
  const int K = a.K, nb = K >> 5, np = K >> 6;
  const int S = a.ksplit, tile = blockIdx.x / S, ks = blockIdx.x % S;
  const MJob jb = find_mjob(a, tile);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x & (kWave - 1);
  const int row0 = (tile - jb.tile_begin) * ROWS;
  const uint32_t rb = static_cast<uint32_t>(jb.row_bytes), rs = a.row_stride;
  const bool q4 = jb.qtype == EF_QTYPE_Q4_0;
  const uint32_t pb = q4 ? 36u : 68u;  // bytes per block pair
  // this workgroup's block pairs [p0, p1): multiples of 4 pairs, so their bytes are 16-byte units
  const int p0 = ks * a.pairs_per_split, p1 = min(np, p0 + a.pairs_per_split);

  // 1. wave w fetches the split's bytes of rows w, w + 8, ... (rows past the end read as zeros)
  {
    const uint32_t mat_bytes = static_cast<uint32_t>(jb.rows) * rb;
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(jb.W, mat_bytes);
    const __amdgpu_buffer_rsrc_t r2 = make_rsrc(EPI == kEpiSwiglu ? jb.W2 : jb.W, mat_bytes);
    const uint32_t bytes = static_cast<uint32_t>(p1 - p0) * pb;
#pragma unroll
    for (int r = 0; r < ROWS / kWavesM; ++r) {
      const int jr = wave + kWavesM * r;
      const uint32_t src = static_cast<uint32_t>(row0 + jr) * rb + static_cast<uint32_t>(p0) * pb;
      dma_copy<kNonTemporal>(r1, src, lb + jr * rs, bytes, lane);
      if (EPI == kEpiSwiglu) dma_copy<kNonTemporal>(r2, src, lb + a.w_stride + jr * rs, bytes, lane);
    }
  }

  // 2. this wave's block pairs m = wave, wave + 8, ...; the A fragments of the next pair are
  //    loaded while the current pair's products run
  // sequence tiles blockIdx.y * NT .. + NT - 1 of the launch (a grid row per group of tiles)
  const int j = lane & 15, g = lane >> 4, s0 = blockIdx.y * NT * kSeqTile;
  const size_t tstride = static_cast<size_t>(nb) * kWave * 16;  // bytes per sequence tile
  const uint8_t* tab = (q4 ? a.t4 : a.t8) + static_cast<size_t>(lane) * 16 + blockIdx.y * NT * tstride;
  float acc[NT][RT][NM][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) acc[t][r][mt][0] = acc[t][r][mt][1] = 0.0f;
  const f4v Z = {0.0f, 0.0f, 0.0f, 0.0f};
  h8 A[2][NT][2];
  auto load_a = [&](h8 (&dst)[NT][2], int m) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint8_t* tp = tab + t * tstride + static_cast<size_t>(2 * m) * kWave * 16;
      dst[t][0] = *reinterpret_cast<const h8*>(tp);
      dst[t][1] = *reinterpret_cast<const h8*>(tp + kWave * 16);
    }
  };
  // All products of a row tile are issued before any result is read, so the matrix pipe stays
  // full instead of draining on every accumulator update.
  auto compute = [&](const h8 (&Ax)[NT][2], int m) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) {
        const PairOps o = pair_ops(lb + mt * a.w_stride + (r * kTileRows + j) * rs, q4, m - p0, g);
        f4v D[NT][2];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          D[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ax[t][0], o.b0, Z, 0, 0, 0);
          D[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ax[t][1], o.b1, Z, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          acc[t][r][mt][0] = fmaf(o.d0, D[t][0][0] + D[t][0][1], acc[t][r][mt][0]);
          acc[t][r][mt][1] = fmaf(o.d0, D[t][0][2] + D[t][0][3], acc[t][r][mt][1]);
          acc[t][r][mt][0] = fmaf(o.d1, D[t][1][0] + D[t][1][1], acc[t][r][mt][0]);
          acc[t][r][mt][1] = fmaf(o.d1, D[t][1][2] + D[t][1][3], acc[t][r][mt][1]);
        }
      }
    }
  };
  if (p0 + wave < p1) load_a(A[0], p0 + wave);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // weight rows (and the first fragments) landed
  __syncthreads();
  for (int m = p0 + wave; m < p1; m += 2 * kWavesM) {
    const int m1 = m + kWavesM;
    if (m1 < p1) load_a(A[1], m1);
    compute(A[0], m);
    if (m1 < p1) {
      if (m1 + kWavesM < p1) load_a(A[0], m1 + kWavesM);
      compute(A[1], m1);
    }
  }

  combine_and_store<EPI, RT, NT>(a, jb, lb, acc, wave, lane, row0, tile, ks, s0);
}

struct FinArgs {
  MJob job[kMaxJobsM];
  int n_jobs, B, rows_wg, S, total;  // total = groups * rows_wg * B outputs
  const float* part;
  const float* post;
};

// One output (sequence, row) per thread: the splits' sums in index order, the scale, the epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void finalize_kernel(FinArgs a) {
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.total) return;
  const int per_group = a.rows_wg * a.B;
  const int tile = idx / per_group, o = idx % per_group;
  MJob jb = a.job[0];
  for (int i = 1; i < a.n_jobs; ++i)
    if (tile >= a.job[i].tile_begin) jb = a.job[i];
  const int sq = o / a.rows_wg, row = (tile - jb.tile_begin) * a.rows_wg + o % a.rows_wg;
  if (row >= jb.rows) return;
  const size_t gsz = static_cast<size_t>(per_group) * NM;
  const float* p = a.part + static_cast<size_t>(tile) * a.S * gsz + static_cast<size_t>(o) * NM;
  float v[NM];
#pragma unroll
  for (int mt = 0; mt < NM; ++mt) {
    float sum = p[mt];
    for (int k = 1; k < a.S; ++k) sum += p[k * gsz + mt];
    v[mt] = sum * a.post[sq];
  }
  float* y = jb.y + sq * jb.ldy + row;
  if (EPI == kEpiResidual) {
    *y = *y + v[0];
  } else if (EPI == kEpiSwiglu) {
    *y = silu_m(v[0]) * v[NM - 1];
  } else {
    *y = v[0];
  }
}

template <int EPI, int RT>
void* pick_mfma_nt(int nt) {
  if (nt <= 1) return reinterpret_cast<void*>(&gemv_mfma_kernel<EPI, RT, 1>);
  if (nt <= 2) return reinterpret_cast<void*>(&gemv_mfma_kernel<EPI, RT, 2>);
  if (nt <= 4) return reinterpret_cast<void*>(&gemv_mfma_kernel<EPI, RT, 4>);
  return reinterpret_cast<void*>(&gemv_mfma_kernel<EPI, RT, 8>);
}

template <int EPI>
void* pick_mfma(int rt, int nt) {
  if constexpr (EPI == kEpiSwiglu) {
    return pick_mfma_nt<EPI, 1>(nt);
  } else {
    return rt == 2 ? pick_mfma_nt<EPI, 2>(nt) : pick_mfma_nt<EPI, 1>(nt);
  }
}

}  // namespace

// Sequence tiles the kernels are instantiated for: 1, 2, 4 or 8 (a launch covers up to 64 sequences).
static int tiles_for(int nseq) {
  const int nt = (std::min(nseq, kMaxTiles * kSeqTile) + kSeqTile - 1) / kSeqTile;
  return nt <= 1 ? 1 : (nt <= 2 ? 2 : (nt <= 4 ? 4 : 8));
}

namespace {

// Shape decisions of one batched launch and the workspace they need.
struct Plan {
  bool ok = false;
  bool q4 = false, q8 = false;
  int nm = 1, NT = 1, RT = 1, groups = 0, S = 1, pps = 0, chunk = 0;
  int NTW = 1, SG = 1;  // sequence tiles per workgroup, and workgroup rows of the grid (NT = NTW * SG)
  size_t max_rb = 0, tab = 0, part_off = 0, bytes = 0, lds = 0;
  uint32_t row_stride = 0, w_stride = 0;
};

// LDS row stride for `pairs` block pairs per row: an odd number of 16-byte units, so the 16 rows a
// B fragment reads fall in distinct banks.
uint32_t odd_stride(size_t pairs, size_t pb, size_t max_rb) {
  const size_t bytes = std::min<size_t>(pairs * pb, max_rb);
  const size_t units = bytes / 16 + ((bytes / 16) % 2 == 0 ? 1 : 2);
  return static_cast<uint32_t>(units * 16);
}

int groups_for(const GemvJob* jobs, int n_jobs, int rows_wg) {
  int g = 0;
  for (int j = 0; j < n_jobs; ++j) g += static_cast<int>((jobs[j].W->rows + rows_wg - 1) / rows_wg);
  return g;
}

Plan plan_mfma(const GemvJob* jobs, int n_jobs, int epi, int batch, size_t ldx) {
  Plan p;
  if (mfma_gemv_disabled() || batch < 2 || n_jobs < 1 || n_jobs > kMaxJobsM) return p;
  const size_t K = jobs[0].W->cols;
  if (K % 256 != 0) return p;  // pairs come in 16-byte multiples of 4 for the LDS-DMA row copies
  for (int j = 0; j < n_jobs; ++j) {
    if (jobs[j].W->qtype != EF_QTYPE_Q4_0 && jobs[j].W->qtype != EF_QTYPE_Q8_0) return Plan{};
    p.q4 = p.q4 || jobs[j].W->qtype == EF_QTYPE_Q4_0;
    p.q8 = p.q8 || jobs[j].W->qtype == EF_QTYPE_Q8_0;
    p.max_rb = std::max(p.max_rb, jobs[j].W->row_bytes);
    if (jobs[j].x != jobs[0].x || (jobs[j].ldx ? jobs[j].ldx : ldx) != (jobs[0].ldx ? jobs[0].ldx : ldx))
      return p;  // one activation matrix per launch
  }
  const size_t xld = jobs[0].ldx ? jobs[0].ldx : ldx;
  if (reinterpret_cast<uintptr_t>(jobs[0].x) % 16 != 0 || xld % 4 != 0) return p;
  p.nm = epi == kEpiSwiglu ? 2 : 1;
  p.chunk = std::min(batch, kMaxTiles * kSeqTile);
  p.NT = tiles_for(batch);
  // Two row tiles halve the fragment re-reads of large batches; SwiGLU already applies every
  // fragment to two matrices (and a second row tile would not fit in registers).
  p.RT = p.NT >= 4 && p.nm == 1 ? 2 : 1;
  const int rows_wg = p.RT * kTileRows;
  p.groups = groups_for(jobs, n_jobs, rows_wg);
  // Every workgroup streams the activation fragments of its K range through its CU's L2 port
  // (B x K x 4 bytes for the whole range).  Split K (one extra, tiny finalize launch) only when
  // that exceeds 512 KB; splits are multiples of 4 block pairs, at least 8 (one per wave).
  const int np = static_cast<int>(K / 64);
  const size_t frag_bytes = static_cast<size_t>(p.chunk) * K * 4;
  int S = static_cast<int>((frag_bytes + (512u << 10) - 1) / (512u << 10));
  S = std::max(1, std::min({S, np / 8, 8}));
  int pps = (np + S - 1) / S;
  pps = (pps + 3) / 4 * 4;
  p.S = (np + pps - 1) / pps;
  p.pps = pps;
  // Sequence groups: a workgroup takes NTW of the launch's NT sequence tiles, halving NTW (and the
  // fragment bytes each workgroup streams) until every CU has a workgroup.  A workgroup's time is
  // mostly its fragment stream, so small row counts (q / o at 64 sequences: 64 workgroups of 32
  // rows) finish in a fraction of the time on 4x the CUs.
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  p.NTW = p.NT;
  while (p.NTW > 1 && static_cast<long>(p.groups) * p.S * (p.NT / p.NTW) < cus) p.NTW /= 2;
  p.SG = p.NT / p.NTW;
  const size_t pb = p.q8 ? 68 : 36;
  p.row_stride = odd_stride(static_cast<size_t>(pps), pb, p.max_rb);
  p.w_stride = static_cast<uint32_t>(rows_wg * p.row_stride);
  p.lds = std::max<size_t>(static_cast<size_t>(p.nm) * p.w_stride,
                           static_cast<size_t>(kWavesM) * p.NTW * p.RT * p.nm * kWave * 2 * 4);
  const size_t lim = ctx().lds_per_block > 0 ? ctx().lds_per_block : 65536;
  if (p.lds > lim) return p;
  // Layout: the A tables, the scales, the split-K partial sums.
  p.tab = static_cast<size_t>(p.NT) * (K / 32) * kWave * 16;
  size_t off = (p.q4 ? p.tab : 0) + (p.q8 ? p.tab : 0) + kMaxTiles * kSeqTile * sizeof(float);
  off = (off + 255) & ~size_t(255);
  p.part_off = off;
  if (p.S > 1) off += static_cast<size_t>(p.groups) * p.S * p.chunk * rows_wg * p.nm * sizeof(float);
  p.bytes = off;
  p.ok = true;
  return p;
}

}  // namespace

size_t gemv_mfma_workspace_bytes(const GemvJob* jobs, int n_jobs, int epi, int batch, size_t ldx) {
  const Plan p = plan_mfma(jobs, n_jobs, epi, batch, ldx);
  return p.ok ? p.bytes : 0;
}

int launch_gemv_mfma(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch, size_t ldx,
                     size_t ldy, void* ws, size_t ws_bytes, hipStream_t stream, bool* taken) {
  *taken = false;
  const Plan pl = plan_mfma(jobs, n_jobs, epi, batch, ldx);
  if (!pl.ok) return EF_HIP_OK;
  if (norm_w != nullptr && reinterpret_cast<uintptr_t>(norm_w) % 16 != 0) return EF_HIP_OK;
  const size_t K = jobs[0].W->cols;
  const size_t xld = jobs[0].ldx ? jobs[0].ldx : ldx;
  // workspace: the caller's, else a stream-ordered allocation freed after the launches
  void* buf = ws;
  bool own = false;
  if (buf == nullptr || ws_bytes < pl.bytes) {
    EFH_HIP(hipMallocAsync(&buf, pl.bytes, stream));
    own = true;
  }
  uint8_t* base = static_cast<uint8_t*>(buf);
  uint8_t* t4 = pl.q4 ? base : nullptr;
  uint8_t* t8 = pl.q8 ? base + (pl.q4 ? pl.tab : 0) : nullptr;
  float* post = reinterpret_cast<float*>(base + (pl.q4 ? pl.tab : 0) + (pl.q8 ? pl.tab : 0));
  int rc = EF_HIP_OK;
  MArgs a{};
  a.row_stride = pl.row_stride;
  a.w_stride = pl.w_stride;
  a.ksplit = pl.S;
  a.pairs_per_split = pl.pps;
  a.part = reinterpret_cast<float*>(base + pl.part_off);
  void* fn = epi == kEpiStore ? pick_mfma<kEpiStore>(pl.RT, pl.NTW)
                              : (epi == kEpiResidual ? pick_mfma<kEpiResidual>(pl.RT, pl.NTW)
                                                     : pick_mfma<kEpiSwiglu>(pl.RT, pl.NTW));
  const int rows_wg = pl.RT * kTileRows;
  for (int b0 = 0; b0 < batch && rc == EF_HIP_OK; b0 += pl.chunk) {
    const int nb = std::min(pl.chunk, batch - b0);
    PrepArgs p{};
    p.x = jobs[0].x + b0 * xld;
    p.ldx = static_cast<long>(xld);
    p.K = static_cast<int>(K);
    p.B = nb;
    p.norm_w = norm_w;
    p.eps = eps;
    p.t4 = t4;
    p.t8 = t8;
    p.post = post;
    hipLaunchKernelGGL(xfrag_kernel, dim3(kPrepSplit, pl.NT), dim3(kTP), 0, stream, p);  // tiles past B get zeros
    a.n_jobs = n_jobs;
    a.K = static_cast<int>(K);
    a.B = nb;
    a.n_tiles = pl.NT;
    a.t4 = t4;
    a.t8 = t8;
    a.post = post;
    int tiles = 0;
    for (int j = 0; j < n_jobs; ++j) {
      MJob& d = a.job[j];
      const size_t yld = jobs[j].ldy ? jobs[j].ldy : ldy;
      d.W = jobs[j].W->dev;
      d.W2 = jobs[j].W2 ? jobs[j].W2->dev : nullptr;
      d.y = jobs[j].y + b0 * yld;
      d.rows = static_cast<int>(jobs[j].W->rows);
      d.qtype = jobs[j].W->qtype;
      d.row_bytes = static_cast<int>(jobs[j].W->row_bytes);
      d.ldy = static_cast<long>(yld);
      d.tile_begin = tiles;
      tiles += (d.rows + rows_wg - 1) / rows_wg;
    }
    void* params[] = {&a};
    // the chunk's sequences cover ceil(nb / 8) tiles; grid rows past them would have no sequences
    const int sg = std::min(pl.SG, (nb + pl.NTW * kSeqTile - 1) / (pl.NTW * kSeqTile));
    hipError_t e = hipLaunchKernel(fn, dim3(tiles * pl.S, sg), dim3(kT), params, pl.lds, stream);
    if (e != hipSuccess) {
      rc = fail_hip(e, "gemv_mfma_kernel");
      break;
    }
    if (pl.S > 1) {
      FinArgs f{};
      for (int j = 0; j < n_jobs; ++j) f.job[j] = a.job[j];
      f.n_jobs = n_jobs;
      f.B = nb;
      f.rows_wg = rows_wg;
      f.S = pl.S;
      f.total = tiles * rows_wg * nb;
      f.part = a.part;
      f.post = post;
      void* fin = epi == kEpiStore ? reinterpret_cast<void*>(&finalize_kernel<kEpiStore>)
                                   : (epi == kEpiResidual ? reinterpret_cast<void*>(&finalize_kernel<kEpiResidual>)
                                                          : reinterpret_cast<void*>(&finalize_kernel<kEpiSwiglu>));
      void* fparams[] = {&f};
      e = hipLaunchKernel(fin, dim3((f.total + 255) / 256), dim3(256), fparams, 0, stream);
      if (e != hipSuccess) rc = fail_hip(e, "finalize_kernel");
    }
  }
  if (own) {
    const hipError_t e = hipFreeAsync(buf, stream);
    if (e != hipSuccess && rc == EF_HIP_OK) rc = fail_hip(e, "hipFreeAsync");
  }
  if (rc == EF_HIP_OK) *taken = true;
  return rc;
}

}  // namespace efh
