// Packed Q4_0 / Q8_0 GEMV for batches of sequences on the matrix cores, in one launch that reads the
// packed rows in place (the replacement of kern::matvec_jobs over many sequences,
// src/qkernels.cpp:280-297).  K = 2048 (every product whose input is the hidden state).
//
// Work split.  A workgroup (8 waves) owns 16 sequences and a run of up to 6 row tiles (16 rows each)
// of one matrix, and is the only workgroup computing those outputs.  The workgroups of one row run
// get ids of one residue mod 8, which the dispatcher places on one XCD, so each weight byte comes
// from HBM once and the run's sequence groups share it through that XCD's L2.  B = 64 over 5632 rows
// is 64 runs of 5 or 6 tiles x 4 sequence groups: 256 workgroups, one per CU.  Wave w owns the K
// blocks [8w, 8w + 8) of every tile and works alone until the final combine: it has a private LDS
// region, its own per-sequence scale, and no workgroup barrier before the combine.
//
// Activations (A operand of v_mfma_f32_16x16x32_f16, 16 sequences x 32 weights).  The wave fetches
// its K range of its 16 sequences' FP32 rows (and of the RMSNorm weights) with LDS-DMA, one 1 KB
// row piece per instruction, reads its fragment values back (lane l: sequence l % 16, lane group
// g = l / 16), takes v = norm_w * x (or x), scales by a power of two keeping |v'| < 2^15 (from the
// maximum over its own range) and splits v' exactly into fp16 hi + lo (v' - hi - lo below
// 2^-22 |v'|), two fused mixed-precision instructions per value.  The fragments stay in 64 VGPRs
// for the whole launch, shared by every row tile.  1 / rms (kern::rmsnorm's statistic, a double sum
// of x^2 combined over the waves) scales the results in the epilogue.
//
// Weights (B operand, 32 weights x 16 rows).  The wave fetches its K range of each tile's 16 rows
// (9 / 17 coalesced 16-byte pieces per row for Q4_0 / Q8_0) into registers, the first tiles at
// entry, and writes each tile into one of two LDS slots before computing it, rows an odd number of
// 16-byte units apart (the 16 rows one B fragment reads fall in distinct banks).  Lane (row
// n = l % 16, group g) then reads aligned dwords of row n per block pair (36 / 68 bytes):
//   Q4_0 pair (dwords 0..8): dw0 = d | c0 c1, dw1..dw3 = c2..c13, dw4 = c14 c15 | d', dw5..dw8 = c'0..c'15.
//     Even block: bytes c4g .. c4g+3 = alignbyte(dw(g+1), dw(g), 2).  Odd block: dw(5 + g).
//   Q8_0 pair (dwords 0..16): dw0 = d | q0 q1, dw1..dw8 = q2..q31 | d', dw9..dw16 = q'0..q'31.
//     Even block: q8g .. q8g+7 from dw(2g) .. dw(2g+2) by two alignbytes.  Odd block: dw(9+2g), dw(10+2g).
//   The scales are the low half of dw0 and the high half of dw4 (dw8).
// Lane group g takes the codes of weights 4g..4g+3 and 16+4g..19+4g (Q4_0) or 8g..8g+7 (Q8_0), the
// slot orders of qfrag.h, and the A fragments follow the same order.  Per block pair the products
// run software-pipelined: D = A_hi B, D += A_lo B through the accumulator input, and d D enters an
// FP32 accumulator per output, while the next pair's codes become B operands.
//
// Combine.  Each wave's sums cover its K range; after the last tile every wave multiplies them by
// its power of two and the 8 partials of every output are added through LDS in wave order (a fixed
// order: same bits every call, for any batch); then 1 / rms (norm) and the epilogue (store, residual
// add, SwiGLU of a gate and an up matrix).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "gemv.h"
#include "qfrag.h"

namespace efh {
namespace {

constexpr int kGMaxTiles = 6;       // row tiles (16 rows) per workgroup
constexpr int kGK = 2048;           // the K this kernel serves
constexpr int kGMaxJobs = 4;

template <bool Q4>
struct QShape {
  static constexpr int kBlock = Q4 ? 18 : 34;
  static constexpr int kRowBytes = kGK / 32 * kBlock;          // 1152 / 2176
  static constexpr int kStride = ((kRowBytes / 16) | 1) * 16;  // LDS row stride: 1168 / 2192
  static constexpr int kPiecesRow = kRowBytes / 16;
  static constexpr int kPieces = 2 * kPiecesRow;               // 16-byte pieces of a wave's two rows
  static constexpr int kLoads = (kPieces + kWave - 1) / kWave;  // 3 / 5 lane loads per tile
  static constexpr int kTileLds = 16 * kStride;
};

struct GJob {
  const uint8_t* W;
  const uint8_t* W2;  // SwiGLU: the up matrix
  float* y;
  long ldy;
  int rows, qtype;
  int g0, groups, tiles;  // row runs [g0, g0 + groups) of the launch over the job's ceil(rows / 16) tiles
};

struct GArgs {
  GJob job[kGMaxJobs];
  int n_jobs, n_sg, B, xcd;
  const float* x;
  long ldx;
  const float* norm_w;
  float eps;
};

typedef __attribute__((address_space(3))) void lds_void;

// fp16 hi and lo parts of v0 * s and v1 * s (s a power of two), packed two per dword:
// hi = RN(v s), lo = RN(v s - hi), each one fused mixed-precision operation (v s - hi is exact in
// its FP32 intermediate), so v s - hi - lo is below 2^-22 |v s|.
__device__ __forceinline__ void split2(float v0, float v1, float s, uint32_t& hi, uint32_t& lo) {
  asm("v_fma_mixlo_f16 %0, %2, %4, 0 op_sel_hi:[0,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0 op_sel_hi:[0,0,0]\n\t"
      "v_fma_mixlo_f16 %1, %2, %4, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %1, %3, %4, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(hi), "=&v"(lo)
      : "v"(v0), "v"(v1), "v"(s));
}

// Workgroup shapes: NW waves split the K blocks, NBW = 64 / NW each.  Each wave owns a private LDS
// region: first its 16 activation rows of its K range (NBW x 128 bytes each, rows an odd number of
// 16-byte units apart so that the 16 rows of one fragment read fall in distinct banks), then, once
// its fragments are formed, two slots of its K range of a row tile's 16 rows (per matrix; rows an
// odd number of 16-byte units apart again).  No wave reads another wave's region, so nothing before
// the final combine waits for the workgroup.
template <int NW>
struct Wg {
  static constexpr int kT = NW * kWave;
  static constexpr int kNBW = kGK / 32 / NW;                  // 8 (8 waves) or 4 (16 waves)
  static constexpr int kARow = kNBW * 128 + 16;
  static constexpr int kWRowQ8 = ((kNBW * 34 + 15) / 16) * 16;
  static constexpr int kAWave = 16 * kARow > 2 * 2 * 16 * kWRowQ8 ? 16 * kARow : 2 * 2 * 16 * kWRowQ8;
  static constexpr int kNormOff = NW * kAWave;
  static constexpr int kLds = kNormOff + NW * kNBW * 128;
  static constexpr int kRed = NW * kGMaxTiles * kWave * 16;  // the waves' partial sums, per matrix
};

template <bool Q4, int NW>
struct WShape {  // one wave's K range of a 16-row tile, whole 16-byte pieces per row
  static constexpr int kPiecesRow = (Wg<NW>::kNBW * (Q4 ? 18 : 34) + 15) / 16;  // 9/5 (Q4_0), 17/9 (Q8_0)
  static constexpr int kRow = kPiecesRow * 16;
  static constexpr int kTile = 16 * kRow;
  static constexpr int kLoads = (16 * kPiecesRow + kWave - 1) / kWave;
};

// Weight tiles whose rows are requested at entry (registers): as many as 72 VGPRs hold (two waves
// per SIMD), 24 with four.
template <bool Q4, int NM, int NW>
constexpr int pre_tiles() {
  const int per = NM * WShape<Q4, NW>::kLoads * 4;
  const int p = (NW == 16 ? 24 : 72) / per;
  return p < 1 ? 1 : (p > kGMaxTiles ? kGMaxTiles : p);
}

template <int EPI, bool NORM, bool Q4, int NW>
__device__ __forceinline__ void gemv_body(const GArgs& a, const GJob& jb, int t_begin, int ntw, int sg,
                                          uint8_t* lds, float* s_postw, double* s_ss) {
  using QS = QShape<Q4>;
  using WS = WShape<Q4, NW>;
  using G = Wg<NW>;
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int kPre = pre_tiles<Q4, NM, NW>();
  constexpr int kSlot = NM * WS::kTile;
  constexpr int kGNBW = G::kNBW;
  constexpr int kGW = NW;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x & (kWave - 1);
  const int m = lane & 15, g = lane >> 4;
  const int kb0 = wave * kGNBW;
  uint8_t* region = lds + wave * G::kAWave;

  // ---- 1. activations: this wave's K range of its 16 sequences, one 1 KB row piece per LDS-DMA
  //      instruction (rows past the batch read zeros), and its 1 KB of norm weights
  const int s_base = sg * 16;
  const int n_valid = min(16, a.B - s_base);
  const uint32_t ldxb = static_cast<uint32_t>(a.ldx) * 4u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + static_cast<size_t>(s_base) * a.ldx, n_valid * ldxb);
  // one instruction per row: NBW x 128 bytes = 64 (8 waves) or 32 (16 waves) lanes of 16 bytes
  const uint32_t kofs = static_cast<uint32_t>(kb0) * 128u + 16u * lane;  // byte offset in a row
  const bool alane = lane < kGNBW * 8;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (alane)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(region + r * G::kARow), 16, r * ldxb + kofs, 0, 0, 0);
  uint8_t* nbuf = lds + G::kNormOff + wave * (kGNBW * 128);
  if constexpr (NORM) {
    if (alane)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(a.norm_w, kGK * 4u), (lds_void*)nbuf, 16, kofs, 0, 0, 0);
  }

  // ---- 2. the first kPre tiles: this wave's K range of their 16 rows (16-byte pieces, 9 / 17 per
  //      row), both matrices, into registers
  const int row0 = t_begin * 16;
  const int live_rows = min(ntw * 16, jb.rows - row0);
  const uint32_t chunk = static_cast<uint32_t>(live_rows) * QS::kRowBytes;  // rows past it read zeros
  __amdgpu_buffer_rsrc_t rW[NM];
  rW[0] = make_rsrc(jb.W + static_cast<size_t>(row0) * QS::kRowBytes, chunk);
  if constexpr (NM == 2) rW[1] = make_rsrc(jb.W2 + static_cast<size_t>(row0) * QS::kRowBytes, chunk);
  uint32_t goff[WS::kLoads];
  bool lv[WS::kLoads];
#pragma unroll
  for (int i = 0; i < WS::kLoads; ++i) {
    const int P = i * kWave + lane;
    lv[i] = P < 16 * WS::kPiecesRow;
    const int r = P / WS::kPiecesRow, c = P % WS::kPiecesRow;
    goff[i] = lv[i] ? static_cast<uint32_t>(r * QS::kRowBytes + kb0 * (Q4 ? 18 : 34) + 16 * c) : 0x80000000u;
  }
  v4i stg[kPre][NM][WS::kLoads];
  auto fetch = [&](v4i (&dst)[NM][WS::kLoads], int t) {
    const uint32_t tb = static_cast<uint32_t>(t) * 16u * QS::kRowBytes;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int i = 0; i < WS::kLoads; ++i)
        dst[mt][i] = __builtin_amdgcn_raw_buffer_load_b128(rW[mt], goff[i] + (lv[i] ? tb : 0u), 0, 0);
  };
#pragma unroll
  for (int t = 0; t < kPre; ++t) fetch(stg[t], t);

  // ---- 3. fragment values from LDS: lane (m, g) takes, per block, the 8 values of its slots
  //      (Q4_0: 4g .. 4g+3 and 16+4g .. 19+4g; Q8_0: 8g .. 8g+7).  The compiler does not order LDS
  //      reads after LDS-DMA loads: wait here until only the weight loads issued after the DMAs
  //      are outstanding (vector-memory operations retire in order).
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPre * NM * WS::kLoads) : "memory");
  const uint8_t* arow = region + m * G::kARow;
  const uint32_t p0 = Q4 ? 16u * g : 32u * g, p1 = Q4 ? 64u + 16u * g : 32u * g + 16u;
  f4v F[kGNBW][2];
#pragma unroll
  for (int bi = 0; bi < kGNBW; ++bi) {
    F[bi][0] = *reinterpret_cast<const f4v*>(arow + bi * 128 + p0);
    F[bi][1] = *reinterpret_cast<const f4v*>(arow + bi * 128 + p1);
    if constexpr (NORM) {  // v = norm_w * x: the tables' values; 1 / rms scales the results
      const f4v W0 = *reinterpret_cast<const f4v*>(nbuf + bi * 128 + p0);
      const f4v W1 = *reinterpret_cast<const f4v*>(nbuf + bi * 128 + p1);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        F[bi][0][c] = W0[c] * F[bi][0][c];
        F[bi][1][c] = W1[c] * F[bi][1][c];
      }
    }
  }
  // statistics of this wave's range: max |v| per sequence (its own power of two), and for the
  // norm the double sum of x^2 (kern::rmsnorm's statistic, combined over the waves at the end)
  float pre;
  {
    float ax = 0.0f;
#pragma unroll
    for (int bi = 0; bi < kGNBW; ++bi)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c) ax = fmaxf(ax, fabsf(F[bi][h][c]));
    ax = fmaxf(ax, __shfl_xor(ax, 16, kWave));  // the four lane groups of a sequence
    ax = fmaxf(ax, __shfl_xor(ax, 32, kWave));
    if constexpr (NORM) {
      double ss = 0.0;
      const uint8_t* xr = region + m * G::kARow;
#pragma unroll
      for (int bi = 0; bi < kGNBW; ++bi)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f4v xv = *reinterpret_cast<const f4v*>(xr + bi * 128 + (h ? p1 : p0));
#pragma unroll
          for (int c = 0; c < 4; ++c) ss += static_cast<double>(xv[c]) * static_cast<double>(xv[c]);
        }
      ss += __shfl_xor(ss, 16, kWave);
      ss += __shfl_xor(ss, 32, kWave);
      if (lane < 16) s_ss[wave * 16 + lane] = ss;
    }
    const float bound = ax * 1.0001f;
    int e = 0;
    if (bound > 0.0f && bound <= 3.0e38f) e = ilogbf(bound) - 14;  // bound * 2^-e < 2^15
    pre = ldexpf(1.0f, -e);
    if (lane < 16) s_postw[wave * 16 + lane] = ldexpf(1.0f, e);
  }
  h8 Ahi[kGNBW], Alo[kGNBW];
  {
    // slot pairs of the fragment dwords: Q4_0 (F0.x F0.z) (F1.x F1.z)/16 (F0.y F0.w) (F1.y F1.w)/16
    // (the high-nibble slots divided by 16); Q8_0 (F0.x F0.z) (F0.y F0.w) (F1.x F1.z) (F1.y F1.w)
    const float pre16 = pre * 0.0625f;
#pragma unroll
    for (int bi = 0; bi < kGNBW; ++bi) {
      const f4v P0 = F[bi][0], P1 = F[bi][1];
      uint32_t hi[4], lo[4];
      if constexpr (Q4) {
        split2(P0[0], P0[2], pre, hi[0], lo[0]);
        split2(P1[0], P1[2], pre16, hi[1], lo[1]);
        split2(P0[1], P0[3], pre, hi[2], lo[2]);
        split2(P1[1], P1[3], pre16, hi[3], lo[3]);
      } else {
        split2(P0[0], P0[2], pre, hi[0], lo[0]);
        split2(P0[1], P0[3], pre, hi[1], lo[1]);
        split2(P1[0], P1[2], pre, hi[2], lo[2]);
        split2(P1[1], P1[3], pre, hi[3], lo[3]);
      }
      __builtin_memcpy(&Ahi[bi], hi, 16);
      __builtin_memcpy(&Alo[bi], lo, 16);
    }
  }

  // ---- 4. row tiles.  Per tile the wave writes its staged rows into its slot, requests the rows
  //      kPre tiles on, reads all its code and scale words, then runs its block pairs
  //      software-pipelined: pair p + 1's codes become B operands on the vector ALU while pair p's
  //      products run on the matrix core.
  f4v acc[kGMaxTiles][NM];  // set by each tile's first pair (tiles a workgroup skips stay unset)
  const f4v Z = {0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int kPairs = kGNBW / 2;
  constexpr int kDw = Q4 ? 5 : 7;  // LDS words a lane reads per pair
#pragma unroll
  for (int t = 0; t < kGMaxTiles; ++t) {
    if (t >= ntw) break;
    uint8_t* slot = region + (t & 1) * kSlot;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int i = 0; i < WS::kLoads; ++i)
        if (lv[i]) *reinterpret_cast<v4i*>(slot + mt * WS::kTile + 16 * (i * kWave + lane)) = stg[t % kPre][mt][i];
    if (t + kPre < kGMaxTiles) fetch(stg[t % kPre], t + kPre);  // tiles past the run read zeros
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
      const uint8_t* rowp = slot + mt * WS::kTile + m * WS::kRow;
      uint32_t R[kPairs][kDw];
#pragma unroll
      for (int p = 0; p < kPairs; ++p) {
        const uint32_t* rp = reinterpret_cast<const uint32_t*>(rowp + p * 2 * QS::kBlock);
        if constexpr (Q4) {
          R[p][0] = rp[g];
          R[p][1] = rp[g + 1];
          R[p][2] = rp[5 + g];
          R[p][3] = rp[0];
          R[p][4] = rp[4];
        } else {
          R[p][0] = rp[2 * g];
          R[p][1] = rp[2 * g + 1];
          R[p][2] = rp[2 * g + 2];
          R[p][3] = rp[9 + 2 * g];
          R[p][4] = rp[10 + 2 * g];
          R[p][5] = rp[0];
          R[p][6] = rp[8];
        }
      }
      auto operands = [&](int p, h8& be, h8& bo) {
        if constexpr (Q4) {
          be = q4_operand(__builtin_amdgcn_alignbyte(R[p][1], R[p][0], 2));
          bo = q4_operand(R[p][2]);
        } else {
          be = q8_operand(__builtin_amdgcn_alignbyte(R[p][1], R[p][0], 2), __builtin_amdgcn_alignbyte(R[p][2], R[p][1], 2));
          bo = q8_operand(R[p][3], R[p][4]);
        }
      };
      // Pipeline per pair p: the hi products of p, then pair p + 1's operands on the vector ALU,
      // the lo products of p (accumulating onto the hi ones), then the scales of pair p - 1,
      // whose products finished while p's ran.  Scheduling groups keep that order.
      h8 be, bo;
      operands(0, be, bo);
      f4v D0p = Z, D1p = Z;
#pragma unroll
      for (int p = 0; p <= kPairs; ++p) {
        f4v D0 = Z, D1 = Z;
        h8 bn0 = be, bn1 = bo;
        if (p < kPairs) {
          D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ahi[2 * p], be, Z, 0, 0, 0);
          D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ahi[2 * p + 1], bo, Z, 0, 0, 0);
          if (p + 1 < kPairs) operands(p + 1, bn0, bn1);
          D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Alo[2 * p], be, D0, 0, 0, 0);
          D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Alo[2 * p + 1], bo, D1, 0, 0, 0);
        }
        if (p > 0) {
          const int q = p - 1;
          const float de = half_bits_to_float(R[q][Q4 ? 3 : 5] & 0xFFFFu);
          const float dd = half_bits_to_float(R[q][Q4 ? 4 : 6] >> 16);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[t][mt][r] = q == 0 ? de * D0p[r] : fmaf(de, D0p[r], acc[t][mt][r]);
            acc[t][mt][r] = fmaf(dd, D1p[r], acc[t][mt][r]);
          }
        }
        if (p < kPairs) {
          // 2 products, the next operands (18 + alignment), 2 products, this scale step (8)
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          if (p + 1 < kPairs) __builtin_amdgcn_sched_group_barrier(0x002, Q4 ? 19 : 38, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          if (p > 0) __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        D0p = D0;
        D1p = D1;
        be = bn0;
        bo = bn1;
      }
    }
  }

  // ---- 5. combine: each wave's sums times its own power of two, added through LDS in wave order
  //      (a fixed order: the same bits every call, for any batch), then 1 / rms (norm), epilogue
  __syncthreads();  // every wave is done with its region
  f4v* red = reinterpret_cast<f4v*>(lds);
  {
    f4v pw;
#pragma unroll
    for (int r = 0; r < 4; ++r) pw[r] = s_postw[wave * 16 + 4 * g + r];
#pragma unroll
    for (int t = 0; t < kGMaxTiles; ++t) {
      if (t >= ntw) break;
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) red[((wave * kGMaxTiles + t) * NM + mt) * kWave + lane] = acc[t][mt] * pw;
    }
  }
  __syncthreads();
  if (wave >= ntw) return;
  const int t = wave;
  f4v v[NM];
#pragma unroll
  for (int mt = 0; mt < NM; ++mt) {
    v[mt] = red[(t * NM + mt) * kWave + lane];
#pragma unroll
    for (int w = 1; w < kGW; ++w) v[mt] += red[((w * kGMaxTiles + t) * NM + mt) * kWave + lane];
  }
  const int row = row0 + t * 16 + m;
  if (row >= jb.rows) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int sl = 4 * g + r, sq = s_base + sl;
    if (sq >= a.B) break;
    float post = 1.0f;
    if constexpr (NORM) {
      double tot = 0.0;
#pragma unroll
      for (int w = 0; w < kGW; ++w) tot += s_ss[w * 16 + sl];
      post = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(kGK) + static_cast<double>(a.eps)));
    }
    float* y = jb.y + static_cast<size_t>(sq) * jb.ldy + row;
    float out;
    if constexpr (EPI == kEpiResidual) {
      out = *y + v[0][r] * post;
    } else if constexpr (EPI == kEpiSwiglu) {
      out = silu_m(v[0][r] * post) * (v[NM - 1][r] * post);
    } else {
      out = v[0][r] * post;
    }
    *y = out;
  }
}

template <int EPI, bool NORM, int NW>
__global__ __launch_bounds__(Wg<NW>::kT) void gemv_batch_kernel(GArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float s_postw[NW * 16];
  __shared__ double s_ss[NW * 16];
  // workgroup -> (row run, sequence group): the runs' groups on one XCD when the launch allows it
  const int id = blockIdx.x;
  int rg, sg;
  if (a.xcd) {
    const int k = id >> 3;
    rg = (k / a.n_sg) * 8 + (id & 7);
    sg = k % a.n_sg;
  } else {
    rg = id / a.n_sg;
    sg = id % a.n_sg;
  }
  GJob jb = a.job[0];
#pragma unroll
  for (int j = 1; j < kGMaxJobs; ++j)
    if (j < a.n_jobs && rg >= a.job[j].g0) jb = a.job[j];
  const int gi = rg - jb.g0;
  const int t_begin = gi * jb.tiles / jb.groups, ntw = (gi + 1) * jb.tiles / jb.groups - t_begin;
  if (jb.qtype == EF_QTYPE_Q4_0) {
    gemv_body<EPI, NORM, true, NW>(a, jb, t_begin, ntw, sg, lds, s_postw, s_ss);
  } else {
    gemv_body<EPI, NORM, false, NW>(a, jb, t_begin, ntw, sg, lds, s_postw, s_ss);
  }
}

template <int EPI, int NW>
void* batch_kernel(bool norm) {
  return norm ? reinterpret_cast<void*>(&gemv_batch_kernel<EPI, true, NW>)
              : reinterpret_cast<void*>(&gemv_batch_kernel<EPI, false, NW>);
}

template <int NW>
size_t batch_lds(int nm) { return std::max<size_t>(static_cast<size_t>(nm) * Wg<NW>::kRed, Wg<NW>::kLds); }

// Waves per workgroup.  Sixteen waves of 4 K blocks measured slower than eight of 8 on the B = 64
// 5632 x 2048 product (12.4 against 12.0 us): the activations still arrive wave rank by wave rank,
// and a wave's tile loop takes about as long with half the blocks.
constexpr int kNW = 8;

}  // namespace

int launch_gemv_batch(const GemvJob* jobs, int n_jobs, int epi, const float* norm_w, float eps, int batch,
                      size_t ldx, size_t ldy, hipStream_t stream, bool* taken) {
  *taken = false;
  if (batch < 2 || n_jobs < 1 || n_jobs > kGMaxJobs) return EF_HIP_OK;
  const size_t xld = jobs[0].ldx ? jobs[0].ldx : ldx;
  for (int j = 0; j < n_jobs; ++j) {
    const ef_hip_weight_s* W = jobs[j].W;
    if (W->cols != static_cast<size_t>(kGK)) return EF_HIP_OK;
    if (W->qtype != EF_QTYPE_Q4_0 && W->qtype != EF_QTYPE_Q8_0) return EF_HIP_OK;
    if (jobs[j].x != jobs[0].x || (jobs[j].ldx ? jobs[j].ldx : ldx) != xld) return EF_HIP_OK;
  }
  // 16-byte lane pieces of the x rows and the norm weights
  if (reinterpret_cast<uintptr_t>(jobs[0].x) % 16 != 0 || xld % 4 != 0) return EF_HIP_OK;
  if (norm_w != nullptr && reinterpret_cast<uintptr_t>(norm_w) % 16 != 0) return EF_HIP_OK;
  if (static_cast<size_t>(std::min(batch, 16)) * xld * 4 >= (size_t(1) << 31)) return EF_HIP_OK;
  const int nm = epi == kEpiSwiglu ? 2 : 1;
  const size_t lds = batch_lds<kNW>(nm);
  const size_t lim = ctx().lds_per_block > 0 ? ctx().lds_per_block : 65536;
  if (lds > lim) return EF_HIP_OK;
  // Row runs: as many as give every CU one workgroup (CUs / sequence groups), at most 6 tiles
  // each, split over the jobs in proportion to their tiles; a multiple of 8 places each run's
  // sequence groups on one XCD.
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  const int n_sg = (batch + 15) / 16;
  int tiles[kGMaxJobs], groups[kGMaxJobs], nt = 0, need = 0;
  for (int j = 0; j < n_jobs; ++j) {
    tiles[j] = static_cast<int>((jobs[j].W->rows + 15) / 16);
    nt += tiles[j];
    groups[j] = (tiles[j] + kGMaxTiles - 1) / kGMaxTiles;
    need += groups[j];
  }
  // Every workgroup streams its 16 sequences' activations once; launches of more workgroups than
  // about one round over the CUs (large batches: prefill) re-stream them per row run and are left
  // to the split-K kernel, which shares each activation fragment over more rows.
  if (static_cast<long>(need) * n_sg > cus + cus / 4) return EF_HIP_OK;
  int target = std::max(need, std::min(nt, std::max(1, cus / n_sg)));
  if (target % 8 != 0 && (target / 8 + 1) * 8 <= nt) target = (target / 8 + 1) * 8;
  int have = need;
  for (int j = 0; j < n_jobs; ++j) {
    const int want = static_cast<int>(static_cast<long>(target) * tiles[j] / nt);
    const int add = std::max(0, std::min(want, tiles[j]) - groups[j]);
    groups[j] += add;
    have += add;
  }
  while (have < target) {  // the job with the most tiles per run gets one more run
    int best = -1;
    for (int j = 0; j < n_jobs; ++j)
      if (groups[j] < tiles[j] &&
          (best < 0 || static_cast<long>(tiles[j]) * groups[best] > static_cast<long>(tiles[best]) * groups[j]))
        best = j;
    if (best < 0) break;
    ++groups[best];
    ++have;
  }
  GArgs a{};
  a.n_jobs = n_jobs;
  a.n_sg = n_sg;
  a.B = batch;
  a.x = jobs[0].x;
  a.ldx = static_cast<long>(xld);
  a.norm_w = norm_w;
  a.eps = eps;
  int g0 = 0;
  for (int j = 0; j < n_jobs; ++j) {
    GJob& d = a.job[j];
    d.W = jobs[j].W->dev;
    d.W2 = jobs[j].W2 ? jobs[j].W2->dev : nullptr;
    d.y = jobs[j].y;
    d.ldy = static_cast<long>(jobs[j].ldy ? jobs[j].ldy : ldy);
    d.rows = static_cast<int>(jobs[j].W->rows);
    d.qtype = jobs[j].W->qtype;
    d.g0 = g0;
    d.groups = groups[j];
    d.tiles = tiles[j];
    g0 += groups[j];
  }
  a.xcd = g0 % 8 == 0 ? 1 : 0;
  const long wgs = static_cast<long>(g0) * n_sg;
  if (wgs > 0x7FFFFFFFL) return EF_HIP_OK;
  const bool nrm = norm_w != nullptr;
  void* fn = epi == kEpiSwiglu ? batch_kernel<kEpiSwiglu, kNW>(nrm)
                                : (epi == kEpiStore ? batch_kernel<kEpiStore, kNW>(nrm) : batch_kernel<kEpiResidual, kNW>(nrm));
  void* params[] = {&a};
  EFH_HIP(hipLaunchKernel(fn, dim3(static_cast<unsigned>(wgs)), dim3(kNW * kWave), params, lds, stream));
  *taken = true;
  return EF_HIP_OK;
}

}  // namespace efh
