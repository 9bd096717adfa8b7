// Packed Q4_0 / Q8_0 GEMV on the matrix cores for batches of sequences (2..64 per launch).
//
// Two kernels per launch (three with a K split):
//  1. xfrag_kernel turns the activations [B][K] (optionally RMS-normalised, kern::rmsnorm order)
//     into the A operands of v_mfma_f32_16x16x32_f16, in global memory, laid out exactly as a wave
//     loads them: for each tile of 16 sequences, each 32-weight block and each part (hi, lo),
//     64 lanes x 16 bytes (one coalesced 1 KB load).  Row i of a tile is sequence i: x' = x * 2^-e_s
//     (a per-sequence power of two keeping |x'| < 2^15) split exactly into fp16 hi + lo
//     (x' - hi - lo is below 2^-22 |x'|).  Columns follow the codes' k order below.
//  2. gemv_mfma_kernel: a workgroup (8 waves) owns RT tiles of 16 rows (x2 matrices for SwiGLU),
//     NS sequence tiles and a range of block pairs; its rows' packed blocks are fetched with
//     coalesced 1 KB LDS-DMA loads into LDS rows an odd number of 16-byte units apart (the 16 rows
//     one B fragment reads fall in distinct banks).  The waves split the block pairs (pair m to wave
//     m % 8).  Per pair, each row tile's codes are converted once into B operands and reused for
//     every sequence tile:
//       B = the row's codes minus their bias as exact fp16, straight out of the packed bytes: one
//           AND-OR of a Q4_0 dword with the fp16 pattern of 1024 yields two codes as 1024 + c
//           ((q & 0x000F000F) | 0x64006400: codes 0 and 2 of the dword's low nibbles; the high
//           nibbles through 0x00F000F0 come out as 1024 + 16 c), and one packed fp16 add removes
//           1024 + 8 (resp. 1024 + 128) exactly.  Q8_0 codes are offset to unsigned (q ^ 0x80) and
//           taken two per AND-OR the same way, minus 1024 + 128.  The A columns are permuted to
//           match, and divided by 16 where the code is a scaled high nibble;
//       D = A_hi x B, then D += A_lo x B on the matrix core (the accumulator input), so D holds
//           sum_k (c_k - bias) x'_k of the block for 16 sequences x 16 rows, and the block adds
//           d * D to an FP32 accumulator: one FMA per output and block, the only per-block VALU
//           work besides the B conversion.
//     The waves' partial sums are combined in LDS in a fixed order, one row tile at a time (the
//     operand LDS is reused); the scale 2^e_s is undone and the epilogue (store / residual /
//     SwiGLU) applied, or, with K split over workgroups, the split's sums go to a workspace.
//  3. finalize_kernel (K split only) adds the splits in index order and applies the epilogue.
// The planner sizes RT (rows per workgroup: every workgroup streams its sequences' A operands
// through its CU, so more rows per workgroup mean fewer re-reads), NS and the K split to fill the
// 256 CUs; measured aggregate L2 read bandwidth when every workgroup streams one shared table is
// ~20-30 TB/s on MI355X.
// (Codes as fp16 subnormals would save the add, but the matrix core does not sum products of
// subnormal operands exactly: measured errors of thousands of ulps, biased; normal operands give
// a few ulps, unbiased.)  Products are exact (fp16 x fp16 in FP32), so results match an FP32 dot
// product to rounding; the order differs from the reference CPU kernels (src/qkernels.cpp:39-65,
// 131-180) and is fixed for a given shape.  Single sequences use the vector-ALU kernels (gemv.hip),
// which are faster when nothing amortises the activation preparation.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "afrag.h"
#include "gemv.h"
#include "qfrag.h"

namespace efh {
namespace {

constexpr int kT = 512;                         // GEMV workgroup: 8 waves split the block pairs
constexpr int kWavesM = kT / kWave;
constexpr int kTP = 1024;                       // prep workgroup
constexpr int kWavesP = kTP / kWave;
constexpr int kTileRows = 16;
constexpr int kSeqTile = 16;                    // sequences per A operand (one per row)
constexpr int kMaxTiles = 64;                   // sequence tiles per launch: 1024 sequences (rows)
constexpr int kMaxJobsM = 4;
constexpr int kPrepBlocks = kTP / kWave;        // blocks per xfrag workgroup: one per wave
// K blocks per wave of one batched GEMV workgroup: 24 for the smallest shapes (two accumulator
// tiles: a whole K of up to 6144 without a split), 8 otherwise (more unrolled blocks would spill)
__host__ __device__ constexpr int max_blocks_per_wave(int rt, int nm, int ns) { return rt * nm * ns <= 2 ? 24 : 8; }

typedef __attribute__((address_space(3))) void lds_void;

struct MJob {
  const uint8_t* W;     // tile-order copies (tile_layout_kernel)
  const uint8_t* W2;
  float* y;
  int rows, qtype, tile_begin;
  uint32_t bytes;       // of each tile-order matrix
  long ldy;
};

struct MArgs {
  MJob job[kMaxJobsM];
  int n_jobs, K, B, n_tiles;
  const uint8_t* t4;    // A tables (Q4_0 and Q8_0 column orders), [tile][block][hi, lo][64 lanes][16 bytes]
  const uint8_t* t8;
  uint32_t tab_bytes;   // bytes of each table
  const float* post;    // [B] 2^e_s
  int ksplit, blocks_per_split;   // split-K: workgroups per row group and blocks each
  float* part;          // [group][split][B][rows of the group][matrices] partial sums (ksplit > 1)
  // Block-scaled tables (staged by the producing kernel): every (sequence, block) has its own power
  // of two, bscale[block * bpad + sequence], by which the block's products are multiplied; the
  // epilogue factor is 1 / rms from ssp[p * bpad + sequence] (n_ssp partial sums of squares of the
  // un-normed input, eps) or 1 without ssp.  post_out gets those factors for finalize_kernel.
  const float* bscale;
  int bpad;
  const double* ssp;
  int n_ssp;
  float eps;
  float* post_out;
  AEmit em;  // the outputs also staged as the next product's tables (store / residual / SwiGLU)
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


// grid (ceil(nb / 16), tiles): workgroup (x, t) prepares sequences 16 t .. 16 t + 15 for blocks
// 16 x .. 16 x + 15.  Every workgroup of a tile recomputes the tile's per-sequence factors (a read of
// 16 x K floats, one wave per sequence), then each wave writes one block's fragments.
__global__ __launch_bounds__(kTP) void xfrag_kernel(PrepArgs a) {
  __shared__ double s_ss[kWavesP];
  __shared__ float s_ax[kWavesP];
  __shared__ float s_aw[kWavesP];
  __shared__ float s_mul[kSeqTile], s_pre[kSeqTile];
  static_assert(kWavesP == kSeqTile, "one wave per sequence of the tile");
  const int K = a.K, tile = blockIdx.y, nb = K >> 5;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const bool has_norm = a.norm_w != nullptr;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 4u;
  // Every load below goes through a buffer resource (zeros past its end: sequences past the batch,
  // a missing norm, blocks past K) and is issued before any of them is used, so the kernel waits on
  // memory about once instead of once per load.
  // 2a. this wave's fragment inputs: block kb, lane l = sequence l % 16 and k group l / 16; both
  //     column orders (Q4_0: weights 4g..4g+3 and 4g+16..4g+19 of the block, Q8_0: 8g..8g+7)
  const int kb = blockIdx.x * kPrepBlocks + wave;
  const int i = lane & 15, g = lane >> 4, sq_f = tile * kSeqTile + i;
  // one resource over the chunk's rows (B * ldx floats, < 16 MiB); a lane of a sequence past the
  // batch, or of a block past K, addresses the resource's end and reads zeros
  const uint32_t x_bytes = static_cast<uint32_t>(a.B) * static_cast<uint32_t>(a.ldx) * 4u;
  const __amdgpu_buffer_rsrc_t rx_all = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.norm_w, has_norm ? row_bytes : 0u);
  const bool frag_live = sq_f < a.B && kb < nb;
  const uint32_t kf = static_cast<uint32_t>(kb) * 128u;  // byte offset of the block in a row
  const uint32_t row0 = static_cast<uint32_t>(sq_f) * static_cast<uint32_t>(a.ldx) * 4u;
  const uint32_t o4[2] = {kf + 16u * g, kf + 64u + 16u * g}, o8[2] = {kf + 32u * g, kf + 32u * g + 16u};
  // the first table's inputs now (Q4_0's when present); a launch with both tables loads the Q8_0
  // order's after the statistics
  const bool q4_first = a.t4 != nullptr;
  float4 fx[2], fw[2];
  auto load_frag = [&](const uint32_t (&o)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      fx[h] = buf_f4(rx_all, frag_live ? row0 + o[h] : x_bytes);
      fw[h] = buf_f4(rw, kb < nb ? o[h] : row_bytes);
    }
  };
  load_frag(q4_first ? o4 : o8);
  // 1. per-sequence sum of squares (double, kern::rmsnorm) and max |x| (wave s reduces sequence
  //    s), and max |norm weight| (every thread), 8 loads in flight per lane
  {
    const int sq = tile * kSeqTile + __builtin_amdgcn_readfirstlane(wave);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (sq < a.B ? sq : 0) * a.ldx, sq < a.B ? row_bytes : 0u);
    double ss = 0.0;
    float ax = 0.0f, aw = 0.0f;
    // the norm weights' first 8192 values are requested with the rows (zeros without a norm)
    const float4 wn0 = buf_f4(rw, threadIdx.x * 16u), wn1 = buf_f4(rw, (kTP + threadIdx.x) * 16u);
    constexpr int kU = 8;
    for (uint32_t base = 0; base < row_bytes; base += kU * kWave * 16u) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = buf_f4(rx, base + (u * kWave + lane) * 16u);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        ss += static_cast<double>(v[u].x) * static_cast<double>(v[u].x);
        ss += static_cast<double>(v[u].y) * static_cast<double>(v[u].y);
        ss += static_cast<double>(v[u].z) * static_cast<double>(v[u].z);
        ss += static_cast<double>(v[u].w) * static_cast<double>(v[u].w);
        ax = fmaxf(ax, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
      }
    }
    aw = fmaxf(fmaxf(fmaxf(fabsf(wn0.x), fabsf(wn0.y)), fmaxf(fabsf(wn0.z), fabsf(wn0.w))),
               fmaxf(fmaxf(fabsf(wn1.x), fabsf(wn1.y)), fmaxf(fabsf(wn1.z), fabsf(wn1.w))));
    if (has_norm) {
      for (uint32_t base = 2 * kTP * 16u; base < row_bytes; base += 2 * kTP * 16u) {
        const float4 w0 = buf_f4(rw, base + threadIdx.x * 16u);
        const float4 w1 = buf_f4(rw, base + (kTP + threadIdx.x) * 16u);
        aw = fmaxf(aw, fmaxf(fmaxf(fabsf(w0.x), fabsf(w0.y)), fmaxf(fabsf(w0.z), fabsf(w0.w))));
        aw = fmaxf(aw, fmaxf(fmaxf(fabsf(w1.x), fabsf(w1.y)), fmaxf(fabsf(w1.z), fabsf(w1.w))));
      }
    }
    ss = wave_sum_d_dpp(ss);
    ax = wave_max_dpp(ax);
    aw = wave_max_dpp(aw);
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
    const double tot = s_ss[s];
    const float ax = s_ax[s];
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
  // 2b. fragments: wave w writes block 16 x + w, lane l the 8 values of sequence l % 16 and k group
  //     l / 16, hi and lo
  if (kb >= nb) return;
  const float inv = s_mul[i], pre = s_pre[i];
  auto frag = [&](float (&out)[8]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float4 v = fx[h];
      if (has_norm) {  // HF order: w * (x * inv)
        const float4 w = fw[h];
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
  // hi and lo parts of the 8 values in slot order `ord`, slots with q16 set divided by 16
  auto store = [&](uint8_t* table, const float (&xv)[8], const int (&ord)[8], const bool (&q16)[8]) {
    h8 hi, lo;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float xp = xv[ord[u]];
      const _Float16 h = static_cast<_Float16>(xp);
      const _Float16 l = static_cast<_Float16>(xp - static_cast<float>(h));
      const _Float16 q = static_cast<_Float16>(q16[u] ? 0.0625f : 1.0f);  // exact powers of two
      hi[u] = h * q;
      lo[u] = l * q;
    }
    uint8_t* f = table + ((static_cast<size_t>(tile) * nb + kb) * 2 * kWave + lane) * 16;
    *reinterpret_cast<h8*>(f) = hi;
    *reinterpret_cast<h8*>(f + kWave * 16) = lo;
  };
  if (a.t4 != nullptr) {  // slots 0..7 = weights 4g + {0, 2, 16, 18, 1, 3, 17, 19}
    float xv[8];
    frag(xv);
    constexpr int ord[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    constexpr bool q16[8] = {false, false, true, true, false, false, true, true};
    store(a.t4, xv, ord, q16);
  }
  if (a.t8 != nullptr) {  // slots 0..7 = weights 8g + {0, 2, 1, 3, 4, 6, 5, 7}
    if (q4_first) load_frag(o8);
    float xv[8];
    frag(xv);
    constexpr int ord[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    constexpr bool q16[8] = {false, false, false, false, false, false, false, false};
    store(a.t8, xv, ord, q16);
  }
}

// One workgroup per sequence (K <= kSeqPrepMaxK): thread t owns fragment pairs p = t + 256 j
// (block p / 4, k group p % 4) of sequence blockIdx.x, so the values it converts are also its share
// of the per-sequence statistics and the row is read once, every load issued before the first
// wait.  Sequences past the batch (up to the last table tile) get zero fragments.
constexpr int kSeqPrepThreads = 256, kSeqPrepPairs = 4;
constexpr int kSeqPrepMaxK = 32 * kSeqPrepThreads * kSeqPrepPairs / 4;  // 8192

__global__ __launch_bounds__(kSeqPrepThreads) void xfrag_seq_kernel(PrepArgs a) {
  __shared__ double s_ss[kSeqPrepThreads / kWave];
  __shared__ float s_ax[kSeqPrepThreads / kWave], s_aw[kSeqPrepThreads / kWave];
  const int sq = blockIdx.x, tile = sq / kSeqTile, i = sq % kSeqTile;
  const int K = a.K, nb = K >> 5, npairs = nb * 4;
  const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
  const bool has_norm = a.norm_w != nullptr, live = sq < a.B;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 4u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (live ? sq : 0) * a.ldx, live ? row_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.norm_w, has_norm ? row_bytes : 0u);
  // byte offsets of a pair's two float4 in the Q4_0 order (weights 4g.. and 16 + 4g.. of the block)
  // or the Q8_0 order (8g .. 8g + 7); pairs past the row read zeros
  auto offs = [&](int pr, bool q4, uint32_t (&o)[2]) {
    const uint32_t kb = static_cast<uint32_t>(pr >> 2), g = static_cast<uint32_t>(pr & 3);
    const uint32_t base = pr < npairs ? kb * 128u : row_bytes;
    o[0] = base + (q4 ? 16u * g : 32u * g);
    o[1] = base + (q4 ? 64u + 16u * g : 32u * g + 16u);
  };
  const bool q4_first = a.t4 != nullptr;
  f4v xv[kSeqPrepPairs][2], wv[kSeqPrepPairs][2];
#pragma unroll
  for (int j = 0; j < kSeqPrepPairs; ++j) {
    uint32_t o[2];
    offs(t + kSeqPrepThreads * j, q4_first, o);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rx, o[h], 0, 0));
      wv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rw, o[h], 0, 0));
    }
  }
  // statistics: every value of the row (and of the norm weights) is in exactly one thread's pairs
  double ss = 0.0;
  float ax = 0.0f, aw = 0.0f;
#pragma unroll
  for (int j = 0; j < kSeqPrepPairs; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = xv[j][h][e];
        ss += static_cast<double>(v) * static_cast<double>(v);
        ax = fmaxf(ax, fabsf(v));
        aw = fmaxf(aw, fabsf(wv[j][h][e]));
      }
  ss = wave_sum_d_dpp(ss);
  ax = wave_max_dpp(ax);
  aw = wave_max_dpp(aw);
  if (lane == 0) {
    s_ss[wave] = ss;
    s_ax[wave] = ax;
    s_aw[wave] = aw;
  }
  __syncthreads();
  double tot = 0.0;
  ax = 0.0f;
  aw = 0.0f;
  for (int w = 0; w < kSeqPrepThreads / kWave; ++w) {
    tot += s_ss[w];
    ax = fmaxf(ax, s_ax[w]);
    aw = fmaxf(aw, s_aw[w]);
  }
  if (!has_norm) aw = 1.0f;
  const float inv = has_norm ? static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(a.eps)))
                             : 1.0f;
  const float bound = ax * inv * aw * 1.0001f;  // >= max |w * (x * inv)|
  int ex = 0;
  if (bound > 0.0f && bound <= 3.0e38f) ex = ilogbf(bound) - 14;  // bound * 2^-ex < 2^15
  const float pre = ldexpf(1.0f, -ex);
  if (t == 0 && live) a.post[sq] = ldexpf(1.0f, ex);
  // fragments: hi and lo of the 8 values in slot order, slots with q16 set divided by 16
  auto emit = [&](uint8_t* table, int pr, const f4v (&x2)[2], const f4v (&w2)[2], bool q4) {
    if (pr >= npairs) return;
    float v[8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y = x2[h][e];
        if (has_norm) y = w2[h][e] * (y * inv);  // HF order: w * (x * inv)
        v[4 * h + e] = y * pre;
      }
    // Q4_0 slots 0..7 = weights 4g + {0, 2, 16, 18, 1, 3, 17, 19}; Q8_0 = 8g + {0, 2, 1, 3, 4, 6, 5, 7}
    constexpr int ord4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    constexpr int ord8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    h8 hi, lo;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float xp = v[q4 ? ord4[u] : ord8[u]];
      const _Float16 hh = static_cast<_Float16>(xp);
      const _Float16 ll = static_cast<_Float16>(xp - static_cast<float>(hh));
      const _Float16 qs = static_cast<_Float16>(q4 && (u & 2) ? 0.0625f : 1.0f);  // exact powers of two
      hi[u] = hh * qs;
      lo[u] = ll * qs;
    }
    const int kb = pr >> 2, g = pr & 3;
    uint8_t* f = table + ((static_cast<size_t>(tile) * nb + kb) * 2 * kWave + (16 * g + i)) * 16;
    *reinterpret_cast<h8*>(f) = hi;
    *reinterpret_cast<h8*>(f + kWave * 16) = lo;
  };
#pragma unroll
  for (int j = 0; j < kSeqPrepPairs; ++j) emit(q4_first ? a.t4 : a.t8, t + kSeqPrepThreads * j, xv[j], wv[j], q4_first);
  if (q4_first && a.t8 != nullptr) {  // both tables: the Q8_0 order's values, read again
#pragma unroll
    for (int j = 0; j < kSeqPrepPairs; ++j) {
      uint32_t o[2];
      offs(t + kSeqPrepThreads * j, false, o);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        xv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rx, o[h], 0, 0));
        wv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rw, o[h], 0, 0));
      }
    }
#pragma unroll
    for (int j = 0; j < kSeqPrepPairs; ++j) emit(a.t8, t + kSeqPrepThreads * j, xv[j], wv[j], false);
  }
}

// Block-scaled tables from activations in memory (no kernel staged them): one workgroup per
// sequence, thread t owns pairs t + 256 j (pair = block kb, k group g), so the four threads of a
// block hold its 32 values.  Each (sequence, block) gets its own power of two 2^e (|v| 2^-e < 2^15
// for v = norm_w * x, or x), written to bscale[kb * bpad + seq]; the fragments hold v 2^-e split
// into fp16 hi + lo in the tables' slot orders; ssp[seq] (one partial per sequence) is the double
// sum of x^2, kern::rmsnorm's statistic, applied by the GEMV's epilogue as 1 / rms.
__global__ __launch_bounds__(kSeqPrepThreads) void xfrag_block_kernel(PrepArgs a, float* bscale, int bpad,
                                                                       double* ssp) {
  __shared__ double s_ss[kSeqPrepThreads / kWave];
  const int sq = blockIdx.x, tile = sq / kSeqTile, i = sq % kSeqTile;
  const int K = a.K, nb = K >> 5, npairs = nb * 4;
  const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
  const bool has_norm = a.norm_w != nullptr, live = sq < a.B;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 4u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (live ? sq : 0) * a.ldx, live ? row_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.norm_w, has_norm ? row_bytes : 0u);
  auto offs = [&](int pr, bool q4, uint32_t (&o)[2]) {
    const uint32_t kb = static_cast<uint32_t>(pr >> 2), g = static_cast<uint32_t>(pr & 3);
    const uint32_t base = pr < npairs ? kb * 128u : row_bytes;
    o[0] = base + (q4 ? 16u * g : 32u * g);
    o[1] = base + (q4 ? 64u + 16u * g : 32u * g + 16u);
  };
  f4v xv[kSeqPrepPairs][2], wv[kSeqPrepPairs][2];
#pragma unroll
  for (int j = 0; j < kSeqPrepPairs; ++j) {
    uint32_t o[2];
    offs(t + kSeqPrepThreads * j, true, o);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rx, o[h], 0, 0));
      wv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rw, o[h], 0, 0));
    }
  }
  double ss = 0.0;
  float pre[kSeqPrepPairs];
#pragma unroll
  for (int j = 0; j < kSeqPrepPairs; ++j) {
    float m = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = xv[j][h][e];
        ss += static_cast<double>(x) * static_cast<double>(x);
        m = fmaxf(m, fabsf(has_norm ? wv[j][h][e] * x : x));
      }
    // the block's four threads (pairs 4 kb .. 4 kb + 3 are threads of one quad)
    m = fmaxf(m, dpp_self_f<0xB1>(m));
    m = fmaxf(m, dpp_self_f<0x4E>(m));
    const float bound = m * 1.0001f;
    int ex = 0;
    if (bound > 0.0f && bound <= 3.0e38f) ex = ilogbf(bound) - 14;  // bound * 2^-ex < 2^15
    pre[j] = ldexpf(1.0f, -ex);
    const int pr = t + kSeqPrepThreads * j;
    if ((pr & 3) == 0 && pr < npairs && live) bscale[static_cast<size_t>(pr >> 2) * bpad + sq] = ldexpf(1.0f, ex);
  }
  ss = wave_sum_d_dpp(ss);
  if (lane == 0) s_ss[wave] = ss;
  __syncthreads();
  if (t == 0 && live) {
    double tot = 0.0;
    for (int w = 0; w < kSeqPrepThreads / kWave; ++w) tot += s_ss[w];
    ssp[sq] = tot;
  }
  auto emit = [&](uint8_t* table, int pr, const f4v (&x2)[2], const f4v (&w2)[2], float pscale, bool q4) {
    if (pr >= npairs) return;
    float v[8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * h + e] = (has_norm ? w2[h][e] * x2[h][e] : x2[h][e]) * pscale;
    constexpr int ord4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    constexpr int ord8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    h8 hi, lo;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float xp = v[q4 ? ord4[u] : ord8[u]];
      const _Float16 hh = static_cast<_Float16>(xp);
      const _Float16 ll = static_cast<_Float16>(xp - static_cast<float>(hh));
      const _Float16 qs = static_cast<_Float16>(q4 && (u & 2) ? 0.0625f : 1.0f);
      hi[u] = hh * qs;
      lo[u] = ll * qs;
    }
    const int kb = pr >> 2, g = pr & 3;
    uint8_t* f = table + ((static_cast<size_t>(tile) * nb + kb) * 2 * kWave + (16 * g + i)) * 16;
    *reinterpret_cast<h8*>(f) = hi;
    *reinterpret_cast<h8*>(f + kWave * 16) = lo;
  };
  if (a.t4 != nullptr) {
#pragma unroll
    for (int j = 0; j < kSeqPrepPairs; ++j) emit(a.t4, t + kSeqPrepThreads * j, xv[j], wv[j], pre[j], true);
  }
  if (a.t8 != nullptr) {  // the Q8_0 order's values
#pragma unroll
    for (int j = 0; j < kSeqPrepPairs; ++j) {
      uint32_t o[2];
      offs(t + kSeqPrepThreads * j, false, o);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        xv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rx, o[h], 0, 0));
        wv[j][h] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rw, o[h], 0, 0));
      }
    }
#pragma unroll
    for (int j = 0; j < kSeqPrepPairs; ++j) emit(a.t8, t + kSeqPrepThreads * j, xv[j], wv[j], pre[j], false);
  }
}

// Weights in tile order: for every 16-row tile T and block b, the 16 rows' codes in the order the
// B fragment's lanes use them (lane l = 16 g + j: row j's code bytes 4g .. 4g + 3 of a Q4_0 block,
// 8g .. 8g + 7 of a Q8_0 block), then the 16 rows' fp16 scales: 288 (Q4_0) or 544 (Q8_0) bytes at
// (T * nb + b) * bytes.  A wave reads one tile-block with one coalesced load per lane.
constexpr uint32_t kTileBlockQ4 = 288, kTileBlockQ8 = 544;

__global__ __launch_bounds__(256) void tile_layout_kernel(const uint8_t* __restrict__ W, int rows, int nb,
                                                          int row_bytes, int q4, uint8_t* __restrict__ out) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;  // (tile, block, lane)
  const int tiles = (rows + kTileRows - 1) / kTileRows;
  const int lane = static_cast<int>(idx % kWave);
  const long tb = idx / kWave;
  const int blk = static_cast<int>(tb % nb), T = static_cast<int>(tb / nb);
  if (T >= tiles) return;
  const int j = lane & 15, g = lane >> 4, row = T * kTileRows + j;
  const uint32_t bb = q4 ? kTileBlockQ4 : kTileBlockQ8;
  uint8_t* o = out + static_cast<size_t>(T * nb + blk) * bb;
  const uint8_t* src = W + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(blk) * (q4 ? 18 : 34);
  const bool live = row < rows;  // rows past the matrix: zero codes and scales
  const int nc = q4 ? 4 : 8;
  for (int c = 0; c < nc; ++c) o[lane * nc + c] = live ? src[2 + nc * g + c] : 0;
  if (g == 0) {  // the scale after the 64 lanes' codes
    uint8_t* sc = o + kWave * nc + 2 * j;
    sc[0] = live ? src[0] : 0;
    sc[1] = live ? src[1] : 0;
  }
}

// B operand and scale of one 16-row tile-block.
template <bool Q4>
struct WRegs {
  uint32_t c0, c1;  // this lane's code bytes (c1 unused for Q4_0)
  uint32_t sc;      // the lane's row scale, fp16 bits in the low half
};

template <bool Q4>
__device__ __forceinline__ WRegs<Q4> load_w(__amdgpu_buffer_rsrc_t r, uint32_t voff_c, uint32_t voff_s,
                                            uint32_t so) {
  WRegs<Q4> w;
  if constexpr (Q4) {
    w.c0 = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, voff_c, so, 0));
    w.c1 = 0;
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff_c, so, 0);
    w.c0 = static_cast<uint32_t>(v[0]);
    w.c1 = static_cast<uint32_t>(v[1]);
  }
  w.sc = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, voff_s, so, 0));
  return w;
}

// Products of one block for every row tile and matrix: D = A_hi B, D += A_lo B on the matrix core,
// acc += d D.  Software-pipelined over the (row tile, matrix) units: while unit u's products run on
// the matrix core, the vector ALU converts unit u + 1's codes and applies unit u - 1's scales, so
// neither pipe waits on the other (each stage is kept together by a scheduling barrier, and inside
// it products and vector instructions alternate).
template <int RT, int NM, int NS, bool Q4, bool BS = false>
__device__ __forceinline__ void block_products(const WRegs<Q4> (&W)[RT][NM], const h8 (&Ax)[NS][2],
                                               f4v (&acc)[RT][NM][NS], const f4v (&Sc)[NS]) {
  constexpr int U = RT * NM;
  const f4v Z = {0.0f, 0.0f, 0.0f, 0.0f};
  auto operand = [&](int u) -> h8 {
    const WRegs<Q4>& w = W[u / NM][u % NM];
    return Q4 ? q4_operand(w.c0) : q8_operand(w.c0, w.c1);
  };
  auto scale = [&](int u) -> float { return f16lo(W[u / NM][u % NM].sc); };
  h8 b = operand(0);
  f4v Dp[NS];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    f4v D[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) D[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ax[t][0], b, Z, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NS; ++t) D[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ax[t][1], b, D[t], 0, 0, 0);
    if (u > 0) {
      const float d = scale(u - 1);
      const int rt = (u - 1) / NM, mt = (u - 1) % NM;
#pragma unroll
      for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[rt][mt][t][r] = fmaf(BS ? d * Sc[t][r] : d, Dp[t][r], acc[rt][mt][t][r]);
    }
    if (u + 1 < U) b = operand(u + 1);
#pragma unroll
    for (int t = 0; t < NS; ++t) Dp[t] = D[t];
    constexpr int kValuPer = (12 + 4 * NS + 2 * NS - 1) / (2 * NS);
#pragma unroll
    for (int i = 0; i < 2 * NS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // one product
      __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);  // vector ALU work
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  {
    const float d = scale(U - 1);
    const int rt = (U - 1) / NM, mt = (U - 1) % NM;
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[rt][mt][t][r] = fmaf(BS ? d * Sc[t][r] : d, Dp[t][r], acc[rt][mt][t][r]);
  }
}

// The wave's blocks b = kb0 + wave + 8 i < kb1: the weights two blocks ahead and the A fragments
// one block ahead are loaded while the current block's products run.  Prefetches past the row
// read its last block instead, so they need no bounds test.
template <int RT, int NM, int NS, bool Q4, bool BS = false>
__device__ __forceinline__ void k_loop(const MJob& jb, int tile_row0, int nb, int kb0, int kb1, int wave, int lane,
                                       __amdgpu_buffer_rsrc_t tab, uint32_t tile0, uint32_t tstride,
                                       f4v (&acc)[RT][NM][NS], __amdgpu_buffer_rsrc_t bsr, uint32_t bpad,
                                       uint32_t seq0) {
  const uint32_t bb = Q4 ? kTileBlockQ4 : kTileBlockQ8;
  const int last_tile = static_cast<int>(jb.bytes / (static_cast<uint32_t>(nb) * bb)) - 1;
  const __amdgpu_buffer_rsrc_t r1 = make_rsrc(jb.W, jb.bytes);
  const __amdgpu_buffer_rsrc_t r2 = make_rsrc(NM == 2 ? jb.W2 : jb.W, jb.bytes);
  const uint32_t voff_c = static_cast<uint32_t>(lane) * (Q4 ? 4 : 8);
  const uint32_t voff_s = (Q4 ? 256u : 512u) + 2u * static_cast<uint32_t>(lane & 15);
  const uint32_t voff_a = static_cast<uint32_t>(lane) * 16;
  // prefetches past the row read its last block and row tiles past the matrix its last tile (never
  // used): every load stays inside its buffer
  auto load_wb = [&](WRegs<Q4> (&dst)[RT][NM], int kb) {
    kb = min(kb, nb - 1);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int tr = min(tile_row0 + rt, last_tile);
      const uint32_t so = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tr * nb + kb) * bb);
      dst[rt][0] = load_w<Q4>(r1, voff_c, voff_s, so);
      if (NM == 2) dst[rt][NM - 1] = load_w<Q4>(r2, voff_c, voff_s, so);
    }
  };
  auto load_a = [&](h8 (&dst)[NS][2], int kb) {
    kb = min(kb, nb - 1);
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t so =
            __builtin_amdgcn_readfirstlane(tile0 + t * tstride + static_cast<uint32_t>(kb * 2 + h) * kWave * 16);
        dst[t][h] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(tab, voff_a, so, 0));
      }
  };
  // Fully unrolled over at most MB blocks.  Every prefetch is issued
  // unconditionally (a block past this workgroup's range is read and never used), so every path
  // has the same loads in flight and the wait before each block's products covers only that
  // block's loads.
  // block scales of the lane's four sequences (4 (l / 16) .. + 3 of each tile) with the A fragments
  auto load_s = [&](f4v (&dst)[NS], int kb) {
    if constexpr (BS) {
      kb = min(kb, nb - 1);
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        const uint32_t off = (static_cast<uint32_t>(kb) * bpad + seq0 + t * kSeqTile + 4u * (lane >> 4)) * 4u;
        dst[t] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(bsr, off, 0, 0));
      }
    }
  };
  constexpr int MB = max_blocks_per_wave(RT, NM, NS);
  WRegs<Q4> W[MB][RT][NM];
  h8 A[2][NS][2];
  f4v Sc[2][NS];
  // Loads are issued in the order their blocks need them and kept there by scheduling barriers:
  // loads complete in order, so a block's wait then never covers a later block's prefetch.
  const int kb = kb0 + wave;
  load_wb(W[0], kb);
  load_a(A[0], kb);
  load_s(Sc[0], kb);
  __builtin_amdgcn_sched_barrier(0);
  load_wb(W[1], kb + kWavesM);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int b = kb + i * kWavesM;
    if (b >= kb1) break;
    if (i + 1 < MB) {
      load_a(A[(i + 1) & 1], b + kWavesM);
      load_s(Sc[(i + 1) & 1], b + kWavesM);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < MB) load_wb(W[i + 2], b + 2 * kWavesM);
    __builtin_amdgcn_sched_barrier(0);
    block_products<RT, NM, NS, Q4, BS>(W[i], A[i & 1], acc, Sc[i & 1]);
  }
}

// Phase 3: the eight waves' partial sums reduced through LDS and scattered: every wave writes its
// D fragments, then wave w adds fragments f = w, w + 8, ... of all eight waves (in wave order, a
// fixed order) and finishes them from registers: the scale undone and the epilogue (one K split)
// or the split's sums to the workspace for finalize_kernel.  acc[rt][mt][t] is fragment
// f = rt * NS + t of matrix mt: lane l holds rows 4 (l / 16) .. + 3 (sequences) of column l % 16.
template <int EPI, int RT, int NS>
__device__ __forceinline__ void combine_and_store(const MArgs& a, const MJob& jb, uint8_t* lb,
                                                  const f4v (&acc)[RT][EPI == kEpiSwiglu ? 2 : 1][NS], int wave,
                                                  int lane, int row0, int grp, int ks, int s0, const float* post_p,
                                                  int post_base) {
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int ROWS = RT * kTileRows;
  constexpr int F = RT * NS;                       // fragments per matrix
  constexpr int wstep = F * NM * kWave * 4;         // floats per wave
  f4v* red = reinterpret_cast<f4v*>(lb);          // [wave][f][mt][lane]
  __syncthreads();  // the operands are no longer read
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) red[(wave * F + rt * NS + t) * NM * kWave + mt * kWave + lane] = acc[rt][mt][t];
  __syncthreads();
  const int S = a.ksplit, j = lane & 15, g = lane >> 4;
  const size_t gsz = static_cast<size_t>(a.B) * ROWS * NM;
  // staged outputs [sequence of the workgroup][row of the workgroup], after the partial sums
  float* stage = reinterpret_cast<float*>(lb + static_cast<size_t>(kWavesM) * F * NM * kWave * 16);
  float* mine = a.part + (static_cast<size_t>(grp) * S + ks) * gsz;
  for (int f = wave; f < F; f += kWavesM) {
    const int rt = f / NS, t = f % NS;
    f4v v[NM];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
      const f4v* p = red + (f * NM + mt) * kWave + lane;
      v[mt] = p[0];
#pragma unroll
      for (int w = 1; w < kWavesM; ++w) v[mt] += p[w * (wstep / 4)];
    }
    const int rl = rt * kTileRows + j, row = row0 + rl;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int sq = s0 + t * kSeqTile + 4 * g + r;
      if (sq >= a.B) break;
      if (S > 1) {  // finalize_kernel adds the splits in index order (the kernel boundary makes
                    // every split visible, no fences needed)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) mine[(static_cast<size_t>(sq) * ROWS + rl) * NM + mt] = v[mt][r];
        continue;
      }
      if (row >= jb.rows) continue;
      const float post = post_p[sq - post_base];
      float* y = jb.y + sq * jb.ldy + row;
      float out;
      if (EPI == kEpiResidual) {
        out = *y + v[0][r] * post;
      } else if (EPI == kEpiSwiglu) {
        out = silu_m(v[0][r] * post) * (v[NM - 1][r] * post);
      } else {
        out = v[0][r] * post;
      }
      *y = out;
      if (a.em.on()) stage[(t * kSeqTile + 4 * g + r) * ROWS + rl] = out;
    }
  }
  if (S > 1 || !a.em.on()) return;
  // the outputs as the next product's tables: one (sequence, 32-row block) per half-wave
  __syncthreads();
  constexpr int kBlocksWg = ROWS / 32, kUnits = NS * kSeqTile * kBlocksWg;
  for (int u0 = 0; u0 < kUnits; u0 += kT / 32) {
    const int u = u0 + static_cast<int>(threadIdx.x) / 32, kk = threadIdx.x & 31;
    const bool ok = u < kUnits;
    const int sl = ok ? u / kBlocksWg : 0, blk = ok ? u % kBlocksWg : 0;
    const int sq = s0 + sl, rowg = row0 + blk * 32;
    const bool live = ok && sq < a.B && rowg < jb.rows;
    emit_block(a.em, sq, rowg >> 5, kk, live ? stage[sl * ROWS + blk * 32 + kk] : 0.0f, live);
  }
}

// RT row tiles of 16 rows per workgroup, NS sequence tiles of 16 sequences per workgroup.
// BS: block-scaled tables staged by the producing kernel (no preparation launch).
template <int EPI, int RT, int NS, bool BS>
__global__ __launch_bounds__(kT) void gemv_mfma_kernel(MArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lb[];
  __shared__ float s_post[BS ? NS * kSeqTile : 1];
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int ROWS = RT * kTileRows;
  const int nb = a.K >> 5;
  const int S = a.ksplit, grp = blockIdx.x / S, ks = blockIdx.x % S;
  const MJob jb = find_mjob(a, grp);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x & (kWave - 1);
  const int row0 = (grp - jb.tile_begin) * ROWS;
  const bool q4 = jb.qtype == EF_QTYPE_Q4_0;
  // this workgroup's blocks [kb0, kb1)
  const int kb0 = ks * a.blocks_per_split, kb1 = min(nb, kb0 + a.blocks_per_split);
  const int s0 = blockIdx.y * NS * kSeqTile;
  // A fragments through a buffer resource: the lane's 16 bytes at voffset 16 l, the wave-uniform
  // fragment offset in a scalar register (no per-lane address arithmetic)
  const uint32_t tstride = static_cast<uint32_t>(nb) * 2 * kWave * 16;  // bytes per sequence tile
  const __amdgpu_buffer_rsrc_t tab = make_rsrc(q4 ? a.t4 : a.t8, a.tab_bytes);
  const uint32_t tile0 = blockIdx.y * NS * tstride;
  f4v acc[RT][NM][NS];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int t = 0; t < NS; ++t) acc[rt][mt][t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  const int tile_row0 = row0 / kTileRows;
  if constexpr (BS) {
    // the epilogue factor of each of this workgroup's sequences: 1 / rms from the producer's
    // partial sums (in index order), or 1; the first row group's first split also hands them to
    // finalize_kernel
    // Eight threads per sequence: thread j adds partials j, j + 8, ... in order (eight loads in
    // flight), then the eight threads' DPP tree.  The order depends on nothing but the partials, so
    // every workgroup, launch shape and batch size gets the same factor for the same input.
    if (threadIdx.x < NS * kSeqTile * 8) {  // whole waves
      constexpr int G = 8;
      const int sl = threadIdx.x / G, j = threadIdx.x % G, sq = s0 + sl;
      const bool has = a.ssp != nullptr && sq < a.B;
      double tot = 0.0;
      if (has) {
        for (int p0 = 0; p0 < a.n_ssp; p0 += 8 * G) {
          double v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int p = p0 + j + i * G;
            v[i] = p < a.n_ssp ? a.ssp[static_cast<size_t>(p) * a.bpad + sq] : 0.0;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) tot += v[i];
        }
      }
      tot = group_sum_dpp<G>(tot);
      if (j == G - 1) {
        const float f =
            has ? static_cast<float>(1.0 / sqrt(tot / static_cast<double>(a.K) + static_cast<double>(a.eps))) : 1.0f;
        s_post[sl] = f;
        if (a.post_out != nullptr && blockIdx.x == 0 && sq < a.B) a.post_out[sq] = f;
      }
    }
    const __amdgpu_buffer_rsrc_t bsr =
        make_rsrc(a.bscale, static_cast<uint32_t>(nb) * static_cast<uint32_t>(a.bpad) * 4u);
    if (q4) {
      k_loop<RT, NM, NS, true, true>(jb, tile_row0, nb, kb0, kb1, wave, lane, tab, tile0, tstride, acc, bsr,
                                     static_cast<uint32_t>(a.bpad), static_cast<uint32_t>(s0));
    } else {
      k_loop<RT, NM, NS, false, true>(jb, tile_row0, nb, kb0, kb1, wave, lane, tab, tile0, tstride, acc, bsr,
                                      static_cast<uint32_t>(a.bpad), static_cast<uint32_t>(s0));
    }
    combine_and_store<EPI, RT, NS>(a, jb, lb, acc, wave, lane, row0, grp, ks, s0, s_post, s0);
  } else {
    if (q4) {
      k_loop<RT, NM, NS, true>(jb, tile_row0, nb, kb0, kb1, wave, lane, tab, tile0, tstride, acc, tab, 0u, 0u);
    } else {
      k_loop<RT, NM, NS, false>(jb, tile_row0, nb, kb0, kb1, wave, lane, tab, tile0, tstride, acc, tab, 0u, 0u);
    }
    combine_and_store<EPI, RT, NS>(a, jb, lb, acc, wave, lane, row0, grp, ks, s0, a.post, 0);
  }
}

struct FinArgs {
  MJob job[kMaxJobsM];
  int n_jobs, B, rows_wg, S, total;  // total = groups * rows_wg * B outputs
  const float* part;
  const float* post;
  AEmit em;
};

// One output (sequence, row) per thread: the splits' sums in index order, the scale, the epilogue.
// With em on, the 32 consecutive threads of a (sequence, 32-row block) also stage their outputs as
// the next product's tables (rows per group are a multiple of 32 then).
template <int EPI>
__global__ __launch_bounds__(256) void finalize_kernel(FinArgs a) {
  constexpr int NM = EPI == kEpiSwiglu ? 2 : 1;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in = idx < a.total;
  const int per_group = a.rows_wg * a.B;
  const int tile = in ? idx / per_group : 0, o = in ? idx % per_group : 0;
  MJob jb = a.job[0];
  for (int i = 1; i < a.n_jobs; ++i)
    if (tile >= a.job[i].tile_begin) jb = a.job[i];
  const int sq = o / a.rows_wg, row = (tile - jb.tile_begin) * a.rows_wg + o % a.rows_wg;
  const bool live = in && row < jb.rows;
  float out = 0.0f;
  if (live) {
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
      out = *y + v[0];
    } else if (EPI == kEpiSwiglu) {
      out = silu_m(v[0]) * v[NM - 1];
    } else {
      out = v[0];
    }
    *y = out;
  }
  if (a.em.on()) emit_block(a.em, sq, row >> 5, row & 31, out, live);
}

// (RT, NS) shapes the kernels are instantiated for: the ones whose registers fit in 256 VGPRs
// (two waves per SIMD) without spilling.  SwiGLU keeps two accumulators per output.
struct Shape {
  int RT, NS;
};
constexpr Shape kShapesStore[] = {{2, 1}, {2, 2}, {2, 4}, {4, 1}, {4, 2}, {4, 4}, {8, 1}, {8, 2}};
constexpr Shape kShapesSwiglu[] = {{2, 1}, {2, 2}, {2, 4}, {3, 1}, {3, 2}, {4, 1}, {4, 2}, {6, 1}};

template <int EPI, int RT, int NS, bool BS>
void* kfn() {
  return reinterpret_cast<void*>(&gemv_mfma_kernel<EPI, RT, NS, BS>);
}

// The instantiated kernel of shape (rt, ns): one of kShapesStore / kShapesSwiglu.
template <int EPI, bool BS = false>
void* pick_mfma(int rt, int ns) {
  if constexpr (EPI == kEpiSwiglu) {
    if (rt == 6) return kfn<EPI, 6, 1, BS>();
    if (rt == 4) return ns == 2 ? kfn<EPI, 4, 2, BS>() : kfn<EPI, 4, 1, BS>();
    if (rt == 3) return ns == 2 ? kfn<EPI, 3, 2, BS>() : kfn<EPI, 3, 1, BS>();
    return ns == 4 ? kfn<EPI, 2, 4, BS>() : (ns == 2 ? kfn<EPI, 2, 2, BS>() : kfn<EPI, 2, 1, BS>());
  } else {
    if (rt == 8) return ns == 2 ? kfn<EPI, 8, 2, BS>() : kfn<EPI, 8, 1, BS>();
    if (rt == 4) return ns == 4 ? kfn<EPI, 4, 4, BS>() : (ns == 2 ? kfn<EPI, 4, 2, BS>() : kfn<EPI, 4, 1, BS>());
    return ns == 4 ? kfn<EPI, 2, 4, BS>() : (ns == 2 ? kfn<EPI, 2, 2, BS>() : kfn<EPI, 2, 1, BS>());
  }
}

}  // namespace

namespace {

// Shape decisions of one batched launch and the workspace they need.
struct Plan {
  bool ok = false;
  bool q4 = false, q8 = false;
  int nm = 1, NT = 1, RT = 2, NS = 1, SG = 1, groups = 0, S = 1, bps = 0, chunk = 0;
  size_t tab = 0, part_off = 0, bytes = 0, lds = 0;
  double cost = 0.0;
};

int groups_for(const GemvJob* jobs, int n_jobs, int rows_wg) {
  int g = 0;
  for (int j = 0; j < n_jobs; ++j) g += static_cast<int>((jobs[j].W->rows + rows_wg - 1) / rows_wg);
  return g;
}

// Estimated time (CU cycles) of one shape: per workgroup its matrix-core time plus most of its
// vector-ALU time (measured on MI355X, the two overlap only partly), or its operand stream if that
// is longer; times the rounds of workgroups (one resident per CU), against the weights' HBM time;
// plus the split-K finalize launch and partial-sum traffic.  Per block and 16-row tile: 2 NS
// products of 16 cycles and about 12 + 4 NS VALU instructions of 4 cycles, over the CU's 4 SIMDs;
// 2 KB of A operands per sequence tile and the tile-block's weights through the CU's L2 port at
// ~40 B/cycle.
double shape_cost(int rt, int nm, int ns, int sg, int groups, int S, int bps, size_t wbytes, size_t part_bytes,
                  int cus, bool emit) {
  const double units = static_cast<double>(rt) * nm * bps;
  const double mfma = units * 2.0 * ns * 16.0 / 4.0;
  const double valu = units * (12.0 + 4.0 * ns) * 4.0 / 4.0;
  const double oper = (2048.0 * ns * bps + units * 300.0) / 40.0;
  const double wg = std::max(mfma + 0.7 * valu, oper) + 2500.0;
  const long wgs = static_cast<long>(groups) * S * sg;
  const double rounds = std::ceil(static_cast<double>(wgs) / cus);
  const double hbm = static_cast<double>(wbytes) * 2.4e9 / 5.0e12;  // cycles at 2.4 GHz, ~5 TB/s
  double t = std::max(rounds * wg, hbm + 2500.0);
  // launch + partial traffic; a finalize that also stages the next product's tables measured
  // 4.6 us per launch at B = 64 (emit)
  if (S > 1) t += (emit ? 11000.0 : 3600.0) + static_cast<double>(part_bytes) / (20.0 * cus);
  return t;
}

// even_rt: only shapes whose workgroup rows are a multiple of 32 (outputs staged as tables).
Plan plan_mfma(const GemvJob* jobs, int n_jobs, int epi, int batch, size_t ldx, bool even_rt = false) {
  Plan p;
  if (batch < 2 || n_jobs < 1 || n_jobs > kMaxJobsM) return p;
  const size_t K = jobs[0].W->cols;
  if (K % 32 != 0 || K > 65536) return p;
  size_t wbytes = 0;
  for (int j = 0; j < n_jobs; ++j) {
    if (jobs[j].W->qtype != EF_QTYPE_Q4_0 && jobs[j].W->qtype != EF_QTYPE_Q8_0) return Plan{};
    p.q4 = p.q4 || jobs[j].W->qtype == EF_QTYPE_Q4_0;
    p.q8 = p.q8 || jobs[j].W->qtype == EF_QTYPE_Q8_0;
    wbytes += jobs[j].W->rows * jobs[j].W->row_bytes * (jobs[j].W2 ? 2 : 1);
    if (jobs[j].x != jobs[0].x || (jobs[j].ldx ? jobs[j].ldx : ldx) != (jobs[0].ldx ? jobs[0].ldx : ldx))
      return p;  // one activation matrix per launch
  }
  const size_t xld = jobs[0].ldx ? jobs[0].ldx : ldx;
  if (reinterpret_cast<uintptr_t>(jobs[0].x) % 16 != 0 || xld % 4 != 0) return p;
  p.nm = epi == kEpiSwiglu ? 2 : 1;
  p.chunk = std::min(batch, kMaxTiles * kSeqTile);
  p.NT = (p.chunk + kSeqTile - 1) / kSeqTile;
  const int nb = static_cast<int>(K / 32);
  const int cus = ctx().cu_count > 0 ? ctx().cu_count : 256;
  const size_t lim = ctx().lds_per_block > 0 ? ctx().lds_per_block : 65536;
  // every instantiated (RT, NS) and split S whose LDS fits, the cheapest by shape_cost (ties: the
  // first found)
  bool found = false;
  const Shape* shapes = p.nm == 2 ? kShapesSwiglu : kShapesStore;
  const int n_shapes = p.nm == 2 ? static_cast<int>(sizeof(kShapesSwiglu) / sizeof(Shape))
                                 : static_cast<int>(sizeof(kShapesStore) / sizeof(Shape));
  for (int si = 0; si < n_shapes; ++si) {
    const int rt = shapes[si].RT, ns = shapes[si].NS;
    if (ns > 1 && p.NT < ns) continue;
    if (even_rt && rt % 2 != 0) continue;
    const int sg = (p.NT + ns - 1) / ns;
    const int rows_wg = rt * kTileRows;
    const int groups = groups_for(jobs, n_jobs, rows_wg);
    // the workgroup's partial sums of every wave in LDS for the reduction
    size_t lds = static_cast<size_t>(kWavesM) * rt * p.nm * ns * kWave * 4 * sizeof(float);
    if (even_rt) lds += static_cast<size_t>(rt) * kTileRows * ns * kSeqTile * sizeof(float);  // staged outputs
    if (lds > lim) continue;
    for (int s_try = 1; s_try <= std::min(32, std::max(1, nb / 8)); ++s_try) {
      const int bps = (nb + s_try - 1) / s_try;
      const int S = (nb + bps - 1) / bps;
      if (S != s_try || bps > kWavesM * max_blocks_per_wave(rt, p.nm, ns)) continue;
      const size_t part = S > 1 ? static_cast<size_t>(groups) * S * p.chunk * rows_wg * p.nm * sizeof(float) : 0;
      const double c = shape_cost(rt, p.nm, ns, sg, groups, S, bps, wbytes, 2 * part, cus, even_rt);
      if (!found || c < p.cost) {
        found = true;
        p.cost = c;
        p.RT = rt;
        p.NS = ns;
        p.SG = sg;
        p.groups = groups;
        p.S = S;
        p.bps = bps;
        p.lds = lds;
      }
    }
  }
  if (!found) return Plan{};
  // Layout: the A tables (every sequence tile of the grid, zeros past the batch), the scales, the
  // split-K partial sums.
  p.tab = static_cast<size_t>(p.SG) * p.NS * nb * 2 * kWave * 16;
  if (p.tab >= (size_t(1) << 32)) return Plan{};  // one buffer resource per table
  size_t off = (p.q4 ? p.tab : 0) + (p.q8 ? p.tab : 0) + kMaxTiles * kSeqTile * sizeof(float);
  off = (off + 255) & ~size_t(255);
  p.part_off = off;
  if (p.S > 1) off += static_cast<size_t>(p.groups) * p.S * p.chunk * p.RT * kTileRows * p.nm * sizeof(float);
  p.bytes = off;
  p.ok = true;
  return p;
}

}  // namespace

size_t tiled_bytes(const ef_hip_weight_s* w) {
  const size_t tiles = (w->rows + kTileRows - 1) / kTileRows, nb = w->cols / 32;
  return tiles * nb * (w->qtype == EF_QTYPE_Q4_0 ? kTileBlockQ4 : kTileBlockQ8);
}

namespace {
void launch_tile_layout(const ef_hip_weight_s* w, uint8_t* out, hipStream_t s) {
  const size_t tiles = (w->rows + kTileRows - 1) / kTileRows, nb = w->cols / 32;
  const size_t threads = tiles * nb * kWave;
  hipLaunchKernelGGL(tile_layout_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s, w->dev,
                     static_cast<int>(w->rows), static_cast<int>(nb), static_cast<int>(w->row_bytes),
                     w->qtype == EF_QTYPE_Q4_0 ? 1 : 0, out);
}
}  // namespace

int refresh_tiled(const ef_hip_weight_s* w, hipStream_t s) {
  if (w->tiled == nullptr) return EF_HIP_OK;
  launch_tile_layout(w, w->tiled, s);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int ensure_tiled(const ef_hip_weight_s* w, hipStream_t s) {
  if (w->tiled != nullptr) return EF_HIP_OK;
  EFH_CHECK(w->qtype == EF_QTYPE_Q4_0 || w->qtype == EF_QTYPE_Q8_0, "tile layout: packed types only");
  EFH_CHECK(w->cols % 32 == 0, "tile layout: cols must be a multiple of 32");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  EFH_HIP(hipStreamIsCapturing(s, &st));
  EFH_CHECK(st == hipStreamCaptureStatusNone,
            "batched GEMV: the weight's tile-order copy must be made before graph capture (a batched call "
            "outside capture, or engine creation, makes it)");
  const size_t bytes = tiled_bytes(w);
  EFH_CHECK(bytes < (size_t(1) << 32), "tile layout: matrix too large for one buffer resource");
  uint8_t* out = nullptr;
  EFH_HIP(hipMalloc(&out, bytes));
  launch_tile_layout(w, out, s);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    (void)hipFree(out);
    return fail_hip(e, "tile_layout_kernel");
  }
  w->tiled = out;
  return EF_HIP_OK;
}

int gemv_mfma_max_rows() { return kMaxTiles * kSeqTile; }

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
  for (int j = 0; j < n_jobs; ++j) {
    EFH_RC(ensure_tiled(jobs[j].W, stream));
    if (jobs[j].W2 != nullptr) EFH_RC(ensure_tiled(jobs[j].W2, stream));
  }
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
  a.ksplit = pl.S;
  a.blocks_per_split = pl.bps;
  a.part = reinterpret_cast<float*>(base + pl.part_off);
  void* fn = epi == kEpiStore ? pick_mfma<kEpiStore>(pl.RT, pl.NS)
                              : (epi == kEpiResidual ? pick_mfma<kEpiResidual>(pl.RT, pl.NS)
                                                     : pick_mfma<kEpiSwiglu>(pl.RT, pl.NS));
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
    const int nbk = static_cast<int>(K / 32);
    if (K <= static_cast<size_t>(kSeqPrepMaxK)) {  // tiles past B get zeros
      hipLaunchKernelGGL(xfrag_seq_kernel, dim3(pl.SG * pl.NS * kSeqTile), dim3(kSeqPrepThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL(xfrag_kernel, dim3((nbk + kPrepBlocks - 1) / kPrepBlocks, pl.SG * pl.NS), dim3(kTP), 0,
                         stream, p);
    }
    a.n_jobs = n_jobs;
    a.K = static_cast<int>(K);
    a.B = nb;
    a.n_tiles = pl.NT;
    a.t4 = t4;
    a.t8 = t8;
    a.tab_bytes = static_cast<uint32_t>(pl.tab);
    a.post = post;
    int tiles = 0;
    for (int j = 0; j < n_jobs; ++j) {
      MJob& d = a.job[j];
      const size_t yld = jobs[j].ldy ? jobs[j].ldy : ldy;
      d.W = jobs[j].W->tiled;
      d.W2 = jobs[j].W2 ? jobs[j].W2->tiled : nullptr;
      d.y = jobs[j].y + b0 * yld;
      d.rows = static_cast<int>(jobs[j].W->rows);
      d.qtype = jobs[j].W->qtype;
      d.bytes = static_cast<uint32_t>(tiled_bytes(jobs[j].W));
      d.ldy = static_cast<long>(yld);
      d.tile_begin = tiles;
      tiles += (d.rows + rows_wg - 1) / rows_wg;
    }
    void* params[] = {&a};
    // the chunk's sequences cover ceil(nb / 16) tiles; grid rows past them would have no sequences
    const int sg = std::min(pl.SG, (nb + pl.NS * kSeqTile - 1) / (pl.NS * kSeqTile));
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


size_t gemv_mfma_staged_workspace_bytes(const GemvJob* jobs, int n_jobs, int epi, int batch, bool emit) {
  const Plan p = plan_mfma(jobs, n_jobs, epi, batch, jobs[0].W->cols, emit);
  return p.ok ? p.bytes : 0;
}

static_assert(kStageMaxK == kSeqPrepMaxK, "launch_stage_tables limit");

size_t stage_table_bytes(int K, int batch) {
  const size_t tiles = (static_cast<size_t>(batch) + kSeqTile - 1) / kSeqTile;
  return tiles * static_cast<size_t>(K / 32) * 2 * kWave * 16;
}
int stage_bpad(int batch) { return ((batch + kSeqTile - 1) / kSeqTile) * kSeqTile; }

int launch_stage_tables(const float* x, size_t ldx, int K, int batch, const float* norm_w, const MfmaStage& st,
                        hipStream_t stream) {
  EFH_CHECK(K % 32 == 0 && K <= kStageMaxK && batch >= 1 && batch <= kMaxTiles * kSeqTile,
            "stage_tables: K must be a multiple of 32 up to 8192, batch in [1, 1024]");
  EFH_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0, "stage_tables: x rows must be 16-byte aligned");
  EFH_CHECK(st.bpad >= stage_bpad(batch) && st.bscale && st.ssp && (st.t4 || st.t8), "stage_tables: outputs");
  PrepArgs p{};
  p.x = x;
  p.ldx = static_cast<long>(ldx);
  p.K = K;
  p.B = batch;
  p.norm_w = norm_w;
  p.t4 = const_cast<uint8_t*>(st.t4);
  p.t8 = const_cast<uint8_t*>(st.t8);
  hipLaunchKernelGGL(xfrag_block_kernel, dim3(batch), dim3(kSeqPrepThreads), 0, stream, p,
                     const_cast<float*>(st.bscale), st.bpad, const_cast<double*>(st.ssp));
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

int launch_gemv_mfma_staged(const GemvJob* jobs, int n_jobs, int epi, const MfmaStage& st, int batch, size_t ldy,
                            void* ws, size_t ws_bytes, hipStream_t stream, const AEmit* em) {
  const size_t K = jobs[0].W->cols;
  const bool emit = em != nullptr && em->on();
  const Plan pl = plan_mfma(jobs, n_jobs, epi, batch, K, emit);
  if (emit) {
    EFH_CHECK(n_jobs == 1 && jobs[0].W->rows % 32 == 0 && static_cast<int>(jobs[0].W->rows / 32) == em->nb &&
                  em->bpad >= stage_bpad(batch),
              "gemv_mfma_staged: staging the outputs needs one job whose rows are the next product's K");
  }
  EFH_CHECK(pl.ok, "gemv_mfma_staged: no matrix-core plan for this launch");
  EFH_CHECK(batch <= pl.chunk, "gemv_mfma_staged: more sequences than one launch covers");
  EFH_CHECK((!pl.q4 || st.t4) && (!pl.q8 || st.t8), "gemv_mfma_staged: a table of the launch's column order is missing");
  EFH_CHECK(st.bscale != nullptr && st.bpad >= stage_bpad(batch), "gemv_mfma_staged: block scales");
  EFH_CHECK(ws != nullptr && ws_bytes >= pl.bytes, "gemv_mfma_staged: workspace too small");
  for (int j = 0; j < n_jobs; ++j) {
    EFH_RC(ensure_tiled(jobs[j].W, stream));
    if (jobs[j].W2 != nullptr) EFH_RC(ensure_tiled(jobs[j].W2, stream));
  }
  uint8_t* base = static_cast<uint8_t*>(ws);
  float* post = reinterpret_cast<float*>(base + (pl.q4 ? pl.tab : 0) + (pl.q8 ? pl.tab : 0));
  MArgs a{};
  a.ksplit = pl.S;
  a.blocks_per_split = pl.bps;
  a.part = reinterpret_cast<float*>(base + pl.part_off);
  a.n_jobs = n_jobs;
  a.K = static_cast<int>(K);
  a.B = batch;
  a.n_tiles = pl.NT;
  a.t4 = st.t4;
  a.t8 = st.t8;
  a.tab_bytes = static_cast<uint32_t>(stage_table_bytes(static_cast<int>(K), batch));
  a.post = post;
  a.bscale = st.bscale;
  a.bpad = st.bpad;
  a.ssp = st.ssp;
  a.n_ssp = st.n_ssp;
  a.eps = st.eps;
  a.post_out = pl.S > 1 ? post : nullptr;
  if (emit) a.em = *em;
  const int rows_wg = pl.RT * kTileRows;
  int tiles = 0;
  for (int j = 0; j < n_jobs; ++j) {
    MJob& d = a.job[j];
    const size_t yld = jobs[j].ldy ? jobs[j].ldy : ldy;
    d.W = jobs[j].W->tiled;
    d.W2 = jobs[j].W2 ? jobs[j].W2->tiled : nullptr;
    d.y = jobs[j].y;
    d.rows = static_cast<int>(jobs[j].W->rows);
    d.qtype = jobs[j].W->qtype;
    d.bytes = static_cast<uint32_t>(tiled_bytes(jobs[j].W));
    d.ldy = static_cast<long>(yld);
    d.tile_begin = tiles;
    tiles += (d.rows + rows_wg - 1) / rows_wg;
  }
  void* fn = epi == kEpiStore ? pick_mfma<kEpiStore, true>(pl.RT, pl.NS)
                              : (epi == kEpiResidual ? pick_mfma<kEpiResidual, true>(pl.RT, pl.NS)
                                                     : pick_mfma<kEpiSwiglu, true>(pl.RT, pl.NS));
  void* params[] = {&a};
  const int sg = std::min(pl.SG, (batch + pl.NS * kSeqTile - 1) / (pl.NS * kSeqTile));
  EFH_HIP(hipLaunchKernel(fn, dim3(tiles * pl.S, sg), dim3(kT), params, pl.lds, stream));
  if (pl.S > 1) {
    FinArgs f{};
    for (int j = 0; j < n_jobs; ++j) f.job[j] = a.job[j];
    f.n_jobs = n_jobs;
    f.B = batch;
    f.rows_wg = rows_wg;
    f.S = pl.S;
    f.total = tiles * rows_wg * batch;
    f.part = a.part;
    f.post = post;
    if (emit) f.em = *em;
    void* fin = epi == kEpiStore ? reinterpret_cast<void*>(&finalize_kernel<kEpiStore>)
                                 : (epi == kEpiResidual ? reinterpret_cast<void*>(&finalize_kernel<kEpiResidual>)
                                                        : reinterpret_cast<void*>(&finalize_kernel<kEpiSwiglu>));
    void* fparams[] = {&f};
    EFH_HIP(hipLaunchKernel(fin, dim3((f.total + 255) / 256), dim3(256), fparams, 0, stream));
  }
  return EF_HIP_OK;
}

}  // namespace efh
