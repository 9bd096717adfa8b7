// Persistent decode step for one sequence: the embedding lookup and every layer of
// Transformer::forward (src/model.cpp:184-262) in ONE cooperative launch, one 1024-thread
// workgroup per CU, the phases (q/k/v, attention, o_proj, gate/up, down per layer) separated by
// grid barriers instead of kernel boundaries.
//
// Why: at one sequence every product is latency-bound.  A kernel boundary costs the launch gap,
// the kernel-argument fetch, the workgroups' start spread and the weights' first HBM round trip,
// which together exceed the work of most phases.  Here a phase's weights are fetched into LDS one
// or two phases ahead, so a phase is: barrier, activation fetch (L2-coherent), RMSNorm, dot
// products from LDS, stores.
//
// Memory model: activations crossing workgroups (x, q/k/v, ctx, act) are written with agent-
// coherent write-through stores and read with agent-coherent loads (cache policy sc1), so no L2
// writeback or invalidate is needed between phases; the barrier is one arrival flag per
// workgroup, stored the same way, which every workgroup polls.  Spins are bounded: a barrier that
// does not complete within kSpinLimit polls sets an error word and every workgroup leaves.
//
// Arithmetic: every row is computed exactly as gemv_dma_kernel computes it (32 lanes per row,
// block pairs p = t + 32 i, the same RMSNorm partial sums, block sums and group tree) and the
// attention as attention_wave_kernel, so logits are bit-identical to the multi-launch step.
#include <algorithm>
#include <string>

#include "gemv.h"
#include "qdot.h"
#include "step.h"

#pragma clang fp contract(off)

namespace efh {
namespace {

constexpr int kStepWaves = kStepThreads / kWave;  // 16
constexpr int kRowsPerPass = 2 * kStepWaves;      // two 32-lane row groups per wave
constexpr int kFetchWaves = 2;                    // the last two waves stage activations and run the barrier
constexpr int kFirstFetchWave = kStepWaves - kFetchWaves;
constexpr int kPrefetchWaves = kFirstFetchWave;   // waves 0..11 fetch weights for later phases
constexpr int kCoherent = 16;                     // cache policy sc1
constexpr unsigned kSpinLimit = 1u << 20;
constexpr int kFlagBase = 64;                     // sync words: [0] epoch, [1] error, flags at 64 + 16 g
constexpr int kSlotsFloats = (kStepMaxK / 64) * kSlot + kStepMaxK / 32;

__device__ __forceinline__ unsigned ld_coh_u(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) { return __uint_as_float(ld_coh_u(reinterpret_cast<const unsigned*>(p))); }
__device__ __forceinline__ void st_coh_u(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) { st_coh_u(reinterpret_cast<unsigned*>(p), __float_as_uint(v)); }

__device__ __forceinline__ void bare_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_all_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Phase descriptors are constant for the whole launch: read through the constant address space
// they become scalar loads, kept in SGPRs (a generic pointer would be read by vector loads).
#if defined(__HIP_DEVICE_COMPILE__)
typedef const __attribute__((address_space(4))) StepPhase const_phase_t;
#else
typedef const StepPhase const_phase_t;  // the host pass only parses the kernel
#endif
// Job j of a phase selected without indexing (j may differ between the lanes of a wave).
template <class PH>
__device__ __forceinline__ StepJob pick_job(const PH& P, int j) {
  StepJob J = P.job[0];
  if (j == 1) J = P.job[1];
  if (j == 2) J = P.job[2];
  return J;
}

struct WgRows {
  int r0, r1;
};
template <class PH>
__device__ __forceinline__ WgRows wg_rows(const PH& P, int wg) {
  const int r0 = wg * P.rpw;
  return {r0, min(r0 + P.rpw, P.rows)};
}

// This workgroup's rows of each job and where they sit in the weight region: job j's rows of W,
// then (SwiGLU) of W2, each span 16-byte aligned.
struct Spans {
  int lo[3], n[3];
  uint32_t off[3], off2[3];
};
template <class PH>
__device__ __forceinline__ Spans spans_of(const PH& P, WgRows w) {
  Spans s;
  uint32_t o = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    s.lo[j] = 0;
    s.n[j] = 0;
    s.off[j] = o;
    s.off2[j] = o;
    if (j < P.n_jobs) {
      const StepJob J = P.job[j];
      const int lo = max(w.r0, J.row0), hi = min(w.r1, J.row0 + J.rows);
      if (hi > lo) {
        s.lo[j] = lo - J.row0;
        s.n[j] = hi - lo;
        const uint32_t b = (static_cast<uint32_t>(s.n[j]) * static_cast<uint32_t>(J.row_bytes) + 15u) & ~15u;
        s.off[j] = o;
        o += b;
        if (P.epi == kEpiSwiglu) {
          s.off2[j] = o;
          o += b;
        }
      }
    }
  }
  return s;
}

// Weights of phase Q (this workgroup's rows) into `region`, as 1 KB LDS-DMA instructions spread
// over waves [0, nwaves).
template <class PH>
__device__ __forceinline__ void fetch_weights(const PH& Q, int wg, uint8_t* region, int wave, int nwaves,
                                              int lane) {
  const WgRows w = wg_rows(Q, wg);
  if (w.r0 >= w.r1) return;
  const Spans s = spans_of(Q, w);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    if (j >= Q.n_jobs || s.n[j] == 0) continue;
    const StepJob J = Q.job[j];
    const uint32_t rb = static_cast<uint32_t>(J.row_bytes);
    const uint32_t mat = static_cast<uint32_t>(J.rows) * rb;
    const uint32_t bytes = (static_cast<uint32_t>(s.n[j]) * rb + 15u) & ~15u;
    const uint32_t src = static_cast<uint32_t>(s.lo[j]) * rb;  // past the matrix end reads zeros
    for (int m = 0; m < (Q.epi == kEpiSwiglu ? 2 : 1); ++m) {
      const __amdgpu_buffer_rsrc_t r = make_rsrc(m ? J.W2 : J.W, mat);
      uint8_t* dst = region + (m ? s.off2[j] : s.off[j]);
      for (uint32_t k = static_cast<uint32_t>(wave) * 1024u; k < bytes; k += static_cast<uint32_t>(nwaves) * 1024u)
        if (k + 16u * lane < bytes) dma16<kNonTemporal>(r, dst + k, src + k + 16u * lane);
    }
  }
}

// `bytes` (a multiple of 16) from p to LDS by the fetch waves (fw = 0, 1), coherent or not.
template <int AUX>
__device__ __forceinline__ void fetch_span(const void* p, uint32_t bytes, uint8_t* dst, int fw, int lane) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
  for (uint32_t k = static_cast<uint32_t>(fw) * 1024u; k < bytes; k += kFetchWaves * 1024u)
    if (k + 16u * lane < bytes) dma16<AUX>(r, dst + k, k + 16u * lane);
}

// Normalises the staged activation into the padded slots + block sums (gemv_dma_kernel's stage:
// the sum of squares by threads 0..255 in that kernel's order, the same per-element arithmetic).
template <class PH>
__device__ __forceinline__ void stage_slots(const PH& P, const float* raw_x, const float* raw_nw,
                                            float* slots, double* red, int tid, int wave, int lane) {
  const int K = P.K, np = K >> 6;
  float* xs = slots + np * kSlot;
  auto put = [&](int i, float4 v) {
    *reinterpret_cast<float4*>(slots + (i >> 6) * kSlot + (i & 63)) = v;
    const float bs = group_sum_dpp<8>((v.x + v.y) + (v.z + v.w));
    if ((tid & 7) == 0) xs[i >> 5] = bs;
  };
  if (P.norm_w != nullptr) {
    double ss = 0.0;
    if (tid < 256) {
      for (int i = tid * 4; i < K; i += 1024) ss += sq_d(*reinterpret_cast<const float4*>(raw_x + i));
      ss = wave_sum_d_dpp(ss);
      if (lane == 0) red[wave] = ss;
    }
    bare_barrier();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w) tot += red[w];  // waves in order
    const float inv = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(K) + static_cast<double>(P.eps)));
    for (int i = tid * 4; i < K; i += 4 * kStepThreads) {
      const float4 v = *reinterpret_cast<const float4*>(raw_x + i);
      put(i, norm4(v, *reinterpret_cast<const float4*>(raw_nw + i), inv));
    }
  } else {
    for (int i = tid * 4; i < K; i += 4 * kStepThreads) put(i, *reinterpret_cast<const float4*>(raw_x + i));
  }
  bare_barrier();
}

// One row (two with SwiGLU: gate and up) per 32-lane group: gemv_dma_kernel's dma_body + tree.
template <int QT, int EPI>
__device__ __forceinline__ void row_dot(const uint8_t* w1, const uint8_t* w2, const float* slots, const float* xs,
                                        int np, int t, float (&acc)[2]) {
  constexpr int PB = PairOf<QT>::PD * 4;
  constexpr int RR = EPI == kEpiSwiglu ? 2 : 1;
  float a[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) a[r] = 0.0f;
  for (int p = t; p < np; p += 32) {
    uint32_t d[RR][PairOf<QT>::PD];
    lds_pair<QT, RR>(w1 + p * PB, d, 0);
    if (EPI == kEpiSwiglu) lds_pair<QT, RR>(w2 + p * PB, d, RR - 1);
    pair_dot<QT, RR>(d, slots + p * kSlot, xs[2 * p], xs[2 * p + 1], a);
  }
#pragma unroll
  for (int r = 0; r < RR; ++r) acc[r] = group_sum_dpp<32>(a[r]);
}

template <int EPI, class PH>
__device__ __forceinline__ void gemv_rows(const PH& P, int wg, const uint8_t* region, const float* slots,
                                          int wave, int lane) {
  const WgRows w = wg_rows(P, wg);
  const int nloc = w.r1 - w.r0;
  if (nloc <= 0) return;
  const Spans s = spans_of(P, w);
  const int np = P.K >> 6, t = lane & 31;
  const float* xs = slots + np * kSlot;
  for (int base = 0; base < nloc; base += kRowsPerPass) {
    const int i = base + 2 * wave + (lane >> 5);
    if (i >= nloc) continue;  // whole 32-lane groups
    const int g = w.r0 + i;
    const int j = (P.n_jobs > 1 && g >= P.job[1].row0) ? ((P.n_jobs > 2 && g >= P.job[2].row0) ? 2 : 1) : 0;
    const StepJob J = pick_job(P, j);
    // select, not index: a runtime index into the local arrays would put them in scratch memory
    const int lo = j == 0 ? s.lo[0] : (j == 1 ? s.lo[1] : s.lo[2]);
    const uint32_t off = j == 0 ? s.off[0] : (j == 1 ? s.off[1] : s.off[2]);
    const uint32_t off2 = j == 0 ? s.off2[0] : (j == 1 ? s.off2[1] : s.off2[2]);
    const uint32_t local = static_cast<uint32_t>(g - J.row0 - lo) * static_cast<uint32_t>(J.row_bytes);
    const uint8_t* w1 = region + off + local;
    const uint8_t* w2 = region + off2 + local;
    float acc[2] = {0.0f, 0.0f};
    if (J.qtype == EF_QTYPE_Q4_0) {
      row_dot<EF_QTYPE_Q4_0, EPI>(w1, w2, slots, xs, np, t, acc);
    } else {
      row_dot<EF_QTYPE_Q8_0, EPI>(w1, w2, slots, xs, np, t, acc);
    }
    if (t != 31) continue;  // lane 31 of each group holds the sums
    float* y = J.y + (g - J.row0);
    if (EPI == kEpiResidual) {
      st_coh(y, ld_coh(y) + acc[0]);
    } else if (EPI == kEpiSwiglu) {
      st_coh(y, silu_f(acc[0]) * acc[1]);
    } else {
      st_coh(y, acc[0]);
    }
  }
}

// Decode attention of one query head (one wave), attention_wave_kernel's arithmetic with the
// activations read coherently and the RoPE row taken from the tables at pos.  The wave holds its
// position's K row in registers (lane r: position c0 + r) and stages 64 V rows at a time in LDS
// (`vrows`, 16 KB) by LDS-DMA, four rows per instruction.
template <class PH>
__device__ __forceinline__ void attend_head(const PersistentArgs& a, const PH& P, int h, int pos, float* sm,
                                            float* vrows, int l) {
  constexpr int hd = 64;
  float* qs = sm;
  float* kn = sm + hd;
  float* sc = sm + 2 * hd;
  const int hpg = a.H / a.KV, g = h / hpg, kvd = a.KV * hd;
  const uint32_t span = static_cast<uint32_t>(a.max_seq - 1) * static_cast<uint32_t>(kvd) * 4u + hd * 4u;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(P.kc + g * hd, span);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(P.vc + g * hd, span);
  const uint32_t row_bytes = static_cast<uint32_t>(kvd) * 4u;
  // lane l of a V-row DMA: row l / 16 of the instruction's four, bytes 16 (l % 16) of it
  const uint32_t v_lane = static_cast<uint32_t>(l >> 4) * row_bytes + 16u * static_cast<uint32_t>(l & 15);
  auto stage_v = [&](int c0) {  // rows c0 .. c0 + 63 (past the cache end: zeros)
#pragma unroll
    for (int k = 0; k < 16; ++k)
      dma16<0>(rv, reinterpret_cast<uint8_t*>(vrows + 256 * k), static_cast<uint32_t>(c0 + 4 * k) * row_bytes + v_lane);
  };
  const int n0 = min(hd, a.max_seq);
  const float q0 = ld_coh(a.q + h * hd + l), q1 = ld_coh(a.q + h * hd + (l ^ 32));
  const float k0 = ld_coh(a.knew + g * hd + l), k1 = ld_coh(a.knew + g * hd + (l ^ 32));
  const float vnew = ld_coh(a.vnew + g * hd + l);
  const float cs = a.cos_t[static_cast<long>(pos) * 32 + (l & 31)], sn = a.sin_t[static_cast<long>(pos) * 32 + (l & 31)];
  float4 kr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) kr[i] = buf_f4(rk, static_cast<uint32_t>(l) * row_bytes + 16u * i);
  stage_v(0);
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
    P.kc[static_cast<long>(pos) * kvd + g * hd + l] = krot;
    P.vc[static_cast<long>(pos) * kvd + g * hd + l] = vnew;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
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
#pragma nounroll
  for (int c0 = hd; c0 < n_pos; c0 += hd) {
    const int r = c0 + l;
    if (r < n_pos) {
      if (r == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[i] = reinterpret_cast<const float4*>(kn)[i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[i] = buf_f4(rk, static_cast<uint32_t>(r) * row_bytes + 16u * i);
      }
      const float sv = dot64_regs(qs, kr) * a.scale;
      sc[r] = sv;
      mx = fmaxf(mx, sv);
    }
  }
  mx = wave_max_dpp(mx);
  const float e0 = l < c0n ? expf(s0 - mx) : 0.0f;
  double ssum = static_cast<double>(e0);
#pragma nounroll
  for (int r = hd + l; r < n_pos; r += hd) {
    const float e = expf(sc[r] - mx);
    sc[r] = e;
    ssum += static_cast<double>(e);
  }
  const float inv = static_cast<float>(1.0 / wave_sum_d_dpp(ssum));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  float o = 0.0f;
  for (int r = 0; r < c0n; ++r) {
    const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), r)) * inv;
    o += p * (r == pos ? vnew : vrows[r * hd + l]);
  }
#pragma nounroll
  for (int c0 = hd; c0 < n_pos; c0 += hd) {
    const int n = min(hd, n_pos - c0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous chunk's reads are done
    stage_v(c0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int r = 0; r < n; ++r) {
      const float p = sc[c0 + r] * inv;
      o += p * (c0 + r == pos ? vnew : vrows[r * hd + l]);
    }
  }
  st_coh(a.ctx + h * hd + l, o);
}

// Grid barrier number `epoch`: the fetch waves store this workgroup's flag and poll every
// workgroup's.  Returns false when the step is abandoned (a spin hit its limit here or elsewhere).
__device__ __forceinline__ bool grid_barrier(unsigned* sync, unsigned epoch, int wg, int nwg, int tid, int* s_abort) {
  bare_barrier();  // every wave has waited for its own stores
  constexpr int kPollFirst = kFirstFetchWave * kWave;
  if (tid == kPollFirst) st_coh_u(sync + kFlagBase + 16 * wg, epoch);
  if (tid >= kPollFirst) {
    for (int g = tid - kPollFirst; g < nwg; g += kFetchWaves * kWave) {
      unsigned it = 0;
      while (static_cast<int>(ld_coh_u(sync + kFlagBase + 16 * g) - epoch) < 0) {
        if ((++it & 63u) == 0u && (ld_coh_u(sync + 1) != 0u || it > kSpinLimit)) {
          st_coh_u(sync + 1, 1u);
          *s_abort = 1;
          break;
        }
      }
    }
  }
  bare_barrier();
  return *s_abort == 0;
}

__global__ __launch_bounds__(kStepThreads) void step_kernel(PersistentArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_region0[kStepRegion0];
  __shared__ __attribute__((aligned(16))) uint8_t s_region1[kStepRegion1];
  __shared__ __attribute__((aligned(16))) float s_slots[kSlotsFloats];
  __shared__ __attribute__((aligned(16))) float s_raw_x[kStepMaxK];
  __shared__ __attribute__((aligned(16))) float s_raw_nw[kStepMaxNormK];
  __shared__ double s_red[kStepWaves];
  __shared__ int s_abort;
  __shared__ unsigned s_epoch;

  const int tid0 = threadIdx.x, lane0 = tid0 & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid0 / kWave);
  const int wg = blockIdx.x, nwg = gridDim.x;
  if (tid0 == 0) {
    s_abort = 0;
    s_epoch = ld_coh_u(a.sync);
  }
  const int pos = __builtin_amdgcn_readfirstlane(*a.pos_dev);
  __syncthreads();
  const unsigned epoch0 = s_epoch;

  for (int ph = 0; ph < a.n_phases; ++ph) {
    const_phase_t& P = ((const_phase_t*)a.phases)[ph];
    // Lane-derived addresses are formed inside each phase: hoisted out of the phase loop, dozens of
    // them would stay live across every phase and spill.
    int lane = lane0, tid = tid0;
    asm volatile("" : "+v"(lane), "+v"(tid));
    if (P.kind == kPhaseGemv) {
      // 1. the activation (and norm weights) by the fetch waves; this phase's weights already sit
      //    in LDS (fetched by waves 0..11 in an earlier phase) unless the phase fetches its own
      if (wave >= kFirstFetchWave) {
        const int fw = wave - kFirstFetchWave;
        if (P.embed) {
          // the embedding row of the step's token, written to the residual stream as well
        } else {
          fetch_span<kCoherent>(P.x, static_cast<uint32_t>(P.K) * 4u, reinterpret_cast<uint8_t*>(s_raw_x), fw, lane);
        }
        if (P.norm_w != nullptr)
          fetch_span<0>(P.norm_w, static_cast<uint32_t>(P.K) * 4u, reinterpret_cast<uint8_t*>(s_raw_nw), fw, lane);
      } else if (P.own) {
        if (P.region == 0) {
          fetch_weights(P, wg, s_region0, wave, kPrefetchWaves, lane);
        } else {
          fetch_weights(P, wg, s_region1, wave, kPrefetchWaves, lane);
        }
      }
      wait_all_vm();
      if (P.embed) {
        const int32_t id = a.hist[pos];
        const bool ok = id >= 0 && id < a.embed_rows;
        const uint8_t* row = a.embed + (ok ? id : 0) * a.embed_rb;
        for (int i = tid; i < P.K; i += kStepThreads) s_raw_x[i] = ok ? decode_elem(row, a.embed_qtype, i) : __int_as_float(0x7FC00000);
        __syncthreads();
        const int per = (a.D + nwg - 1) / nwg;
        if (tid < per && wg * per + tid < a.D) st_coh(a.x + wg * per + tid, s_raw_x[wg * per + tid]);
      }
      bare_barrier();
      // 2. RMSNorm + slots, 3. rows
      stage_slots(P, s_raw_x, s_raw_nw, s_slots, s_red, tid, wave, lane);
      const uint8_t* region = P.region == 0 ? s_region0 : s_region1;
      if (P.epi == kEpiSwiglu) {
        gemv_rows<kEpiSwiglu>(P, wg, region, s_slots, wave, lane);
      } else if (P.epi == kEpiResidual) {
        gemv_rows<kEpiResidual>(P, wg, region, s_slots, wave, lane);
      } else {
        gemv_rows<kEpiStore>(P, wg, region, s_slots, wave, lane);
      }
    } else {
      if (wg < a.H && wave == kFirstFetchWave) attend_head(a, P, wg, pos, s_raw_x, s_slots, lane);
    }
    if (ph + 1 == a.n_phases) break;
    // 4. weights of a later phase into the region this phase no longer reads, then the barrier
    wait_all_vm();   // this wave's stores have completed (before its workgroup's flag is raised)
    bare_barrier();  // ... and every wave is done reading this phase's weights
    if (P.pf >= 0 && wave < kPrefetchWaves) {
      const_phase_t& Q = ((const_phase_t*)a.phases)[P.pf];
      if (Q.region == 0) {
        fetch_weights(Q, wg, s_region0, wave, kPrefetchWaves, lane);
      } else {
        fetch_weights(Q, wg, s_region1, wave, kPrefetchWaves, lane);
      }
    }
    if (!grid_barrier(a.sync, epoch0 + static_cast<unsigned>(ph) + 1u, wg, nwg, tid, &s_abort)) break;
  }
  if (wg == 0 && tid0 == 0) st_coh_u(a.sync, epoch0 + static_cast<unsigned>(a.n_phases));
}

}  // namespace

int step_groups() { return std::min(ctx().cu_count > 0 ? ctx().cu_count : 256, kStepMaxGroups); }

std::string step_unsupported(const StepPhase* phases, int n_phases, int groups, int hd, int H, int KV, int max_seq,
                             int D) {
  if (hd != 64) return "head_dim must be 64";
  if (H > groups) return "more query heads than workgroups";
  if (max_seq + 2 * hd > kStepMaxK) return "max_seq too large for the staged scores";
  (void)KV;
  if (D > kStepMaxK) return "hidden size too large";
  for (int i = 0; i < n_phases; ++i) {
    const StepPhase& P = phases[i];
    if (P.kind != kPhaseGemv) continue;
    if (P.K % 64 != 0 || P.K > kStepMaxK) return "activation length must be a multiple of 64 up to 6144";
    if (P.norm_w != nullptr && P.K > kStepMaxNormK) return "fused RMSNorm over more than 2048 values";
    size_t bytes = 0;
    // the largest per-workgroup span set: rows [r0, r1) of every workgroup
    for (int g = 0; g < groups; ++g) {
      const int r0 = g * P.rpw, r1 = std::min(r0 + P.rpw, P.rows);
      size_t b = 0;
      for (int j = 0; j < P.n_jobs; ++j) {
        const StepJob& J = P.job[j];
        if (J.qtype != EF_QTYPE_Q4_0 && J.qtype != EF_QTYPE_Q8_0) return "packed Q4_0 / Q8_0 matrices only";
        const int lo = std::max(r0, J.row0), hi = std::min(r1, J.row0 + J.rows);
        if (hi > lo) b += ((static_cast<size_t>(hi - lo) * J.row_bytes + 15) & ~size_t(15)) * (P.epi == kEpiSwiglu ? 2 : 1);
      }
      bytes = std::max(bytes, b);
    }
    if (bytes > static_cast<size_t>(P.region == 0 ? kStepRegion0 : kStepRegion1)) return "a phase's rows exceed its LDS region";
  }
  return std::string();
}

std::string step_launch_unsupported() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&step_kernel), kStepThreads,
                                                   0) != hipSuccess)
    return "occupancy query failed";
  if (per_cu < 1 || ctx().cu_count < step_groups()) return "the step kernel's workgroups do not fit one per CU";
  return std::string();
}

int launch_step(const PersistentArgs& a, hipStream_t s) {
  void* params[] = {const_cast<PersistentArgs*>(&a)};
  EFH_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&step_kernel), dim3(step_groups()),
                                     dim3(kStepThreads), params, 0, s));
  return EF_HIP_OK;
}

}  // namespace efh
