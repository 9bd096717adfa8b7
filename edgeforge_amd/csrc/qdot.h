// Device building blocks of the packed Q4_0 / Q8_0 dot products shared by the decode GEMV
// (gemv.hip) and the persistent decode-step kernel (step.hip): staged-activation slots, block-pair
// dot products over the reference's 18 / 34-byte blocks (include/ef/quant.h:22-35), LDS-DMA
// fetches and LDS accesses the compiler does not see.
#pragma once

#include "common.h"

namespace efh {
namespace {

constexpr int kSlot = 68;  // 64 floats of a block pair + 4 floats of bank padding

// Element c of a row in any storage type (kern::row_f32: exact for F32 / F16 / BF16, code times
// scale for Q4_0 / Q8_0, src/quant.cpp:158-249).
__device__ __forceinline__ float decode_elem(const uint8_t* row, int qtype, long c) {
  if (qtype == EF_QTYPE_F32) return reinterpret_cast<const float*>(row)[c];
  if (qtype == EF_QTYPE_BF16) return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(row)[c]) << 16);
  if (qtype == EF_QTYPE_F16) return half_bits_to_float(reinterpret_cast<const uint16_t*>(row)[c]);
  const long blk = c >> 5, j = c & 31;
  if (qtype == EF_QTYPE_Q4_0) {
    const uint8_t* p = row + blk * 18;
    const float d = half_bits_to_float(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
    const int code = j < 16 ? (p[2 + j] & 15) : (p[2 + j - 16] >> 4);
    return static_cast<float>(code - 8) * d;
  }
  const uint8_t* p = row + blk * 34;
  const float d = half_bits_to_float(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
  return static_cast<float>(static_cast<int8_t>(p[2 + j])) * d;
}

__device__ __forceinline__ double sq_d(float4 v) {
  double ss = static_cast<double>(v.x) * static_cast<double>(v.x);
  ss += static_cast<double>(v.y) * static_cast<double>(v.y);
  ss += static_cast<double>(v.z) * static_cast<double>(v.z);
  ss += static_cast<double>(v.w) * static_cast<double>(v.w);
  return ss;
}

__device__ __forceinline__ float4 norm4(float4 v, float4 w, float inv) {  // HF order: w * (x * inv)
  v.x = w.x * (v.x * inv);
  v.y = w.y * (v.y * inv);
  v.z = w.z * (v.z * inv);
  v.w = w.w * (v.w * inv);
  return v;
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

template <int QT>
struct PairOf {
  static constexpr int PD = QT == EF_QTYPE_Q4_0 ? 9 : 17;  // dwords per block pair (36 / 68 bytes)
};

// Adds one staged block pair's dot product with the RR weight rows held in d.
template <int QT, int RR>
__device__ __forceinline__ void pair_dot(const uint32_t (&d)[RR][PairOf<QT>::PD], const float* slot, float xsA,
                                         float xsB, float (&acc)[RR]) {
  float4 xv[8];
  // block A of the pair: scale in bytes 0-1, codes from byte 2 (realigned by 2 bytes)
  load_x_block(slot, xv);
#pragma unroll
  for (int r = 0; r < RR; ++r) {
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
#pragma unroll
  for (int r = 0; r < RR; ++r) {
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

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }  // src/kernels.cpp:94

typedef __attribute__((address_space(3))) void lds_void;

template <int AUX>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, uint32_t voff) {
  // lds_dst is wave-uniform: the 16 bytes of lane l land at lds_dst + 16 l
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(lds_dst), 16, voff, 0, 0, AUX);
}

// Copies `bytes` (a multiple of 16) from buffer offset src_off to LDS as 1 KB wave instructions.
template <int AUX>
__device__ __forceinline__ void dma_span(__amdgpu_buffer_rsrc_t r, uint32_t src_off, uint8_t* lds_dst, uint32_t bytes,
                                         int lane) {
  for (uint32_t o = 0; o < bytes; o += 1024u) {
    if (o + 16u * lane < bytes) dma16<AUX>(r, lds_dst + o, src_off + o + 16u * lane);
  }
}

// LDS accesses the compiler does not see (inline assembly).  After an LDS-DMA load the compiler
// makes every later LDS access of the same array wait for all outstanding vector-memory operations,
// which would make the x staging wait for the weight rows it is meant to overlap; these helpers
// wait only for their own LDS operation.
__device__ __forceinline__ uint32_t lds_off(const void* p) {
  typedef const __attribute__((address_space(3))) void* lds_ptr;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}
typedef float f4n __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 lds_read4(const float* p) {
  f4n v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_off(p)) : "memory");
  return make_float4(v.x, v.y, v.z, v.w);
}
// Two 16-byte LDS reads issued together, one wait for both.
__device__ __forceinline__ void lds_read4x2(const float* p0, const float* p1, float4& v0, float4& v1) {
  f4n a, b;
  asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(a), "=&v"(b)
               : "v"(lds_off(p0)), "v"(lds_off(p1))
               : "memory");
  v0 = make_float4(a.x, a.y, a.z, a.w);
  v1 = make_float4(b.x, b.y, b.z, b.w);
}
__device__ __forceinline__ void lds_read4x4(const float* p0, const float* p1, const float* p2, const float* p3,
                                            float4& v0, float4& v1, float4& v2, float4& v3) {
  f4n a, b, c, d;
  asm volatile(
      "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
      : "v"(lds_off(p0)), "v"(lds_off(p1)), "v"(lds_off(p2)), "v"(lds_off(p3))
      : "memory");
  v0 = make_float4(a.x, a.y, a.z, a.w);
  v1 = make_float4(b.x, b.y, b.z, b.w);
  v2 = make_float4(c.x, c.y, c.z, c.w);
  v3 = make_float4(d.x, d.y, d.z, d.w);
}
__device__ __forceinline__ void lds_write4(float* p, float4 v) {
  const f4n w = {v.x, v.y, v.z, v.w};
  asm volatile("ds_write_b128 %0, %1" : : "v"(lds_off(p)), "v"(w) : "memory");
}
__device__ __forceinline__ void lds_write1(float* p, float v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(lds_off(p)), "v"(v) : "memory");
}
// Workgroup barrier after this wave's LDS writes completed, without waiting for vector memory.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Waits until at most n of this wave's vector-memory operations are outstanding (n wave-uniform;
// counts above 24 wait for all).  Operations retire in issue order, so issuing x before the weight
// rows lets the x staging start while the rows are still in flight.
__device__ __forceinline__ void wait_vmcnt_at_most(int n) {
  switch (n) {
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

template <int QT, int RR>
__device__ __forceinline__ void lds_pair(const uint8_t* p, uint32_t (&d)[RR][PairOf<QT>::PD], int r) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int k = 0; k < PairOf<QT>::PD; ++k) d[r][k] = q[k];
}

// q . k over 64 values, q in LDS and k in registers, in kern::dot_f32's order: partial j sums the
// products i = j mod 8 in increasing i, then ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7))
// (src/kernels.cpp:27-43), multiplies and adds kept apart (no contraction into FMA).
__device__ __forceinline__ float dot64_regs(const float* qv, const float4 (&kr)[16]) {
#pragma clang fp contract(off)
  float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f, p4 = 0.0f, p5 = 0.0f, p6 = 0.0f, p7 = 0.0f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float4 qa = *reinterpret_cast<const float4*>(qv + 8 * m), qb = *reinterpret_cast<const float4*>(qv + 8 * m + 4);
    const float4 ka = kr[2 * m], kb = kr[2 * m + 1];
    p0 += qa.x * ka.x;
    p1 += qa.y * ka.y;
    p2 += qa.z * ka.z;
    p3 += qa.w * ka.w;
    p4 += qb.x * kb.x;
    p5 += qb.y * kb.y;
    p6 += qb.z * kb.z;
    p7 += qb.w * kb.w;
  }
  return ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7));
}

}  // namespace
}  // namespace efh
