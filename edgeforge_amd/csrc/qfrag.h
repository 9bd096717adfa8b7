// Matrix-core operands of packed Q4_0 / Q8_0 codes (v_mfma_f32_16x16x32_f16), shared by the
// batched GEMV kernels.
//
// B operand: a lane's 8 codes minus their bias as exact fp16, straight out of the packed bytes.
// One AND-OR of a code dword with the fp16 pattern of 1024 yields two codes as 1024 + c
// ((q & 0x000F000F) | 0x64006400: the low nibbles of bytes 0 and 2; the high nibbles through
// 0x00F000F0 come out as 1024 + 16 c), and one packed fp16 add removes 1024 + 8 (1024 + 128 for the
// scaled high nibbles) exactly.  Q8_0 codes are offset to unsigned (q ^ 0x80) and taken two per
// AND-OR the same way, minus 1024 + 128.
//
// Slot orders (the A operand's columns must follow them):
//   q4_operand(q), q = bytes (b0, b1, b2, b3):  lo(b0) lo(b2) 16hi(b0) 16hi(b2) lo(b1) lo(b3) 16hi(b1) 16hi(b3)
//   q8_operand(q0, q1):                         q0.b0 q0.b2 q0.b1 q0.b3 q1.b0 q1.b2 q1.b1 q1.b3
// (lo / hi: the byte's low / high nibble; a Q4_0 byte j holds weights j and j + 16 of its block.)
#pragma once

#include "common.h"

namespace efh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

// (v & mask) | fp16(1024) pattern in both halves, minus (1024 + bias) in both halves: exact.  The
// mask comes in a scalar register and the pattern in a vector register, so that the AND-OR is one
// v_and_or_b32 (its three-operand encoding takes no literal constants).
__device__ __forceinline__ uint32_t codes2(uint32_t v, uint32_t mask, _Float16 minus) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(mask);
  uint32_t pat = 0x64006400u, r;
  asm("" : "+v"(pat));  // keep the pattern in a register
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(pat));
  h2 h;
  __builtin_memcpy(&h, &r, 4);
  const h2 c = {minus, minus};
  h = h + c;
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

}  // namespace efh
