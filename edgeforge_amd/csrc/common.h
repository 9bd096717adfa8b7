// Shared internals of libedgeforge_hip.so: device context, error reporting, weight handles and
// small device helpers used by several kernels.  gfx950 (MI355X) only: wave64, 160 KB LDS per CU.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/ef_hip.h"

namespace efh {

constexpr int kWave = 64;

// ---- error reporting (per calling thread) ---------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int fail_hip(hipError_t e, const char* what);

#define EFH_HIP(call)                                         \
  do {                                                        \
    hipError_t efh_e_ = (call);                               \
    if (efh_e_ != hipSuccess) return ::efh::fail_hip(efh_e_, #call); \
  } while (0)

#define EFH_RC(expr)                                  \
  do {                                                \
    int efh_rc_ = (expr);                             \
    if (efh_rc_ != EF_HIP_OK) return efh_rc_;         \
  } while (0)

#define EFH_CHECK(cond, msg)                                  \
  do {                                                        \
    if (!(cond)) return ::efh::fail(EF_HIP_EINVAL, (msg));    \
  } while (0)

// ---- context ----------------------------------------------------------------------------------
struct Context {
  bool ready = false;
  int device = -1;
  int cu_count = 0;
  size_t lds_per_block = 0;
  hipStream_t stream = nullptr;  // library default stream (default priority)
  char name[256] = {};
};
Context& ctx();
int require_ready();
inline hipStream_t pick(void* s) { return s ? static_cast<hipStream_t>(s) : ctx().stream; }

}  // namespace efh

// ---- weight handle (opaque in the C-ABI) ------------------------------------------------------
struct ef_hip_weight_s {
  int qtype = 0;
  size_t rows = 0, cols = 0, row_bytes = 0;
  const uint8_t* dev = nullptr;
  bool owned = false;
  uint32_t magic = 0;
  // Copy of a Q4_0 / Q8_0 matrix in the batched GEMV's tile order (gemv_mfma.hip), made on the
  // first batched use or at engine creation, freed with the handle.
  mutable uint8_t* tiled = nullptr;
};

namespace efh {

constexpr uint32_t kWeightMagic = 0x45464857u;  // "EFHW"
int check_weight(ef_hip_weight w);
size_t row_bytes_of(int qtype, size_t cols);  // 0 when invalid

// ---- device helpers ---------------------------------------------------------------------------
__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
  // v_cvt_f32_f16 is exact for every binary16 value (subnormals, inf, NaN).
  _Float16 h;
  const uint16_t b = static_cast<uint16_t>(h16);
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

// Raw buffer resources (CDNA dword-3 format bits for 32-bit raw data).  Accesses at or beyond
// num_records return zeros without touching memory, so loads through them need no branch and the
// compiler can count outstanding loads exactly.
constexpr int kRawBufferFlags = 0x00020000;
constexpr int kNonTemporal = 2;  // cache policy of streamed, read-once data
typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kRawBufferFlags);
}

__device__ __forceinline__ float4 buf_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Cross-lane sums on the data-parallel-primitive (DPP) paths: a VALU operand modifier, where a
// __shfl_xor is an LDS permute with its round trip.  gfx9 DPP controls: quad_perm [1,0,3,2] (0xB1)
// and [2,3,0,1] (0x4E), row_mirror (0x140), row_half_mirror (0x141), row_bcast:15 (0x142) and
// row_bcast:31 (0x143); a row is 16 lanes, lanes outside row_mask read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b & 0xFFFFFFFFu), CTRL, ROW_MASK, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), CTRL, ROW_MASK, 0xF, false);
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 32) |
                                                     static_cast<unsigned>(lo)));
}

// Sum over aligned groups of G lanes (G = 8, 16 or 32).  G = 8, 16: every lane of a group holds
// its sum; G = 32: lanes 16..31 of each half-wave do.  Lane G - 1 of a group always does.
template <int G, typename T>
__device__ __forceinline__ T group_sum_dpp(T v) {
  auto mv = [](T x, auto ctrl) {
    if constexpr (sizeof(T) == 8) {
      return dpp_d<decltype(ctrl)::value>(x);
    } else {
      return dpp_f<decltype(ctrl)::value>(x);
    }
  };
  v = v + mv(v, std::integral_constant<int, 0xB1>{});
  v = v + mv(v, std::integral_constant<int, 0x4E>{});
  v = v + mv(v, std::integral_constant<int, 0x141>{});
  if constexpr (G >= 16) v = v + mv(v, std::integral_constant<int, 0x140>{});
  if constexpr (G >= 32) {
    if constexpr (sizeof(T) == 8) {
      v = v + dpp_d<0x142, 0xA>(v);
    } else {
      v = v + dpp_f<0x142, 0xA>(v);
    }
  }
  return v;
}

// Wave-wide float max through DPP, returned on every lane.  Lanes a DPP step does not feed keep
// their own value (max with itself), so negative values are safe.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_self_f(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_self_f<0xB1>(v));
  v = fmaxf(v, dpp_self_f<0x4E>(v));
  v = fmaxf(v, dpp_self_f<0x141>(v));
  v = fmaxf(v, dpp_self_f<0x140>(v));
  v = fmaxf(v, dpp_self_f<0x142, 0xA>(v));
  v = fmaxf(v, dpp_self_f<0x143, 0xC>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave-wide unsigned max through DPP, returned on every lane (lanes a step does not feed keep their
// own value).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_self_u(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  v = max(v, dpp_self_u<0xB1>(v));
  v = max(v, dpp_self_u<0x4E>(v));
  v = max(v, dpp_self_u<0x141>(v));
  v = max(v, dpp_self_u<0x140>(v));
  v = max(v, dpp_self_u<0x142, 0xA>(v));
  v = max(v, dpp_self_u<0x143, 0xC>(v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Wave-wide double sum through DPP, returned on every lane (lane 63 holds it, then a broadcast).
__device__ __forceinline__ double wave_sum_d_dpp(double v) {
  v = group_sum_dpp<32>(v);
  v = v + dpp_d<0x143, 0xC>(v);
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = __builtin_amdgcn_readlane(static_cast<int>(b & 0xFFFFFFFFu), 63);
  const unsigned hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), 63);
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

}  // namespace efh
