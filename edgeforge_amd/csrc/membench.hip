// Achievable HBM read bandwidth: the reference's STREAM-style read test (include/ef/membench.h,
// src/membench.cpp) on the GPU.  A buffer of 64-bit words w[i] = i * 0x9E3779B97F4A7C15 +
// 0x0123456789ABCDEF is summed (mod 2^64) `passes` times per run by every CU, and the sum is
// checked against the closed form, so no read can be skipped or wrong.  Runs are timed with HIP
// events on the library stream; a 1 GiB default buffer is four times the 256 MB Infinity Cache,
// so the figure is HBM, not cache.  It is the software-achievable ceiling the GEMV fractions
// can be read against (the published 8 TB/s is the hardware peak).
#include <algorithm>
#include <vector>

#include "common.h"

namespace efh {
namespace {

constexpr uint64_t kMul = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kAdd = 0x0123456789ABCDEFull;
constexpr int kThreadsM = 256;

__global__ __launch_bounds__(kThreadsM) void fill_pattern_kernel(uint64_t* __restrict__ p, size_t words) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreadsM;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreadsM + threadIdx.x; i < words; i += stride)
    p[i] = i * kMul + kAdd;
}

// Every lane reads 16 bytes per step (two words), four steps in flight; `words` is a multiple of
// 2 * 4 * the grid's lane count (the host rounds the buffer), so there is no tail.
__global__ __launch_bounds__(kThreadsM) void read_sum_kernel(const uint64_t* __restrict__ p, size_t pairs,
                                                             int passes, unsigned long long* __restrict__ out) {
  using u64x2 = unsigned long long __attribute__((ext_vector_type(2)));
  const u64x2* v = reinterpret_cast<const u64x2*>(p);
  const size_t lanes = static_cast<size_t>(gridDim.x) * kThreadsM;
  const size_t first = static_cast<size_t>(blockIdx.x) * kThreadsM + threadIdx.x;
  unsigned long long s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  for (int pass = 0; pass < passes; ++pass) {
    for (size_t i = first; i < pairs; i += 4 * lanes) {
      const u64x2 a = __builtin_nontemporal_load(v + i);
      const u64x2 b = __builtin_nontemporal_load(v + i + lanes);
      const u64x2 c = __builtin_nontemporal_load(v + i + 2 * lanes);
      const u64x2 d = __builtin_nontemporal_load(v + i + 3 * lanes);
      s0 += a.x + a.y;
      s1 += b.x + b.y;
      s2 += c.x + c.y;
      s3 += d.x + d.y;
    }
  }
  unsigned long long s = (s0 + s1) + (s2 + s3);
  for (int off = kWave / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if ((threadIdx.x & (kWave - 1)) == 0) atomicAdd(out, s);  // wrapping adds commute: order-free
}

}  // namespace
}  // namespace efh

using namespace efh;

extern "C" {

uint64_t ef_hip_membench_expected_pass_sum(uint64_t n) {
  // sum_{i<n} (i * kMul + kAdd) = kMul * n (n - 1) / 2 + kAdd * n  (mod 2^64); the halving is done
  // on whichever factor is even so the product never needs more than 64 bits
  const uint64_t tri = n % 2 == 0 ? (n / 2) * (n - 1) : n * ((n - 1) / 2);
  return kMul * tri + kAdd * n;
}

int ef_hip_membench(const ef_hip_membench_options* o, ef_hip_membench_result* r) {
  EFH_RC(require_ready());
  EFH_CHECK(o != nullptr && r != nullptr, "membench: null argument");
  EFH_CHECK(o->buffer_bytes >= 64 * 1024, "membench: buffer must be at least 64 KiB");
  EFH_CHECK(o->runs >= 1, "membench: --runs must be >= 1");
  EFH_CHECK(o->passes >= 1, "membench: --passes must be >= 1");
  EFH_CHECK(o->warmup_runs >= 0, "membench: --warmup must be >= 0");
  const int blocks = std::max(ctx().cu_count, 1) * 8;
  const size_t unit = static_cast<size_t>(blocks) * kThreadsM * 8 * sizeof(uint64_t);  // 4 steps x 2 words
  const size_t bytes = static_cast<size_t>(o->buffer_bytes) / unit * unit;
  EFH_CHECK(bytes >= unit, "membench: buffer smaller than one sweep of the grid");
  size_t free_b = 0, total_b = 0;
  EFH_HIP(hipMemGetInfo(&free_b, &total_b));
  if (static_cast<double>(bytes) > 0.8 * static_cast<double>(free_b))
    return fail(EF_HIP_EINVAL, "membench: " + std::to_string(bytes >> 20) + " MiB requested but only " +
                                   std::to_string(free_b >> 20) + " MiB of device memory is free");
  const size_t words = bytes / sizeof(uint64_t);
  hipStream_t s = ctx().stream;
  uint64_t* buf = nullptr;
  unsigned long long* sum = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  auto cleanup = [&]() {
    if (buf) (void)hipFree(buf);
    if (sum) (void)hipFree(sum);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
  };
  if (hipMalloc(&buf, bytes) != hipSuccess || hipMalloc(&sum, sizeof(*sum)) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    cleanup();
    return fail(EF_HIP_ENOMEM, "membench: device buffer");
  }
  hipLaunchKernelGGL(fill_pattern_kernel, dim3(blocks), dim3(kThreadsM), 0, s, buf, words);
  const uint64_t want = ef_hip_membench_expected_pass_sum(words) * static_cast<uint64_t>(o->passes);
  std::vector<double> gbps;
  bool ok = true;
  unsigned long long got = 0;
  int rc = EF_HIP_OK;
  for (int run = 0; run < o->warmup_runs + o->runs && rc == EF_HIP_OK; ++run) {
    float ms = 0.0f;
    if (hipMemsetAsync(sum, 0, sizeof(*sum), s) != hipSuccess || hipEventRecord(e0, s) != hipSuccess) {
      rc = fail(EF_HIP_ERUNTIME, "membench: enqueue");
      break;
    }
    hipLaunchKernelGGL(read_sum_kernel, dim3(blocks), dim3(kThreadsM), 0, s, buf, words / 2, o->passes, sum);
    if (hipGetLastError() != hipSuccess || hipEventRecord(e1, s) != hipSuccess ||
        hipMemcpyAsync(&got, sum, sizeof(got), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
      rc = fail(EF_HIP_ERUNTIME, "membench: run");
      break;
    }
    ok = ok && got == want;
    if (run >= o->warmup_runs) gbps.push_back(static_cast<double>(bytes) * o->passes / (ms * 1e-3) / 1e9);
  }
  cleanup();
  if (rc != EF_HIP_OK) return rc;
  std::sort(gbps.begin(), gbps.end());
  const size_t m = gbps.size() / 2;
  r->buffer_bytes = bytes;
  r->passes = o->passes;
  r->bytes_per_run = static_cast<uint64_t>(bytes) * o->passes;
  r->best_gbps = gbps.back();
  r->worst_gbps = gbps.front();
  r->median_gbps = gbps.size() % 2 ? gbps[m] : 0.5 * (gbps[m - 1] + gbps[m]);
  r->checksum = got;
  r->expected_checksum = want;
  r->checksum_ok = ok ? 1 : 0;
  return EF_HIP_OK;
}

}  // extern "C"
