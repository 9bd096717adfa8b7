// Quality measures of eval-quant on device logits (src/eval_quant.cpp:48-102): per position,
// the log-sum-exp of each distribution, KL(P_ref || P_ours) in double, top-1 agreement, whether the
// reference is confident (p_top1 >= 0.5), finiteness of ours; and the negative log-likelihood of a
// target token.  One workgroup per position; sums over the vocabulary are per-thread partials
// combined in a fixed order (the reference adds left to right: the results differ in the last bits
// of a double).  Aggregation over positions is done by the caller in position order.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.h"

namespace efh {
namespace {

constexpr int kThreadsE = 1024;
constexpr int kWavesE = kThreadsE / kWave;

// Block-wide max / sum of doubles (every thread gets the result).
__device__ double block_max(double v, double* red) {
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  double m = red[0];
  for (int w = 1; w < kWavesE; ++w) m = fmax(m, red[w]);
  __syncthreads();
  return m;
}

__device__ double block_sum(double v, double* red) {
  v = wave_sum_d(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  double s = 0.0;
  for (int w = 0; w < kWavesE; ++w) s += red[w];
  __syncthreads();
  return s;
}

// log_sum_exp (src/eval_quant.cpp:52-58): max in double, then log of the sum of exp(x - max).
__device__ double lse(const float* x, int V, double* red) {
  double m = -INFINITY;
  for (int i = threadIdx.x; i < V; i += kThreadsE) m = fmax(m, static_cast<double>(x[i]));
  m = block_max(m, red);
  double s = 0.0;
  for (int i = threadIdx.x; i < V; i += kThreadsE) s += exp(static_cast<double>(x[i]) - m);
  return m + log(block_sum(s, red));
}

// kern::argmax (src/kernels.cpp:105-111): first maximum by strict '>' from index 0 (a NaN never
// wins, and a NaN at index 0 is kept).  Returns the index on every thread.
__device__ int block_argmax(const float* x, int V, float* rv, int* ri) {
  float best = x[0];
  int bi = 0;
  for (int i = threadIdx.x; i < V; i += kThreadsE) {
    if (x[i] > best) {
      best = x[i];
      bi = i;
    }
  }
  // combine (value, index): larger value wins, equal values the lower index; NaN values only
  // stay when nothing is larger (as a left-to-right strict scan from x[0])
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & (kWave - 1)) == 0) {
    rv[threadIdx.x / kWave] = best;
    ri[threadIdx.x / kWave] = bi;
  }
  __syncthreads();
  float b = rv[0];
  int id = ri[0];
  for (int w = 1; w < kWavesE; ++w) {
    if (rv[w] > b || (rv[w] == b && ri[w] < id)) {
      b = rv[w];
      id = ri[w];
    }
  }
  __syncthreads();
  return id;
}

// out[p] = {kl, top1, confident, finite} for position p (compare_dist, src/eval_quant.cpp:60-75).
__global__ __launch_bounds__(kThreadsE) void compare_dist_kernel(const float* ref, const float* ours, int V, long ld_ref,
                                                                 long ld_ours, double* kl, int* flags) {
  __shared__ double red[kWavesE];
  __shared__ float rv[kWavesE];
  __shared__ int ri[kWavesE];
  const long p = blockIdx.x;
  const float* r = ref + p * ld_ref;
  const float* q = ours + p * ld_ours;
  int fin = 1;
  for (int i = threadIdx.x; i < V; i += kThreadsE) fin &= isfinite(q[i]) ? 1 : 0;
  fin = block_sum(static_cast<double>(fin), red) == static_cast<double>(kThreadsE) ? 1 : 0;
  if (!fin) {
    if (threadIdx.x == 0) {
      kl[p] = 0.0;
      flags[p] = 0;
    }
    return;
  }
  const double lr = lse(r, V, red), lq = lse(q, V, red);
  double s = 0.0;
  for (int i = threadIdx.x; i < V; i += kThreadsE) {
    const double a = static_cast<double>(r[i]) - lr, b = static_cast<double>(q[i]) - lq;
    s += exp(a) * (a - b);
  }
  s = block_sum(s, red);
  const int ar = block_argmax(r, V, rv, ri);
  const int aq = block_argmax(q, V, rv, ri);
  if (threadIdx.x == 0) {
    kl[p] = fmax(s, 0.0);
    const int confident = exp(static_cast<double>(r[ar]) - lr) >= 0.5 ? 1 : 0;
    flags[p] = 1 | (ar == aq ? 2 : 0) | (confident ? 4 : 0);
  }
}

// nll[p] = log_sum_exp(logits_p) - logits_p[target_p] (neg_log_prob, src/eval_quant.cpp:100-102).
__global__ __launch_bounds__(kThreadsE) void nll_kernel(const float* logits, int V, long ld, const int32_t* targets,
                                                        double* nll) {
  __shared__ double red[kWavesE];
  const long p = blockIdx.x;
  const float* x = logits + p * ld;
  const double l = lse(x, V, red);
  if (threadIdx.x == 0) {
    const int t = targets[p];
    nll[p] = t >= 0 && t < V ? l - static_cast<double>(x[t]) : NAN;
  }
}

}  // namespace

int launch_nll(const float* logits, int V, long ld, const int32_t* targets, int n, double* nll, hipStream_t s) {
  if (n <= 0) return EF_HIP_OK;
  hipLaunchKernelGGL(nll_kernel, dim3(n), dim3(kThreadsE), 0, s, logits, V, ld, targets, nll);
  EFH_HIP(hipGetLastError());
  return EF_HIP_OK;
}

}  // namespace efh

using namespace efh;

extern "C" {

int ef_hip_compare_dist(const float* ref, const float* ours, size_t V, size_t n, size_t ld_ref, size_t ld_ours,
                        double* kl_host, ef_hip_dist_stats* agg, void* stream) {
  EFH_RC(require_ready());
  EFH_CHECK(ref && ours && agg, "compare_dist: null argument");
  EFH_CHECK(V >= 1 && V < 0x7FFFFFFF && ld_ref >= V && ld_ours >= V, "compare_dist: bad vocabulary or stride");
  *agg = ef_hip_dist_stats{};
  if (n == 0) return EF_HIP_OK;
  hipStream_t s = pick(stream);
  double* kl = nullptr;
  int* flags = nullptr;
  EFH_HIP(hipMallocAsync(reinterpret_cast<void**>(&kl), n * sizeof(double), s));
  EFH_HIP(hipMallocAsync(reinterpret_cast<void**>(&flags), n * sizeof(int), s));
  hipLaunchKernelGGL(compare_dist_kernel, dim3(static_cast<unsigned>(n)), dim3(kThreadsE), 0, s, ref, ours,
                     static_cast<int>(V), static_cast<long>(ld_ref), static_cast<long>(ld_ours), kl, flags);
  std::vector<double> k(n);
  std::vector<int> f(n);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(k.data(), kl, n * sizeof(double), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(f.data(), flags, n * sizeof(int), hipMemcpyDeviceToHost, s);
  (void)hipFreeAsync(kl, s);
  (void)hipFreeAsync(flags, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail_hip(e, "compare_dist");
  // DistAgg::add in position order (src/eval_quant.cpp:77-96)
  for (size_t p = 0; p < n; ++p) {
    ++agg->n;
    if (!(f[p] & 1)) {
      ++agg->nonfinite;
      continue;
    }
    const bool top1 = f[p] & 2, conf = f[p] & 4;
    agg->top1 += top1;
    agg->confident += conf;
    agg->confident_top1 += conf && top1;
    agg->kl_sum += k[p];
    agg->kl_max = std::max(agg->kl_max, k[p]);
  }
  agg->kl_mean = agg->n > agg->nonfinite ? agg->kl_sum / static_cast<double>(agg->n - agg->nonfinite) : 0.0;
  if (kl_host) std::copy(k.begin(), k.end(), kl_host);
  return EF_HIP_OK;
}

int ef_hip_neg_log_prob(const float* logits, size_t V, size_t n, size_t ld, const int32_t* targets_dev,
                        double* nll_dev, void* stream) {
  EFH_RC(require_ready());
  EFH_CHECK(logits && targets_dev && nll_dev, "neg_log_prob: null argument");
  EFH_CHECK(V >= 1 && V < 0x7FFFFFFF && ld >= V, "neg_log_prob: bad vocabulary or stride");
  return launch_nll(logits, static_cast<int>(V), static_cast<long>(ld), targets_dev, static_cast<int>(n), nll_dev,
                    pick(stream));
}

}  // extern "C"
