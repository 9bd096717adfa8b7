// C entry points over the EdgeForge reference sources, compiled from where they lie under
// /root/reference into oracle/_ref/libefref.so (see oracle/Makefile, target `ref`).
//
// TEST INFRASTRUCTURE ONLY: this file wraps the reference's own functions so the tests can pin
// the plain-C oracle (oracle/*.c) against them bit for bit.  It contains no copy of reference
// code; every function forwards to the reference symbol named in its comment.  Errors the
// reference throws (ef::Error) become a -1 return.
#include <cstdint>
#include <cstring>
#include <memory>
#include <random>
#include <vector>

#include "ef/error.h"
#include "ef/fp16.h"
#include "ef/kernels.h"
#include "ef/model.h"
#include "ef/qkernels.h"
#include "ef/quant.h"
#include "ef/sampler.h"
#include "ef/threadpool.h"

using namespace ef;

namespace {
QType qt(int t) { return static_cast<QType>(t); }  // same enum order as include/ef/quant.h:35
}  // namespace

extern "C" {

float ref_fp16_to_f32(std::uint16_t h) { return fp16_to_f32(h); }          // include/ef/fp16.h:44
std::uint16_t ref_f32_to_fp16(float f) { return f32_to_fp16(f); }          // include/ef/fp16.h:69
float ref_bf16_to_f32(std::uint16_t h) { return bf16_to_f32(h); }          // include/ef/fp16.h:28
std::uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16(f); }          // include/ef/fp16.h:32

int ref_row_bytes(int t, std::uint64_t cols, std::uint64_t* out) {          // src/quant.cpp:136
  try {
    *out = qtype_row_bytes(qt(t), cols);
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

int ref_quantize_row(int t, const float* x, std::size_t n, void* out, int search) {  // src/quant.cpp:182
  try {
    quantize_row(qt(t), x, n, out, search != 0);
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

int ref_dequantize_row(int t, const void* in, std::size_t n, float* out) {  // src/quant.cpp:219
  try {
    dequantize_row(qt(t), in, n, out);
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

void ref_fake_quant_q4_group(const float* x, std::size_t n, float* out, int search) {  // src/quant.cpp:251
  fake_quant_q4_group(x, n, out, search != 0);
}

float ref_dot_q4_0(const std::uint8_t* r, const float* x, std::size_t n) { return kern::dot_q4_0(r, x, n); }
float ref_dot_q8_0(const std::uint8_t* r, const float* x, std::size_t n) { return kern::dot_q8_0(r, x, n); }
#if defined(EF_HAVE_AVX2)
float ref_dot_q4_0_avx2(const std::uint8_t* r, const float* x, std::size_t n) { return kern::dot_q4_0_avx2(r, x, n); }
float ref_dot_q8_0_avx2(const std::uint8_t* r, const float* x, std::size_t n) { return kern::dot_q8_0_avx2(r, x, n); }
#endif
int ref_avx2_compiled() { return kern::avx2_compiled() ? 1 : 0; }

// y = W x for several jobs with backend 0 = scalar, 1 = avx2, over `threads` threads
// (src/qkernels.cpp:280 matvec_jobs; src/threadpool.cpp).
int ref_matvec_jobs(int backend, int n_jobs, float* const* ys, const int* types, const std::uint8_t* const* data,
                    const std::size_t* rows, const std::size_t* cols, const float* const* xs, unsigned threads) {
  try {
    kern::set_backend(backend == 1 ? kern::Backend::Avx2 : kern::Backend::Scalar);
    std::vector<WeightView> views(static_cast<std::size_t>(n_jobs));
    std::vector<kern::MatvecJob> jobs(static_cast<std::size_t>(n_jobs));
    for (int j = 0; j < n_jobs; ++j) {
      views[j] = WeightView{qt(types[j]), data[j], rows[j], cols[j]};
      jobs[j] = kern::MatvecJob{ys[j], &views[j], xs[j]};
    }
    std::unique_ptr<ThreadPool> pool = threads > 1 ? std::make_unique<ThreadPool>(threads) : nullptr;
    kern::matvec_jobs(jobs.data(), jobs.size(), pool.get());
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

// ---- sampler (include/ef/sampler.h:13-35, src/sampler.cpp:13-70)
void* ref_sampler_create(float temperature, int top_k, float top_p, float rep, std::uint64_t seed) {
  SamplerConfig c;
  c.temperature = temperature;
  c.top_k = top_k;
  c.top_p = top_p;
  c.repetition_penalty = rep;
  c.seed = seed;
  return new Sampler(c);
}
void ref_sampler_destroy(void* s) { delete static_cast<Sampler*>(s); }
int ref_sampler_sample(void* s, const float* logits, std::size_t vocab, const std::int32_t* hist, std::size_t n_hist,
                       std::int32_t* out) {
  try {
    const std::vector<std::int32_t> h(hist, hist + n_hist);
    *out = static_cast<Sampler*>(s)->sample(logits, vocab, h);
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

// The library calls the sampler draws from: std::mt19937_64 words and the uniform double.
void ref_mt64_words(std::uint64_t seed, std::size_t n, std::uint64_t* out) {
  std::mt19937_64 g(seed);
  for (std::size_t i = 0; i < n; ++i) out[i] = g();
}
void ref_uniform_doubles(std::uint64_t seed, std::size_t n, double* out) {
  std::mt19937_64 g(seed);
  std::uniform_real_distribution<double> u(0.0, 1.0);
  for (std::size_t i = 0; i < n; ++i) out[i] = u(g);
}

// ---- FP32 glue (src/kernels.cpp)
void ref_rmsnorm(float* o, const float* x, const float* w, std::size_t n, float eps) { kern::rmsnorm(o, x, w, n, eps); }
void ref_softmax(float* x, std::size_t n) { kern::softmax_inplace(x, n); }
float ref_silu(float x) { return kern::silu(x); }
void ref_swiglu(float* o, const float* g, const float* u, std::size_t n) { kern::swiglu(o, g, u, n); }
std::size_t ref_argmax(const float* x, std::size_t n) { return kern::argmax(x, n); }
float ref_dot_f32(const float* a, const float* b, std::size_t n) { return kern::dot_f32(a, b, n); }
void ref_rope_table(float* inv_freq, float* cos_t, float* sin_t, std::size_t max_pos, std::size_t hd, float theta) {
  const kern::RopeTable t(max_pos, hd, theta);
  std::memcpy(inv_freq, t.inv_freq(), hd / 2 * sizeof(float));
  for (std::size_t p = 0; p < max_pos; ++p) {
    std::memcpy(cos_t + p * (hd / 2), t.cos_row(p), hd / 2 * sizeof(float));
    std::memcpy(sin_t + p * (hd / 2), t.sin_row(p), hd / 2 * sizeof(float));
  }
}
void ref_rope_apply(float* x, std::size_t nh, std::size_t hd, const float* c, const float* s) {
  kern::rope_apply(x, nh, hd, c, s);
}
void ref_attention(float* out, const float* q, const float* k, const float* v, std::size_t n_pos, std::size_t H,
                   std::size_t KV, std::size_t hd, float* scores) {
  kern::attention(out, q, k, v, n_pos, H, KV, hd, scores);
}

// ---- engine on an .efq file (src/model.cpp:66-111, 184-276; src/bench_decode.cpp:30-49)
struct RefEngine {
  Model model;
  std::unique_ptr<ThreadPool> pool;
  std::unique_ptr<Transformer> tr;
};

void* ref_engine_open(const char* efq_path, std::size_t max_seq, unsigned threads, int backend) {
  try {
    kern::set_backend(backend == 1 ? kern::Backend::Avx2 : kern::Backend::Scalar);
    auto* e = new RefEngine{Model::load_efq(efq_path), nullptr, nullptr};
    if (threads > 1) e->pool = std::make_unique<ThreadPool>(threads);
    e->tr = std::make_unique<Transformer>(e->model, max_seq, e->pool.get());
    return e;
  } catch (const Error&) {
    return nullptr;
  }
}
void ref_engine_close(void* e) { delete static_cast<RefEngine*>(e); }
std::uint64_t ref_engine_bytes_per_token(void* e) { return static_cast<RefEngine*>(e)->model.weight_bytes_per_token(); }

// Logits [V] into `out` when compute_logits; returns -1 on a rejected token / position.
int ref_engine_forward(void* ve, std::int32_t token, std::size_t pos, int compute_logits, float* out) {
  auto* e = static_cast<RefEngine*>(ve);
  try {
    const float* lg = e->tr->forward(token, pos, compute_logits != 0);
    if (lg != nullptr && out != nullptr) {
      std::memcpy(out, lg, static_cast<std::size_t>(e->model.config().vocab_size) * sizeof(float));
    }
    return 0;
  } catch (const Error&) {
    return -1;
  }
}

// ---- .efq reader (src/qfile.cpp:125-243, src/model.cpp:66-111): accept / reject with the message
namespace {
int put_msg(const std::string& m, char* err, std::size_t cap) {
  if (err != nullptr && cap > 0) {
    const std::size_t n = std::min(m.size(), cap - 1);
    std::memcpy(err, m.data(), n);
    err[n] = '\0';
  }
  return -1;
}
}  // namespace

// parse_efq over a buffer: the tensor count, or -1 with the exception text in err.
long ref_efq_parse(const std::uint8_t* buf, std::size_t n, char* err, std::size_t cap) {
  try {
    return static_cast<long>(parse_efq(buf, n).tensors.size());
  } catch (const Error& e) {
    return put_msg(e.what(), err, cap);
  }
}

// Model::load_efq: bytes per token and the description, or -1 with the message.
long ref_model_load_efq(const char* path, std::uint64_t* bytes_per_token, char* desc, std::size_t cap) {
  try {
    const Model m = Model::load_efq(path);
    if (bytes_per_token) *bytes_per_token = m.weight_bytes_per_token();
    if (desc != nullptr && cap > 0) {
      const std::string& d = m.description();
      const std::size_t k = std::min(d.size(), cap - 1);
      std::memcpy(desc, d.data(), k);
      desc[k] = '\0';
    }
    return 0;
  } catch (const Error& e) {
    return put_msg(e.what(), desc, cap);
  }
}

}  // extern "C"
