// ef::hip: EdgeForge's kernel and sampler signatures over the C-ABI of libedgeforge_hip.so.
#include "ef_hip_kern.hpp"

#include <map>
#include <mutex>
#include <tuple>

#include "../../include/ef_hip.h"

namespace ef {

#if defined(EF_HIP_STANDALONE) || !__has_include("ef/qkernels.h")
std::size_t WeightView::row_bytes() const {  // src/quant.cpp:136-149
  switch (type) {
    case QType::F32: return cols * 4;
    case QType::F16:
    case QType::BF16: return cols * 2;
    case QType::Q8_0:
      if (cols % 32) throw Error("Q8_0 needs a row length divisible by 32, got " + std::to_string(cols));
      return cols / 32 * 34;
    case QType::Q4_0:
      if (cols % 32) throw Error("Q4_0 needs a row length divisible by 32, got " + std::to_string(cols));
      return cols / 32 * 18;
  }
  return 0;
}
#endif

namespace hip {
namespace {

std::mutex g_mu;
bool g_ready = false;
std::string g_error;  // first failure of a noexcept entry point

struct Scratch {
  void* p = nullptr;
  std::size_t bytes = 0;
};
Scratch g_x, g_y, g_ids;

using Key = std::tuple<const std::uint8_t*, int, std::size_t, std::size_t>;
std::map<Key, ef_hip_weight> g_weights;

std::string msg(const char* what) { return std::string(what) + ": " + ef_hip_last_error(); }

void record(const std::string& m) {
  if (g_error.empty()) g_error = m;
}

bool ensure_ready_locked() {
  if (g_ready) return true;
  if (ef_hip_init(0) != EF_HIP_OK) {
    record(msg("ef_hip_init"));
    return false;
  }
  g_ready = true;
  return true;
}

bool grow(Scratch& s, std::size_t bytes) {
  if (s.bytes >= bytes) return true;
  if (s.p) ef_hip_free(s.p);
  s.p = nullptr;
  s.bytes = 0;
  if (ef_hip_malloc(&s.p, bytes) != EF_HIP_OK) {
    record(msg("device scratch"));
    return false;
  }
  s.bytes = bytes;
  return true;
}

bool is_device(const void* p) {
  int kind = 0;
  return ef_hip_pointer_kind(p, &kind) == EF_HIP_OK && kind == 1;
}

// Device handle of a view's bytes, uploaded on first use.
ef_hip_weight weight_of(const WeightView& W) {
  const Key k{W.data, static_cast<int>(W.type), W.rows, W.cols};
  auto it = g_weights.find(k);
  if (it != g_weights.end()) return it->second;
  ef_hip_weight h = nullptr;
  const int rc = is_device(W.data)
                     ? ef_hip_weight_register_device(W.data, static_cast<int>(W.type), W.rows, W.cols, &h)
                     : ef_hip_weight_register_host(W.data, static_cast<int>(W.type), W.rows, W.cols, &h);
  if (rc != EF_HIP_OK) {
    record(msg("weight upload"));
    return nullptr;
  }
  g_weights.emplace(k, h);
  return h;
}

// Runs a group of same-width jobs with device x / y, staging host pointers.
void run_jobs_locked(const kern::MatvecJob* jobs, std::size_t n) {
  std::vector<ef_hip_job> dj(n);
  std::size_t xfloats = 0, yfloats = 0;
  for (std::size_t j = 0; j < n; ++j) {
    if (!is_device(jobs[j].x)) xfloats += jobs[j].W->cols;
    if (!is_device(jobs[j].y)) yfloats += jobs[j].W->rows;
  }
  if ((xfloats && !grow(g_x, xfloats * 4)) || (yfloats && !grow(g_y, yfloats * 4))) return;
  std::size_t xo = 0, yo = 0;
  for (std::size_t j = 0; j < n; ++j) {
    ef_hip_weight h = weight_of(*jobs[j].W);
    if (!h) return;
    const float* xd = jobs[j].x;
    float* yd = jobs[j].y;
    if (!is_device(xd)) {
      float* s = static_cast<float*>(g_x.p) + xo;
      if (ef_hip_memcpy_h2d(s, jobs[j].x, jobs[j].W->cols * 4, nullptr) != EF_HIP_OK) return record(msg("x upload"));
      xd = s;
      xo += jobs[j].W->cols;
    }
    if (!is_device(yd)) {
      yd = static_cast<float*>(g_y.p) + yo;
      yo += jobs[j].W->rows;
    }
    dj[j] = ef_hip_job{yd, h, xd};
  }
  if (ef_hip_matvec_jobs(dj.data(), n, 1, 0, 0, nullptr) != EF_HIP_OK) return record(msg("ef_hip_matvec_jobs"));
  for (std::size_t j = 0; j < n; ++j) {
    if (!is_device(jobs[j].y)) {
      if (ef_hip_memcpy_d2h(jobs[j].y, dj[j].y_dev, jobs[j].W->rows * 4, nullptr) != EF_HIP_OK)
        return record(msg("y download"));
    }
  }
  if (ef_hip_stream_sync(nullptr) != EF_HIP_OK) record(msg("stream sync"));
}

}  // namespace

void set_device(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) return;
  if (ef_hip_init(device) != EF_HIP_OK) throw Error(msg("ef_hip_init"));
  g_ready = true;
}

bool available() noexcept {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) return true;
  g_ready = ef_hip_init(0) == EF_HIP_OK;
  return g_ready;
}

std::string last_error() {
  std::lock_guard<std::mutex> lk(g_mu);
  return g_error;
}

void clear_error() noexcept {
  std::lock_guard<std::mutex> lk(g_mu);
  g_error.clear();
}

void throw_if_error() {
  std::string e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    e.swap(g_error);
  }
  if (!e.empty()) throw Error(e);
}

void matvec(float* y, const WeightView& W, const float* x, ThreadPool*) noexcept {
  const kern::MatvecJob j{y, &W, x};
  hip::matvec_jobs(&j, 1, nullptr);  // qualified: argument-dependent lookup also finds ef::kern's
}

// kern::matvec_jobs (src/qkernels.cpp:280-297): jobs of equal width share one launch; jobs are
// otherwise independent, so a width change simply starts the next launch.
void matvec_jobs(const kern::MatvecJob* jobs, std::size_t n_jobs, ThreadPool*) noexcept {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!ensure_ready_locked() || n_jobs == 0) return;
  std::size_t i = 0;
  while (i < n_jobs) {
    std::size_t j = i + 1;
    while (j < n_jobs && j - i < 4 && jobs[j].W->cols == jobs[i].W->cols) ++j;
    run_jobs_locked(jobs + i, j - i);
    i = j;
  }
}

void matvec_rows(float* y, const WeightView& W, const float* x, std::size_t begin, std::size_t end) noexcept {
  if (begin >= end) return;
  WeightView sub = W;
  sub.data = W.data + begin * W.row_bytes();
  sub.rows = end - begin;
  matvec(y + begin, sub, x);
}

void matvec_q4_0(float* y, const std::uint8_t* W, const float* x, std::size_t rows, std::size_t cols) noexcept {
  matvec(y, WeightView{QType::Q4_0, W, rows, cols}, x);
}

void matvec_q8_0(float* y, const std::uint8_t* W, const float* x, std::size_t rows, std::size_t cols) noexcept {
  matvec(y, WeightView{QType::Q8_0, W, rows, cols}, x);
}

float dot_q4_0(const std::uint8_t* row, const float* x, std::size_t n) noexcept {
  float y = 0.0f;
  matvec_q4_0(&y, row, x, 1, n);
  return y;
}

float dot_q8_0(const std::uint8_t* row, const float* x, std::size_t n) noexcept {
  float y = 0.0f;
  matvec_q8_0(&y, row, x, 1, n);
  return y;
}

void row_f32(float* out, const WeightView& W, std::size_t r) noexcept {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!ensure_ready_locked()) return;
  ef_hip_weight h = weight_of(W);
  if (!h) return;
  const bool dev_out = is_device(out);
  if (!grow(g_ids, 4) || (!dev_out && !grow(g_y, W.cols * 4))) return;
  const std::int32_t id = static_cast<std::int32_t>(r);
  if (ef_hip_memcpy_h2d(g_ids.p, &id, 4, nullptr) != EF_HIP_OK) return record(msg("id upload"));
  float* o = dev_out ? out : static_cast<float*>(g_y.p);
  if (ef_hip_rows_f32(h, static_cast<const std::int32_t*>(g_ids.p), 1, o, W.cols, nullptr) != EF_HIP_OK)
    return record(msg("ef_hip_rows_f32"));
  if (!dev_out && ef_hip_memcpy_d2h(out, o, W.cols * 4, nullptr) != EF_HIP_OK) return record(msg("row download"));
  if (ef_hip_stream_sync(nullptr) != EF_HIP_OK) record(msg("stream sync"));
}

std::size_t argmax(const float* x, std::size_t n) noexcept {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!ensure_ready_locked() || n == 0) return 0;
  const float* xd = x;
  if (!is_device(x)) {
    if (!grow(g_x, n * 4)) return 0;
    if (ef_hip_memcpy_h2d(g_x.p, x, n * 4, nullptr) != EF_HIP_OK) {
      record(msg("argmax upload"));
      return 0;
    }
    xd = static_cast<const float*>(g_x.p);
  }
  if (!grow(g_ids, 4)) return 0;
  std::int32_t r = 0;
  if (ef_hip_argmax(xd, n, 1, n, static_cast<std::int32_t*>(g_ids.p), nullptr) != EF_HIP_OK ||
      ef_hip_memcpy_d2h(&r, g_ids.p, 4, nullptr) != EF_HIP_OK) {
    record(msg("ef_hip_argmax"));
    return 0;
  }
  return static_cast<std::size_t>(r);
}

float* device_alloc(std::size_t floats) {
  set_device(0);
  void* p = nullptr;
  if (ef_hip_malloc(&p, floats * sizeof(float)) != EF_HIP_OK) throw Error(msg("ef_hip_malloc"));
  return static_cast<float*>(p);
}

void device_free(void* p) noexcept {
  if (p) ef_hip_free(p);
}

void upload(float* dev, const float* host, std::size_t floats) {
  if (ef_hip_memcpy_h2d(dev, host, floats * 4, nullptr) != EF_HIP_OK) throw Error(msg("upload"));
}

void download(float* host, const float* dev, std::size_t floats) {
  if (ef_hip_memcpy_d2h(host, dev, floats * 4, nullptr) != EF_HIP_OK) throw Error(msg("download"));
}

// ---- Sampler ------------------------------------------------------------------------------------------
Sampler::Sampler(const SamplerConfig& cfg) : cfg_(cfg) {
  set_device(0);
  void* out = nullptr;
  if (ef_hip_malloc(&rng_, ef_hip_rng_state_bytes()) != EF_HIP_OK || ef_hip_malloc(&out, 16) != EF_HIP_OK)
    throw Error(msg("sampler state"));
  out_ = static_cast<std::int32_t*>(out);
  const std::uint64_t seed = cfg.seed;  // std::mt19937_64 rng_(cfg.seed) (include/ef/sampler.h:23)
  if (ef_hip_rng_seed(rng_, &seed, 1, nullptr) != EF_HIP_OK) throw Error(msg("sampler seed"));
}

Sampler::~Sampler() {
  ef_hip_free(rng_);
  ef_hip_free(ws_);
  ef_hip_free(logits_);
  ef_hip_free(hist_);
  ef_hip_free(out_);
}

std::int32_t Sampler::sample(const float* logits, std::size_t vocab, const std::vector<std::int32_t>& history) {
  if (vocab == 0) throw Error("sampler: empty vocabulary");  // src/sampler.cpp:14
  if (ws_vocab_ < vocab) {
    ef_hip_free(ws_);
    ws_ = nullptr;
    if (ef_hip_malloc(&ws_, ef_hip_sample_workspace_bytes(vocab, 1)) != EF_HIP_OK) throw Error(msg("sampler workspace"));
    ws_vocab_ = vocab;
  }
  const float* ld = logits;
  if (!is_device(logits)) {
    if (logits_cap_ < vocab) {
      ef_hip_free(logits_);
      void* p = nullptr;
      if (ef_hip_malloc(&p, vocab * 4) != EF_HIP_OK) throw Error(msg("sampler logits"));
      logits_ = static_cast<float*>(p);
      logits_cap_ = vocab;
    }
    if (ef_hip_memcpy_h2d(logits_, logits, vocab * 4, nullptr) != EF_HIP_OK) throw Error(msg("logits upload"));
    ld = logits_;
  }
  const std::size_t nh = history.size();
  if (hist_cap_ < nh + 1) {
    ef_hip_free(hist_);
    void* p = nullptr;
    if (ef_hip_malloc(&p, (nh + 1) * 4) != EF_HIP_OK) throw Error(msg("sampler history"));
    hist_ = static_cast<std::int32_t*>(p);
    hist_cap_ = nh + 1;
  }
  if (nh && ef_hip_memcpy_h2d(hist_, history.data(), nh * 4, nullptr) != EF_HIP_OK) throw Error(msg("history upload"));
  const std::int32_t len = static_cast<std::int32_t>(nh);
  if (ef_hip_memcpy_h2d(out_ + 1, &len, 4, nullptr) != EF_HIP_OK) throw Error(msg("history length"));
  const ef_hip_sampler_config c{cfg_.temperature, cfg_.top_k, cfg_.top_p, cfg_.repetition_penalty, cfg_.seed};
  if (ef_hip_sample(ld, vocab, 1, vocab, &c, hist_, out_ + 1, nh ? nh : 1, rng_, out_, ws_, nullptr) != EF_HIP_OK)
    throw Error(msg("ef_hip_sample"));
  std::int32_t tok = 0;
  if (ef_hip_memcpy_d2h(&tok, out_, 4, nullptr) != EF_HIP_OK) throw Error(msg("token download"));
  return tok;
}

}  // namespace hip
}  // namespace ef
