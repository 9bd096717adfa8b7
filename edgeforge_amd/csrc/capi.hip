// C-ABI entry points (include/ef_hip.h): context, memory, weights and the GEMV family.
#include <cstdio>
#include <cstring>
#include <string>

#include <mutex>

#include "codec.h"
#include "common.h"
#include "gemv.h"
#include "sampler.h"

namespace efh {

namespace {
thread_local std::string t_last_error;
Context g_ctx;

// Scratch of the no-allocation sampler entry point (ef_hip_sample_noalloc): a file-scope device
// array, one copy per GPU the library runs on, held until the process ends.  Host code never uses
// the array's name as an address (on the host it is only a stand-in for the symbol): ef_hip_init
// resolves each device's own copy with hipGetSymbolAddress and every later use goes through that
// pointer.
constexpr size_t kScratchBytes = size_t(16) << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxScratchDevices = 64;
void* g_scratch_dev[kMaxScratchDevices] = {};
}  // namespace

void set_error(const std::string& msg) { t_last_error = msg; }
int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}
int fail_hip(hipError_t e, const char* what) {
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return e == hipErrorOutOfMemory ? EF_HIP_ENOMEM : EF_HIP_ERUNTIME;
}

Context& ctx() { return g_ctx; }

int require_ready() {
  if (!g_ctx.ready) return fail(EF_HIP_ESTATE, "ef_hip_init has not been called");
  return EF_HIP_OK;
}

size_t row_bytes_of(int qtype, size_t cols) {  // src/quant.cpp:136-149
  switch (qtype) {
    case EF_QTYPE_F32: return cols * 4;
    case EF_QTYPE_F16:
    case EF_QTYPE_BF16: return cols * 2;
    case EF_QTYPE_Q8_0: return cols % 32 ? 0 : cols / 32 * 34;
    case EF_QTYPE_Q4_0: return cols % 32 ? 0 : cols / 32 * 18;
    default: return 0;
  }
}

int check_weight(ef_hip_weight w) {
  if (w == nullptr) return fail(EF_HIP_EINVAL, "null weight handle");
  if (w->magic != kWeightMagic) return fail(EF_HIP_ESTATE, "weight handle was released or is not a weight");
  return EF_HIP_OK;
}

}  // namespace efh

using namespace efh;

#define EFH_READY()                         \
  do {                                      \
    int efh_rc_ = require_ready();          \
    if (efh_rc_ != EF_HIP_OK) return efh_rc_; \
  } while (0)


extern "C" {

int ef_hip_init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(EF_HIP_ENODEV, "no HIP device is visible");
  if (device < 0 || device >= n) return fail(EF_HIP_ENODEV, "device index out of range");
  if (g_ctx.ready) {
    if (g_ctx.device == device) return EF_HIP_OK;
    return fail(EF_HIP_ESTATE, "the library is already initialised on another device");
  }
  hipDeviceProp_t prop;
  EFH_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return fail(EF_HIP_ENODEV, std::string("this build targets gfx950 (MI355X); device is ") + prop.gcnArchName);
  }
  EFH_HIP(hipSetDevice(device));
  if (device < kMaxScratchDevices && g_scratch_dev[device] == nullptr) {  // once per device, device current
    void* p = nullptr;
    EFH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_dev[device] = p;
  }
  EFH_HIP(hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking));
  g_ctx.device = device;
  g_ctx.cu_count = prop.multiProcessorCount;
  g_ctx.lds_per_block = prop.sharedMemPerBlock;
  std::snprintf(g_ctx.name, sizeof g_ctx.name, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
  g_ctx.ready = true;
  return EF_HIP_OK;
}

int ef_hip_shutdown(void) {
  if (!g_ctx.ready) return EF_HIP_OK;
  EFH_HIP(hipStreamSynchronize(g_ctx.stream));
  EFH_HIP(hipStreamDestroy(g_ctx.stream));
  g_ctx = Context{};
  return EF_HIP_OK;
}

const char* ef_hip_last_error(void) { return t_last_error.c_str(); }

int ef_hip_device_name(char* buf, size_t cap) {
  EFH_READY();
  EFH_CHECK(buf && cap > 0, "device_name: null buffer");
  std::snprintf(buf, cap, "%s", g_ctx.name);
  return EF_HIP_OK;
}

int ef_hip_version(int* major, int* minor) {
  if (major) *major = 0;
  if (minor) *minor = 1;
  return EF_HIP_OK;
}

// ---- memory / streams / events --------------------------------------------------------------------
int ef_hip_malloc(void** dev, size_t bytes) {
  EFH_READY();
  EFH_CHECK(dev != nullptr, "malloc: null out pointer");
  *dev = nullptr;
  if (bytes == 0) return EF_HIP_OK;
  EFH_HIP(hipMalloc(dev, bytes));
  return EF_HIP_OK;
}

int ef_hip_free(void* dev) {
  EFH_READY();
  if (dev) EFH_HIP(hipFree(dev));
  return EF_HIP_OK;
}

int ef_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  EFH_READY();
  if (bytes == 0) return EF_HIP_OK;
  EFH_CHECK(dst && src, "memcpy_h2d: null pointer");
  hipStream_t s = pick(stream);
  EFH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
  EFH_HIP(hipStreamSynchronize(s));
  return EF_HIP_OK;
}

int ef_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  EFH_READY();
  if (bytes == 0) return EF_HIP_OK;
  EFH_CHECK(dst && src, "memcpy_d2h: null pointer");
  hipStream_t s = pick(stream);
  EFH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
  EFH_HIP(hipStreamSynchronize(s));
  return EF_HIP_OK;
}

int ef_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  EFH_READY();
  if (bytes == 0) return EF_HIP_OK;
  EFH_CHECK(dst && src, "memcpy_d2d: null pointer");
  EFH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, pick(stream)));
  return EF_HIP_OK;
}

int ef_hip_memset(void* dev, int value, size_t bytes, void* stream) {
  EFH_READY();
  if (bytes == 0) return EF_HIP_OK;
  EFH_CHECK(dev != nullptr, "memset: null pointer");
  EFH_HIP(hipMemsetAsync(dev, value, bytes, pick(stream)));
  return EF_HIP_OK;
}

int ef_hip_stream_create(void** stream) {
  EFH_READY();
  EFH_CHECK(stream != nullptr, "stream_create: null out pointer");
  hipStream_t s;
  EFH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return EF_HIP_OK;
}

int ef_hip_stream_destroy(void* stream) {
  EFH_READY();
  if (stream) EFH_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return EF_HIP_OK;
}

int ef_hip_stream_sync(void* stream) {
  EFH_READY();
  EFH_HIP(hipStreamSynchronize(pick(stream)));
  return EF_HIP_OK;
}

int ef_hip_pointer_kind(const void* p, int* kind) {
  EFH_READY();
  EFH_CHECK(kind != nullptr, "pointer_kind: null out pointer");
  *kind = 0;
  if (p == nullptr) return EF_HIP_OK;
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();  // unregistered host memory: not an error for this query
    return EF_HIP_OK;
  }
  if (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged) *kind = 1;
  else if (a.type == hipMemoryTypeHost) *kind = 2;
  return EF_HIP_OK;
}

int ef_hip_event_create(void** ev) {
  EFH_READY();
  EFH_CHECK(ev != nullptr, "event_create: null out pointer");
  hipEvent_t e;
  EFH_HIP(hipEventCreate(&e));
  *ev = e;
  return EF_HIP_OK;
}

int ef_hip_event_destroy(void* ev) {
  EFH_READY();
  if (ev) EFH_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return EF_HIP_OK;
}

int ef_hip_event_record(void* ev, void* stream) {
  EFH_READY();
  EFH_CHECK(ev != nullptr, "event_record: null event");
  EFH_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), pick(stream)));
  return EF_HIP_OK;
}

int ef_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  EFH_READY();
  EFH_CHECK(start && stop && ms, "event_elapsed_ms: null argument");
  EFH_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  EFH_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return EF_HIP_OK;
}

// ---- weights ----------------------------------------------------------------------------------------
int ef_hip_row_bytes(int qtype, size_t cols, size_t* out) {
  EFH_CHECK(out != nullptr, "row_bytes: null out pointer");
  const size_t rb = row_bytes_of(qtype, cols);
  if (rb == 0) {
    return fail(EF_HIP_EINVAL, (qtype == EF_QTYPE_Q4_0 || qtype == EF_QTYPE_Q8_0)
                                   ? "block types need a row length divisible by 32, got " + std::to_string(cols)
                                   : "unknown storage type or zero cols");
  }
  *out = rb;
  return EF_HIP_OK;
}

static int make_weight(const void* dev, int qtype, size_t rows, size_t cols, bool owned, ef_hip_weight* out) {
  auto* w = new ef_hip_weight_s;
  w->qtype = qtype;
  w->rows = rows;
  w->cols = cols;
  w->row_bytes = row_bytes_of(qtype, cols);
  w->dev = static_cast<const uint8_t*>(dev);
  w->owned = owned;
  w->magic = kWeightMagic;
  *out = w;
  return EF_HIP_OK;
}

int ef_hip_weight_register_host(const void* host, int qtype, size_t rows, size_t cols, ef_hip_weight* out) {
  EFH_READY();
  EFH_CHECK(host && out, "weight_register_host: null argument");
  size_t rb = 0;
  EFH_RC(ef_hip_row_bytes(qtype, cols, &rb));
  EFH_CHECK(rows > 0, "weight_register_host: rows must be > 0");
  void* dev = nullptr;
  const size_t bytes = rb * rows;
  EFH_HIP(hipMalloc(&dev, bytes));
  hipError_t e = hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, g_ctx.stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_ctx.stream);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return fail_hip(e, "weight upload");
  }
  return make_weight(dev, qtype, rows, cols, true, out);
}

int ef_hip_weight_register_device(const void* dev, int qtype, size_t rows, size_t cols, ef_hip_weight* out) {
  EFH_READY();
  EFH_CHECK(dev && out, "weight_register_device: null argument");
  size_t rb = 0;
  EFH_RC(ef_hip_row_bytes(qtype, cols, &rb));
  EFH_CHECK(rows > 0, "weight_register_device: rows must be > 0");
  return make_weight(dev, qtype, rows, cols, false, out);
}

int ef_hip_weight_release(ef_hip_weight w) {
  EFH_READY();
  EFH_RC(check_weight(w));
  w->magic = 0;
  if (w->owned || w->tiled != nullptr) EFH_HIP(hipStreamSynchronize(g_ctx.stream));
  if (w->owned) EFH_HIP(hipFree(const_cast<uint8_t*>(w->dev)));
  if (w->tiled != nullptr) EFH_HIP(hipFree(w->tiled));
  delete w;
  return EF_HIP_OK;
}

int ef_hip_weight_refresh(ef_hip_weight w, void* stream) {
  EFH_READY();
  EFH_RC(check_weight(w));
  return refresh_tiled(w, pick(stream));
}

int ef_hip_weight_info(ef_hip_weight w, int* qtype, size_t* rows, size_t* cols, const void** dev) {
  EFH_RC(check_weight(w));
  if (qtype) *qtype = w->qtype;
  if (rows) *rows = w->rows;
  if (cols) *cols = w->cols;
  if (dev) *dev = w->dev;
  return EF_HIP_OK;
}

// ---- GEMV ---------------------------------------------------------------------------------------------
int ef_hip_matvec(ef_hip_weight W, const float* x, float* y, int batch, size_t ldx, size_t ldy, void* stream) {
  EFH_READY();
  EFH_RC(check_weight(W));
  const GemvJob j{W, nullptr, x, y};
  return launch_gemv(&j, 1, kEpiStore, nullptr, 0.0f, batch, ldx, ldy, pick(stream));
}

static int jobs_common(const ef_hip_job* jobs, size_t n_jobs, int epi, const float* norm_w, float eps, int batch,
                       size_t ldx, size_t ldy, void* stream) {
  EFH_READY();
  EFH_CHECK(jobs != nullptr && n_jobs > 0, "matvec_jobs: no jobs");
  // Jobs are launched in groups of up to 4 that share cols (one launch per group).
  size_t i = 0;
  while (i < n_jobs) {
    GemvJob g[4];
    int n = 0;
    EFH_RC(check_weight(jobs[i].W));
    const size_t cols = jobs[i].W->cols;
    while (i < n_jobs && n < 4) {
      EFH_RC(check_weight(jobs[i].W));
      if (jobs[i].W->cols != cols) break;
      g[n++] = GemvJob{jobs[i].W, nullptr, jobs[i].x_dev, jobs[i].y_dev};
      ++i;
    }
    EFH_RC(launch_gemv(g, n, epi, norm_w, eps, batch, ldx, ldy, pick(stream)));
  }
  return EF_HIP_OK;
}

int ef_hip_matvec_jobs(const ef_hip_job* jobs, size_t n_jobs, int batch, size_t ldx, size_t ldy, void* stream) {
  return jobs_common(jobs, n_jobs, kEpiStore, nullptr, 0.0f, batch, ldx, ldy, stream);
}

int ef_hip_matvec_jobs_rmsnorm(const ef_hip_job* jobs, size_t n_jobs, const float* norm_w, float eps, int batch,
                               size_t ldx, size_t ldy, void* stream) {
  return jobs_common(jobs, n_jobs, kEpiStore, norm_w, eps, batch, ldx, ldy, stream);
}

int ef_hip_matvec_residual(ef_hip_weight W, const float* x, float* y, int batch, size_t ldx, size_t ldy,
                           void* stream) {
  EFH_READY();
  EFH_RC(check_weight(W));
  const GemvJob j{W, nullptr, x, y};
  return launch_gemv(&j, 1, kEpiResidual, nullptr, 0.0f, batch, ldx, ldy, pick(stream));
}

int ef_hip_matvec_swiglu(ef_hip_weight G, ef_hip_weight U, const float* x, const float* norm_w, float eps, float* y,
                         int batch, size_t ldx, size_t ldy, void* stream) {
  EFH_READY();
  EFH_RC(check_weight(G));
  EFH_RC(check_weight(U));
  const GemvJob j{G, U, x, y};
  return launch_gemv(&j, 1, kEpiSwiglu, norm_w, eps, batch, ldx, ldy, pick(stream));
}

int ef_hip_profile_matvec(int epi, const ef_hip_weight* W, const ef_hip_weight* W2, size_t n_weights,
                          const float* x, const float* norm_w, float eps, float* y, int batch, int launches,
                          void* stream, float* avg_ms) {
  EFH_READY();
  EFH_CHECK(W && n_weights > 0 && x && y && avg_ms && launches > 0, "profile_matvec: bad argument");
  EFH_CHECK(epi >= kEpiStore && epi <= kEpiSwiglu, "profile_matvec: unknown epilogue");
  EFH_CHECK(epi != kEpiSwiglu || W2 != nullptr, "profile_matvec: swiglu needs the up matrices");
  for (size_t i = 0; i < n_weights; ++i) {
    EFH_RC(check_weight(W[i]));
    if (W2) EFH_RC(check_weight(W2[i]));
  }
  hipStream_t s = pick(stream);
  hipEvent_t e0, e1;
  EFH_HIP(hipEventCreate(&e0));
  EFH_HIP(hipEventCreate(&e1));
  int rc = EF_HIP_OK;
  const size_t ldx = W[0]->cols, ldy = W[0]->rows;
  // batched launches get their activation workspace and the matrices' tile-order copies up front,
  // as the decode engine does
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (batch > 1) {
    for (size_t i = 0; i < n_weights; ++i) {
      for (const ef_hip_weight_s* w : {W[i], W2 ? W2[i] : nullptr}) {
        if (w != nullptr && (w->qtype == EF_QTYPE_Q4_0 || w->qtype == EF_QTYPE_Q8_0) && w->cols % 32 == 0)
          EFH_RC(ensure_tiled(w, s));
      }
    }
    const GemvJob j0{W[0], epi == kEpiSwiglu ? W2[0] : nullptr, x, y};
    ws_bytes = gemv_mfma_workspace_bytes(&j0, 1, epi, batch, ldx);
    if (ws_bytes > 0) EFH_HIP(hipMalloc(&ws, ws_bytes));
  }
  // the launches run as one captured HIP graph (as the decode engine runs its steps), so the time
  // is the device's, not the host's launch rate
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipError_t he = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (he == hipSuccess) {
    for (int i = 0; i < launches && rc == EF_HIP_OK; ++i) {
      const size_t k = static_cast<size_t>(i) % n_weights;
      const GemvJob j{W[k], epi == kEpiSwiglu ? W2[k] : nullptr, x, y};
      rc = launch_gemv(&j, 1, epi, norm_w, eps, batch, ldx, ldy, s, ws, ws_bytes);
    }
    he = hipStreamEndCapture(s, &graph);
  }
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  float ms = 0.0f;
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipEventRecord(e0, s);
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipGraphLaunch(exec, s);
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipEventRecord(e1, s);
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipEventSynchronize(e1);
  if (he == hipSuccess && rc == EF_HIP_OK) he = hipEventElapsedTime(&ms, e0, e1);
  if (exec != nullptr) (void)hipGraphExecDestroy(exec);
  if (graph != nullptr) (void)hipGraphDestroy(graph);
  if (ws != nullptr) (void)hipFree(ws);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc != EF_HIP_OK) return rc;
  if (he != hipSuccess) return fail_hip(he, "profile_matvec: graph capture / launch");
  *avg_ms = ms / static_cast<float>(launches);
  return EF_HIP_OK;
}

// ---- codec / row lookup ---------------------------------------------------------------------------
int ef_hip_quantize(int qtype, const float* w, size_t rows, size_t cols, int search, void* out, void* stream) {
  EFH_READY();
  EFH_CHECK(w && out, "quantize: null pointer");
  EFH_CHECK(rows > 0, "quantize: rows must be > 0");
  size_t rb = 0;
  EFH_RC(ef_hip_row_bytes(qtype, cols, &rb));
  return launch_quantize(qtype, w, rows, cols, search, out, pick(stream));
}

int ef_hip_fill_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float mean, float scale, void* stream) {
  EFH_READY();
  EFH_CHECK(out != nullptr || n == 0, "fill_normal: null pointer");
  if (n == 0) return EF_HIP_OK;
  return launch_fill_normal(out, n, seed, offset, mean, scale, pick(stream));
}

int ef_hip_rows_f32(ef_hip_weight W, const int32_t* ids, int batch, float* out, size_t ldo, void* stream) {
  EFH_READY();
  EFH_RC(check_weight(W));
  EFH_CHECK(ids && out, "rows_f32: null pointer");
  EFH_CHECK(batch >= 1 && batch <= 65535, "rows_f32: batch must be in [1, 65535]");
  EFH_CHECK(batch == 1 || ldo >= W->cols, "rows_f32: ldo smaller than cols");
  return launch_rows_f32(W, ids, batch, out, ldo, pick(stream));
}

// ---- selection ------------------------------------------------------------------------------------------
int ef_hip_argmax(const float* x, size_t n, int batch, size_t ld, int32_t* out, void* stream) {
  EFH_READY();
  EFH_CHECK(x && out, "argmax: null pointer");
  EFH_CHECK(n > 0 && n <= 0x7FFFFFFF, "argmax: n must be in [1, 2^31)");
  EFH_CHECK(batch >= 1 && batch <= 65535 && (batch == 1 || ld >= n), "argmax: bad batch / ld");
  return launch_argmax(x, static_cast<int>(n), static_cast<long>(ld), batch, out, pick(stream));
}

int ef_hip_sampler_exp(const double* x, double* y, size_t n, void* stream) {
  EFH_READY();
  EFH_CHECK(n == 0 || (x && y), "sampler_exp: null pointer");
  return launch_exp(x, y, n, pick(stream));
}

size_t ef_hip_rng_state_bytes(void) { return kRngStateBytes; }

int ef_hip_rng_seed(void* rng, const uint64_t* seeds_host, int batch, void* stream) {
  EFH_READY();
  EFH_CHECK(rng && seeds_host, "rng_seed: null pointer");
  EFH_CHECK(batch >= 1 && batch <= 65535, "rng_seed: batch must be in [1, 65535]");
  hipStream_t s = pick(stream);
  void* seeds = nullptr;
  EFH_HIP(hipMallocAsync(&seeds, sizeof(uint64_t) * batch, s));
  EFH_HIP(hipMemcpyAsync(seeds, seeds_host, sizeof(uint64_t) * batch, hipMemcpyHostToDevice, s));
  int rc = launch_rng_seed(rng, static_cast<const uint64_t*>(seeds), batch, s);
  EFH_HIP(hipFreeAsync(seeds, s));
  if (rc == EF_HIP_OK) EFH_HIP(hipStreamSynchronize(s));
  return rc;
}

size_t ef_hip_sample_workspace_bytes(size_t vocab, int batch) {
  if (vocab == 0 || vocab > (1u << 24) || batch < 1) return 0;
  return sample_workspace_stride(static_cast<int>(vocab)) * static_cast<size_t>(batch);
}

namespace {
std::mutex g_ws_mu;
void* g_ws = nullptr;
size_t g_ws_bytes = 0;
}  // namespace

namespace {
int check_sample_args(const float* logits, size_t vocab, int batch, size_t ld, const ef_hip_sampler_config* cfg,
                      const int32_t* hist, const int32_t* hist_len, void* rng, int32_t* out) {
  EFH_CHECK(logits && cfg && out, "sample: null pointer");
  if (vocab == 0) return fail(EF_HIP_EINVAL, "sampler: empty vocabulary");  // src/sampler.cpp:14
  EFH_CHECK(vocab <= (1u << 24), "sample: vocab above 2^24");
  EFH_CHECK(batch >= 1 && batch <= 65535 && (batch == 1 || ld >= vocab), "sample: bad batch / ld");
  EFH_CHECK(cfg->temperature <= 0.0f || rng != nullptr, "sample: temperature > 0 needs an rng state");
  EFH_CHECK(cfg->repetition_penalty == 1.0f || (hist && hist_len), "sample: penalty needs a history");
  return EF_HIP_OK;
}
}  // namespace

int ef_hip_sample(const float* logits, size_t vocab, int batch, size_t ld, const ef_hip_sampler_config* cfg,
                  const int32_t* hist, const int32_t* hist_len, size_t hist_ld, void* rng, int32_t* out, void* ws,
                  void* stream) {
  EFH_READY();
  EFH_RC(check_sample_args(logits, vocab, batch, ld, cfg, hist, hist_len, rng, out));
  hipStream_t s = pick(stream);
  if (ws == nullptr) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    const size_t need = ef_hip_sample_workspace_bytes(vocab, batch);
    if (need > g_ws_bytes) {
      EFH_HIP(hipDeviceSynchronize());
      if (g_ws) EFH_HIP(hipFree(g_ws));
      g_ws = nullptr;
      g_ws_bytes = 0;
      EFH_HIP(hipMalloc(&g_ws, need));
      g_ws_bytes = need;
    }
    ws = g_ws;
  }
  return launch_sample(logits, static_cast<int>(vocab), batch, static_cast<long>(ld), *cfg, hist, hist_len,
                       static_cast<long>(hist_ld), rng, out, ws, s);
}

// ef_hip_sample over the library's fixed device scratch: no allocation of any kind.  The kernels
// write every workspace word they later read, so the scratch needs no clearing between calls.
int ef_hip_sample_noalloc(const float* logits, size_t vocab, int batch, size_t ld, const ef_hip_sampler_config* cfg,
                          const int32_t* hist, const int32_t* hist_len, size_t hist_ld, void* rng, int32_t* out,
                          void* stream) {
  EFH_READY();
  EFH_RC(check_sample_args(logits, vocab, batch, ld, cfg, hist, hist_len, rng, out));
  const size_t need = ef_hip_sample_workspace_bytes(vocab, batch);
  if (need > kScratchBytes) {
    const size_t per = ef_hip_sample_workspace_bytes(vocab, 1);
    return fail(EF_HIP_EINVAL, "sample_noalloc: " + std::to_string(batch) + " sequences of vocab " +
                                   std::to_string(vocab) + " need " + std::to_string(need) +
                                   " bytes of scratch, above the fixed " + std::to_string(kScratchBytes) +
                                   " (at most " + std::to_string(kScratchBytes / per) +
                                   " sequences of this vocab); use ef_hip_sample with a workspace");
  }
  void* ws = g_ctx.device < kMaxScratchDevices ? g_scratch_dev[g_ctx.device] : nullptr;
  EFH_CHECK(ws != nullptr, "sample_noalloc: no scratch on this device (device index above 63)");
  return launch_sample(logits, static_cast<int>(vocab), batch, static_cast<long>(ld), *cfg, hist, hist_len,
                       static_cast<long>(hist_ld), rng, out, ws, pick(stream));
}

}  // extern "C"
