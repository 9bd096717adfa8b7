// .efq files on the device: the C-ABI over the host reader (efq.hip) and Model::load_efq
// (src/model.cpp:66-111) as one upload into HBM.
//
// Upload: the reference maps the file and streams every weight from the page cache on every
// token.  Here the tensor region of the file, [first tensor offset, end of last tensor), is copied
// once into a single device arena with the file's own layout, so every tensor keeps its 64-byte
// aligned offset (arena base + offset - first offset) and the arena is one sequential stream
// (pinned double-buffered staging, 64 MiB chunks, copies overlapping the next chunk's read from
// the mapping).  Matrices become weight handles over the arena; norms are FP32 device arrays in
// place.  Tied embeddings (tie_word_embeddings) use the embedding handle as the lm_head, as the
// reference does (src/model.cpp:86).
#include <atomic>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "efq.h"

namespace efh {
void engine_set_owner(ef_hip_engine e, std::atomic<int>* refs);
}

namespace {
constexpr uint32_t kEfqMagic = 0x45465146u;    // "EFQF"
constexpr uint32_t kModelMagic = 0x4546514Du;  // "EFQM"
constexpr size_t kChunk = size_t{64} << 20;
}  // namespace

struct ef_hip_efq_s {
  uint32_t magic = kEfqMagic;
  std::unique_ptr<efh::efq::File> file;
};

struct ef_hip_model_s {
  uint32_t magic = kModelMagic;
  ef_hip_model_config cfg{};
  bool tied = false;
  int64_t bos = -1, eos = -1;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  std::vector<ef_hip_layer> layers;
  std::vector<ef_hip_weight> handles;
  ef_hip_weight embed = nullptr, lm_head = nullptr;
  const float* final_norm = nullptr;
  std::string description;
  uint64_t bytes_per_token = 0;
  std::atomic<int> engines{0};
};

namespace efh {
namespace {

int check_efq(ef_hip_efq f) {
  if (f == nullptr || f->magic != kEfqMagic || !f->file) return fail(EF_HIP_ESTATE, "not an open .efq handle");
  return EF_HIP_OK;
}

int check_model(ef_hip_model m) {
  if (m == nullptr || m->magic != kModelMagic) return fail(EF_HIP_ESTATE, "not a device model handle");
  return EF_HIP_OK;
}

ef_hip_model_config config_of(const efq::Config& c) {
  ef_hip_model_config o{};
  o.D = static_cast<size_t>(c.hidden_size);
  o.F = static_cast<size_t>(c.intermediate_size);
  o.H = static_cast<size_t>(c.num_attention_heads);
  o.KV = static_cast<size_t>(c.num_key_value_heads);
  o.hd = static_cast<size_t>(c.head_dim);
  o.V = static_cast<size_t>(c.vocab_size);
  o.L = static_cast<size_t>(c.num_hidden_layers);
  o.max_pos = static_cast<size_t>(c.max_position_embeddings);
  o.eps = static_cast<float>(c.rms_norm_eps);
  o.rope_theta = static_cast<float>(c.rope_theta);
  return o;
}

void release_model(ef_hip_model m) {
  for (ef_hip_weight w : m->handles) (void)ef_hip_weight_release(w);
  if (m->arena != nullptr) (void)hipFree(m->arena);
  m->magic = 0;
  delete m;
}

// Copies [lo, hi) of the mapping into the arena through two pinned buffers on `s`.
int upload_region(const uint8_t* base, uint64_t lo, uint64_t hi, uint8_t* arena, hipStream_t s) {
  uint8_t* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int rc = EF_HIP_OK;
  auto cleanup = [&]() {
    (void)hipStreamSynchronize(s);
    for (int k = 0; k < 2; ++k) {
      if (stage[k] != nullptr) (void)hipHostFree(stage[k]);
      if (done[k] != nullptr) (void)hipEventDestroy(done[k]);
    }
  };
  const size_t chunk = static_cast<size_t>(std::min<uint64_t>(kChunk, hi - lo));
  for (int k = 0; k < 2; ++k) {
    if (hipHostMalloc(reinterpret_cast<void**>(&stage[k]), chunk, hipHostMallocDefault) != hipSuccess) {
      cleanup();
      return fail(EF_HIP_ENOMEM, "efq upload: pinned staging");
    }
    if (hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess) {
      cleanup();
      return fail(EF_HIP_ERUNTIME, "efq upload: event");
    }
  }
  uint64_t off = lo;
  for (int k = 0; off < hi && rc == EF_HIP_OK; ++k) {
    const int b = k & 1;
    const size_t n = static_cast<size_t>(std::min<uint64_t>(chunk, hi - off));
    if (k >= 2 && hipEventSynchronize(done[b]) != hipSuccess) {
      rc = fail(EF_HIP_ERUNTIME, "efq upload: wait for staging buffer");
      break;
    }
    std::memcpy(stage[b], base + off, n);
    if (hipMemcpyAsync(arena + (off - lo), stage[b], n, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipEventRecord(done[b], s) != hipSuccess) {
      rc = fail(EF_HIP_ERUNTIME, "efq upload: host-to-device copy");
      break;
    }
    off += n;
  }
  if (rc == EF_HIP_OK && hipStreamSynchronize(s) != hipSuccess) rc = fail(EF_HIP_ERUNTIME, "efq upload: sync");
  cleanup();
  return rc;
}

int build_model(const efq::File& f, ef_hip_model* out) {
  const efq::Layout& L = f.layout();
  auto* m = new ef_hip_model_s;
  m->cfg = config_of(L.cfg);
  m->tied = L.cfg.tie_word_embeddings;
  m->bos = L.cfg.bos_token_id;
  m->eos = L.cfg.eos_token_id;
  m->bytes_per_token = f.bytes_per_token();
  uint64_t lo = ~uint64_t{0}, hi = 0;
  for (const efq::Tensor& t : L.tensors) {
    lo = std::min(lo, t.offset);
    hi = std::max(hi, t.offset + t.bytes);
  }
  m->arena_bytes = static_cast<size_t>(hi - lo);
  if (hipMalloc(&m->arena, std::max<size_t>(m->arena_bytes, 1)) != hipSuccess) {
    release_model(m);
    return fail(EF_HIP_ENOMEM, "efq upload: device arena of " + std::to_string(hi - lo) + " bytes");
  }
  int rc = upload_region(f.base(), lo, hi, static_cast<uint8_t*>(m->arena), ctx().stream);
  if (rc != EF_HIP_OK) {
    release_model(m);
    return rc;
  }
  auto dev_of = [&](const efq::Tensor& t) { return static_cast<uint8_t*>(m->arena) + (t.offset - lo); };
  size_t n_q4 = 0, n_q8 = 0, n_other = 0;
  auto matrix = [&](const std::string& name, bool count, ef_hip_weight* w) -> int {
    const efq::Tensor& t = f.at(name);
    if (t.shape.size() != 2) return fail(EF_HIP_EINVAL, "'" + name + "' must be a matrix");
    EFH_RC(ef_hip_weight_register_device(dev_of(t), t.qtype, t.rows(), t.cols(), w));
    m->handles.push_back(*w);
    if (count) (t.qtype == EF_QTYPE_Q4_0 ? n_q4 : t.qtype == EF_QTYPE_Q8_0 ? n_q8 : n_other)++;
    return EF_HIP_OK;
  };
  auto vec = [&](const std::string& name) { return reinterpret_cast<const float*>(dev_of(f.at(name))); };
  try {
    if ((rc = matrix("model.embed_tokens.weight", false, &m->embed)) != EF_HIP_OK) {
      release_model(m);
      return rc;
    }
    if (m->tied) {
      m->lm_head = m->embed;
    } else if ((rc = matrix("lm_head.weight", true, &m->lm_head)) != EF_HIP_OK) {
      release_model(m);
      return rc;
    }
    m->final_norm = vec("model.norm.weight");
    m->layers.resize(m->cfg.L);
    for (size_t l = 0; l < m->cfg.L; ++l) {
      const std::string p = "model.layers." + std::to_string(l) + ".";
      ef_hip_layer& w = m->layers[l];
      if ((rc = matrix(p + "self_attn.q_proj.weight", true, &w.wq)) || (rc = matrix(p + "self_attn.k_proj.weight", true, &w.wk)) ||
          (rc = matrix(p + "self_attn.v_proj.weight", true, &w.wv)) || (rc = matrix(p + "self_attn.o_proj.weight", true, &w.wo)) ||
          (rc = matrix(p + "mlp.gate_proj.weight", true, &w.w_gate)) || (rc = matrix(p + "mlp.up_proj.weight", true, &w.w_up)) ||
          (rc = matrix(p + "mlp.down_proj.weight", true, &w.w_down))) {
        release_model(m);
        return rc;
      }
      w.attn_norm_dev = vec(p + "input_layernorm.weight");
      w.ffn_norm_dev = vec(p + "post_attention_layernorm.weight");
    }
  } catch (const efq::Error& e) {
    release_model(m);
    return fail(EF_HIP_EINVAL, e.what());
  }
  // Model::description for an .efq model (src/model.cpp:102-107)
  const std::string& policy = L.policy.name;
  m->description = "efq" + (policy.empty() ? std::string() : ", policy " + policy) + ": " + std::to_string(n_q4) +
                   " Q4_0 + " + std::to_string(n_q8) + " Q8_0" +
                   (n_other ? " + " + std::to_string(n_other) + " other" : std::string()) + " matrices, embedding " +
                   efq::qtype_name(f.at("model.embed_tokens.weight").qtype);
  *out = m;
  return EF_HIP_OK;
}

int copy_str(const std::string& s, char* buf, size_t cap) {
  EFH_CHECK(buf != nullptr && cap > 0, "null or empty output buffer");
  const size_t n = std::min(s.size(), cap - 1);
  std::memcpy(buf, s.data(), n);
  buf[n] = '\0';
  return s.size() < cap ? EF_HIP_OK : fail(EF_HIP_EINVAL, "output buffer too small");
}

}  // namespace
}  // namespace efh

using namespace efh;

extern "C" {

int ef_hip_efq_open(const char* path, ef_hip_efq* out) {
  EFH_CHECK(path != nullptr && out != nullptr, "efq_open: null argument");
  try {
    auto* f = new ef_hip_efq_s;
    try {
      f->file = efq::File::open(path);
    } catch (...) {
      delete f;
      throw;
    }
    *out = f;
    return EF_HIP_OK;
  } catch (const efq::Error& e) {
    return fail(EF_HIP_EINVAL, e.what());
  } catch (const std::bad_alloc&) {
    return fail(EF_HIP_ENOMEM, "efq_open: out of host memory");
  }
}

int ef_hip_efq_parse(const void* bytes, size_t size, ef_hip_efq* out) {
  EFH_CHECK((bytes != nullptr || size == 0) && out != nullptr, "efq_parse: null argument");
  static const uint8_t kNone[1] = {0};
  try {
    auto* f = new ef_hip_efq_s;
    try {
      f->file = efq::File::over(bytes ? static_cast<const uint8_t*>(bytes) : kNone, size);
    } catch (...) {
      delete f;
      throw;
    }
    *out = f;
    return EF_HIP_OK;
  } catch (const efq::Error& e) {
    return fail(EF_HIP_EINVAL, e.what());
  } catch (const std::bad_alloc&) {
    return fail(EF_HIP_ENOMEM, "efq_parse: out of host memory");
  }
}

int ef_hip_efq_close(ef_hip_efq f) {
  EFH_RC(check_efq(f));
  f->magic = 0;
  delete f;
  return EF_HIP_OK;
}

int ef_hip_efq_config(ef_hip_efq f, ef_hip_model_config* cfg, int* tie_word_embeddings, int64_t* bos_token_id,
                      int64_t* eos_token_id) {
  EFH_RC(check_efq(f));
  const efq::Config& c = f->file->layout().cfg;
  if (cfg) *cfg = config_of(c);
  if (tie_word_embeddings) *tie_word_embeddings = c.tie_word_embeddings ? 1 : 0;
  if (bos_token_id) *bos_token_id = c.bos_token_id;
  if (eos_token_id) *eos_token_id = c.eos_token_id;
  return EF_HIP_OK;
}

int ef_hip_efq_tensor_count(ef_hip_efq f, size_t* n) {
  EFH_RC(check_efq(f));
  EFH_CHECK(n != nullptr, "efq_tensor_count: null argument");
  *n = f->file->layout().tensors.size();
  return EF_HIP_OK;
}

int ef_hip_efq_tensor_info(ef_hip_efq f, size_t i, ef_hip_efq_tensor* out) {
  EFH_RC(check_efq(f));
  EFH_CHECK(out != nullptr, "efq_tensor_info: null argument");
  const auto& ts = f->file->layout().tensors;
  EFH_CHECK(i < ts.size(), "efq_tensor_info: index out of range");
  const efq::Tensor& t = ts[i];
  out->name = t.name.c_str();
  out->rule = t.rule.c_str();
  out->qtype = t.qtype;
  out->ndim = static_cast<int>(t.shape.size());
  out->rows = static_cast<size_t>(t.rows());
  out->cols = static_cast<size_t>(t.cols());
  out->offset = t.offset;
  out->bytes = t.bytes;
  out->rel_rmse = t.rel_rmse;
  out->max_abs_err = t.max_abs_err;
  out->host_data = f->file->data(t);
  return EF_HIP_OK;
}

int ef_hip_efq_find(ef_hip_efq f, const char* name, size_t* index) {
  EFH_RC(check_efq(f));
  EFH_CHECK(name != nullptr && index != nullptr, "efq_find: null argument");
  const efq::Tensor* t = f->file->find(name);
  if (t == nullptr) return fail(EF_HIP_EINVAL, std::string("tensor '") + name + "' not found in '" + f->file->path() + "'");
  *index = static_cast<size_t>(t - f->file->layout().tensors.data());
  return EF_HIP_OK;
}

int ef_hip_efq_bytes_per_token(ef_hip_efq f, uint64_t* out) {
  EFH_RC(check_efq(f));
  EFH_CHECK(out != nullptr, "efq_bytes_per_token: null argument");
  *out = f->file->bytes_per_token();
  return EF_HIP_OK;
}

int ef_hip_efq_policy(ef_hip_efq f, int* layers, int* lm_head, int* embed, size_t* n_overrides, char* name,
                      size_t name_cap) {
  EFH_RC(check_efq(f));
  const efq::Policy& p = f->file->layout().policy;
  if (layers) *layers = p.layers;
  if (lm_head) *lm_head = p.lm_head;
  if (embed) *embed = p.embed;
  if (n_overrides) *n_overrides = p.overrides.size();
  if (name != nullptr) return copy_str(p.name, name, name_cap);
  return EF_HIP_OK;
}

int ef_hip_model_upload(ef_hip_efq f, ef_hip_model* out) {
  EFH_RC(require_ready());
  EFH_RC(check_efq(f));
  EFH_CHECK(out != nullptr, "model_upload: null argument");
  return build_model(*f->file, out);
}

int ef_hip_model_load_efq(const char* path, ef_hip_model* out) {
  EFH_RC(require_ready());
  ef_hip_efq f = nullptr;
  EFH_RC(ef_hip_efq_open(path, &f));
  const int rc = ef_hip_model_upload(f, out);
  (void)ef_hip_efq_close(f);  // the device copy does not need the mapping
  return rc;
}

int ef_hip_model_free(ef_hip_model m) {
  EFH_RC(check_model(m));
  if (m->engines.load() != 0)
    return fail(EF_HIP_ESTATE, "model_free: destroy the engines created from this model first");
  release_model(m);
  return EF_HIP_OK;
}

int ef_hip_model_config_get(ef_hip_model m, ef_hip_model_config* cfg, int* tie_word_embeddings, int64_t* eos_token_id) {
  EFH_RC(check_model(m));
  if (cfg) *cfg = m->cfg;
  if (tie_word_embeddings) *tie_word_embeddings = m->tied ? 1 : 0;
  if (eos_token_id) *eos_token_id = m->eos;
  return EF_HIP_OK;
}

int ef_hip_model_description(ef_hip_model m, char* buf, size_t cap) {
  EFH_RC(check_model(m));
  return copy_str(m->description, buf, cap);
}

int ef_hip_model_bytes_per_token(ef_hip_model m, uint64_t* out) {
  EFH_RC(check_model(m));
  EFH_CHECK(out != nullptr, "model_bytes_per_token: null argument");
  *out = m->bytes_per_token;
  return EF_HIP_OK;
}

int ef_hip_model_layer(ef_hip_model m, size_t l, ef_hip_layer* out) {
  EFH_RC(check_model(m));
  EFH_CHECK(out != nullptr && l < m->layers.size(), "model_layer: null argument or layer out of range");
  *out = m->layers[l];
  return EF_HIP_OK;
}

int ef_hip_model_tensors(ef_hip_model m, ef_hip_weight* embed, ef_hip_weight* lm_head, const float** final_norm_dev) {
  EFH_RC(check_model(m));
  if (embed) *embed = m->embed;
  if (lm_head) *lm_head = m->lm_head;
  if (final_norm_dev) *final_norm_dev = m->final_norm;
  return EF_HIP_OK;
}

int ef_hip_model_engine_create(ef_hip_model m, size_t max_seq, int batch, ef_hip_engine* out) {
  EFH_RC(check_model(m));
  EFH_CHECK(out != nullptr, "model_engine_create: null argument");
  EFH_RC(ef_hip_engine_create(&m->cfg, m->layers.data(), m->embed, m->lm_head, m->final_norm, max_seq, batch, out));
  m->engines.fetch_add(1);
  engine_set_owner(*out, &m->engines);
  return EF_HIP_OK;
}

}  // extern "C"
