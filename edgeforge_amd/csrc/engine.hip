// Device decode engine: Transformer::forward (src/model.cpp:184-276) for `batch` independent
// sequences sharing one set of packed weights, plus the reference decode protocol
// (src/bench_decode.cpp:30-49) driven entirely on the device.
//
// HBM layout: activations [batch][dim] FP32; KV cache [L][batch][max_seq][KV*hd] FP32 (the
// reference's [L][max_seq][kv_dim] with the sequence index inserted); token history
// [batch][max_seq] int32 (prompt, then picked tokens); the position is one int32 in device memory.
// Every kernel of a step reads the position and the input token from device memory, so each step
// kind is captured once as a HIP graph and replayed: a whole generation is a chain of graph
// launches with no host round-trip between tokens.
//
// One step per layer: [rmsnorm + q/k/v GEMV] -> [RoPE + attention, cache write] -> [o GEMV +
// residual] -> [rmsnorm + gate/up GEMV + SwiGLU] -> [down GEMV + residual]; then [final rmsnorm +
// lm_head GEMV] and the token pick (argmax or the sampler) when logits are needed.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <vector>

#include "codec.h"
#include "common.h"
#include "gemv.h"
#include "glue.h"
#include "sampler.h"

namespace {
constexpr uint32_t kEngineMagic = 0x45464845u;  // "EFHE"
enum StepMode : int {
  kLogits = 1, kGreedy = 2, kSample = 4, kAdvance = 8, kPrefill = 16, kEos = 32, kAllLogits = 64,
  kSplit = 128  // decode attention by the position-split kernels (a step at a position >= kSplitFrom)
};
// Kernel groups of a decode step (the reference's ForwardProfile buckets, include/ef/model.h:89-94,
// merged where this build fuses them): a step enqueues the groups its mask selects, so a profile
// can capture and time each group's launches on their own.
enum StepGroup : unsigned {
  kGEmbed = 1u << EF_HIP_PROF_EMBED,
  kGQkv = 1u << EF_HIP_PROF_QKV,
  kGAttn = 1u << EF_HIP_PROF_ATTENTION,
  kGOproj = 1u << EF_HIP_PROF_OPROJ,
  kGGateUp = 1u << EF_HIP_PROF_GATE_UP,
  kGDown = 1u << EF_HIP_PROF_DOWN,
  kGLmHead = 1u << EF_HIP_PROF_LM_HEAD,
  kGPick = 1u << EF_HIP_PROF_PICK,
  kAllGroups = (1u << EF_HIP_PROF_GROUPS) - 1u,
};
// Decode positions from which a step uses the position-split attention (when the engine has its
// workspace): below, the single-pass kernels are faster (measured crossover: about 130 positions at
// B = 1, 210 at B = 16, TinyLlama shapes).
constexpr size_t kSplitFrom = 192;
// Rows (sequences x positions) of one batched prefill launch; longer prompts go in chunks.
constexpr size_t kPrefillRows = 4096;
}  // namespace

struct ef_hip_engine_s {
  uint32_t magic = 0;
  ef_hip_model_config c{};
  std::vector<ef_hip_layer> layers;
  ef_hip_weight embed = nullptr, lm_head = nullptr;
  const float* final_norm = nullptr;
  size_t max_seq = 0, kvd = 0, cached = 0;
  int B = 1;
  hipStream_t stream = nullptr;
  float *x = nullptr, *q = nullptr, *knew = nullptr, *vnew = nullptr, *ctx = nullptr, *act = nullptr;
  float *logits = nullptr, *hidden = nullptr, *kc = nullptr, *vc = nullptr, *cos_t = nullptr, *sin_t = nullptr;
  float* rope_now = nullptr;  // RoPE's cos / sin rows at the step's position (written by embed_at)
  int32_t *hist = nullptr, *hist_len = nullptr, *next_tok = nullptr, *pos = nullptr, *n_prompt = nullptr;
  uint32_t* step_counter = nullptr;  // zero between steps (argmax_finish re-arms it)
  // position-split decode attention (long caches, few sequences): partial results, or null when
  // the step does not split
  float* attn_part = nullptr;
  int attn_splits = 1, attn_span = 0;
  int32_t* out_tokens = nullptr;
  void* sample_ws = nullptr;
  void* gemv_ws = nullptr;  // prepared activation fragments of the batched GEMVs (B > 1)
  size_t gemv_ws_bytes = 0;
  int32_t* stage = nullptr;  // pinned host staging
  int32_t* tok_dev = nullptr;  // device staging of token ids ([batch][n] rows before they move into hist)
  std::vector<void*> allocs;
  std::map<int, hipGraphExec_t> graphs;
  // Graph executables taken out of use (stale arguments, a finished profile) are kept until the
  // engine is destroyed instead of being destroyed mid-process: a profiler that traces the graphs'
  // kernels may still be reading a just-finished launch's records when its executable would go.
  std::vector<hipGraphExec_t> retired;
  ef_hip_sampler_config scfg{};
  void* rng = nullptr;
  std::atomic<int>* owner_refs = nullptr;  // live-engine count of the device model it was made from
  // batched prefill: activations of `pf_rows` rows (sequence-major: row b * n + i) and the GEMV
  // workspace for that many rows, allocated on first use
  size_t pf_rows = 0;
  float *pf_x = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr, *pf_ctx = nullptr, *pf_act = nullptr;
  void* pf_ws = nullptr;
  size_t pf_ws_bytes = 0;
  float* pf_logits = nullptr;  // [pf_rows][V], teacher-forced scoring only (allocated on first use)
  size_t pf_logit_rows = 0;
  // chat turns (ef_hip_engine_reply): the token ids whose K / V the cache holds, P(EOS) per
  // sequence and per generated token, and a copy of the RNG states taken before each window of steps
  std::vector<int32_t> chat_ids;
  int eos_id = -1;
  double* eos_cur = nullptr;  // [B]
  double* eos_out = nullptr;  // [B][max_seq]
  void* rng_snap = nullptr;
  // several-sequence step over producer-staged tables (afrag.h): table set a holds the inputs of
  // q/k/v, gate/up and lm_head (K = D, with the RMSNorm's per-block partial sums), set b those of
  // o_proj and down; each set has both column orders
  bool staged = false;
  std::string staged_why;  // why the staged step is off (empty when on)
  uint8_t *ta4 = nullptr, *ta8 = nullptr, *tb4 = nullptr, *tb8 = nullptr;
  float *ta_s = nullptr, *tb_s = nullptr;
  double *ta_ssp = nullptr, *tb_ssp = nullptr;
  int bpad = 0;
};

namespace efh {
namespace {

int check_engine(ef_hip_engine e) {
  if (e == nullptr) return fail(EF_HIP_EINVAL, "null engine");
  if (e->magic != kEngineMagic) return fail(EF_HIP_ESTATE, "engine was destroyed or is not an engine");
  return EF_HIP_OK;
}

template <class T>
int dev_alloc(ef_hip_engine e, T** p, size_t count) {
  void* v = nullptr;
  EFH_HIP(hipMalloc(&v, std::max<size_t>(count, 1) * sizeof(T)));
  e->allocs.push_back(v);
  *p = static_cast<T*>(v);
  return EF_HIP_OK;
}

// Every storage type runs through the GEMVs (Q4_0 / Q8_0 packed, F32 / F16 / BF16 dense), as
// kern::matvec_rows dispatches all five (src/qkernels.cpp:213-269).
int check_matrix(ef_hip_weight w, size_t rows, size_t cols, const char* what) {
  int rc = check_weight(w);
  if (rc != EF_HIP_OK) return fail(rc, std::string(what) + ": bad weight handle");
  if (w->rows != rows || w->cols != cols) {
    return fail(EF_HIP_EINVAL, std::string(what) + ": shape " + std::to_string(w->rows) + "x" +
                                   std::to_string(w->cols) + ", config needs " + std::to_string(rows) + "x" +
                                   std::to_string(cols));
  }
  if (!is_dense_qtype(w->qtype) && cols % 32 != 0)
    return fail(EF_HIP_EINVAL, std::string(what) + ": Q4_0 / Q8_0 need cols % 32 == 0");
  if (is_dense_qtype(w->qtype) && cols > kMaxDenseCols)
    return fail(EF_HIP_EINVAL, std::string(what) + ": F32 / F16 / BF16 matrices need cols <= 16320");
  return EF_HIP_OK;
}


int enqueue_tail(ef_hip_engine e, int mode, unsigned groups = kAllGroups, bool staged_in = false);

// hist[b][pos .. pos + n) = stage[b * n .. b * n + n) for every sequence b: one contiguous copy of
// the pinned staging words (plus the 8 words after them) to the device, then a row-copy kernel into
// the history rows.  The caller has filled e->stage and keeps it untouched until the stream syncs.
int put_tokens(ef_hip_engine e, size_t pos, size_t n) {
  const size_t words = n * static_cast<size_t>(e->B);
  EFH_HIP(hipMemcpyAsync(e->tok_dev, e->stage, (words + 8) * 4, hipMemcpyHostToDevice, e->stream));
  return launch_copy_rows(e->tok_dev, static_cast<long>(n), e->hist + pos, static_cast<long>(e->max_seq),
                          static_cast<int>(n), e->B, e->stream);
}

AttnArgs attn_args(ef_hip_engine e, bool split) {
  const ef_hip_model_config& c = e->c;
  AttnArgs a{};
  a.q = e->q;
  a.knew = e->knew;
  a.vnew = e->vnew;
  a.cos_t = e->cos_t;
  a.sin_t = e->sin_t;
  a.pos_dev = e->pos;
  a.rope_now = e->rope_now;
  a.ctx = e->ctx;
  a.ldq = static_cast<long>(c.D);
  a.H = static_cast<int>(c.H);
  a.KV = static_cast<int>(c.KV);
  a.hd = static_cast<int>(c.hd);
  a.max_seq = static_cast<int>(e->max_seq);
  a.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.hd)));  // src/kernels.cpp:158
  a.part = split ? e->attn_part : nullptr;
  a.splits = e->attn_splits;
  a.span = e->attn_span;
  return a;
}

// Staging of a product's input tables: set a (with the norm's partial sums, norm weights nw) or
// set b, in the column orders of the consuming matrices.
AEmit table_emit(ef_hip_engine e, bool set_a, std::initializer_list<ef_hip_weight> consumers, const float* nw,
                 size_t K) {
  AEmit m{};
  bool q4 = false, q8 = false;
  for (ef_hip_weight w : consumers) {
    q4 = q4 || w->qtype == EF_QTYPE_Q4_0;
    q8 = q8 || w->qtype == EF_QTYPE_Q8_0;
  }
  m.t4 = q4 ? (set_a ? e->ta4 : e->tb4) : nullptr;
  m.t8 = q8 ? (set_a ? e->ta8 : e->tb8) : nullptr;
  m.bscale = set_a ? e->ta_s : e->tb_s;
  m.ssp = set_a ? e->ta_ssp : nullptr;
  m.nw = nw;
  m.nb = static_cast<int>(K / 32);
  m.bpad = e->bpad;
  return m;
}

MfmaStage table_set(ef_hip_engine e, bool set_a) {
  MfmaStage st{};
  st.t4 = set_a ? e->ta4 : e->tb4;
  st.t8 = set_a ? e->ta8 : e->tb8;
  st.bscale = set_a ? e->ta_s : e->tb_s;
  st.bpad = e->bpad;
  if (set_a) {
    st.ssp = e->ta_ssp;
    st.n_ssp = static_cast<int>(e->c.D / 32);
    st.eps = e->c.eps;
  }
  return st;
}

// The step's product jobs of layer l (q/k/v, o, gate/up, down) and lm_head.
struct LayerJobs {
  GemvJob qkv[3], o, gu, dn;
};
LayerJobs layer_jobs(ef_hip_engine e, size_t l) {
  const ef_hip_layer& w = e->layers[l];
  const size_t D = e->c.D, F = e->c.F, kvd = e->kvd;
  return LayerJobs{{{w.wq, nullptr, e->x, e->q, D, D}, {w.wk, nullptr, e->x, e->knew, D, kvd},
                    {w.wv, nullptr, e->x, e->vnew, D, kvd}},
                   {w.wo, nullptr, e->ctx, e->x, D, D},
                   {w.w_gate, w.w_up, e->x, e->act, D, F},
                   {w.w_down, nullptr, e->act, e->x, F, D}};
}
GemvJob lm_job(ef_hip_engine e) { return GemvJob{e->lm_head, nullptr, e->x, e->logits, e->c.D, e->c.V}; }

// Whether the several-sequence step runs over producer-staged tables: the embedding lookup, the
// KV-group attention and the o / gate-up / down products write the next product's input tables as
// they store their outputs (afrag.h), so no product runs a preparation launch (the o projection
// gets one when the attention kernel is not the KV-group one).  Needs packed matrices with a
// matrix-core plan for every product; EF_HIP_DECODE_TABLES=prep keeps the per-product preparation.
// Allocates the table sets and grows the GEMV workspace to the staged plans.
int build_staged(ef_hip_engine e) {
  const ef_hip_model_config& c = e->c;
  e->staged = false;
  const char* env = std::getenv("EF_HIP_DECODE_TABLES");
  if (env != nullptr && std::strcmp(env, "prep") == 0) {
    e->staged_why = "off: EF_HIP_DECODE_TABLES=prep";
    return EF_HIP_OK;
  }
  if (e->B < 2) {
    e->staged_why = "one sequence";
    return EF_HIP_OK;
  }
  if (c.D > static_cast<size_t>(kStageMaxK)) {
    e->staged_why = "D above the table preparation's limit";
    return EF_HIP_OK;
  }
  const int B = e->B;
  size_t need = 0;
  auto plan = [&](const GemvJob* j, int n, int epi, bool emit) {
    const size_t b = gemv_mfma_staged_workspace_bytes(j, n, epi, B, emit);
    need = std::max(need, b);
    return b > 0;
  };
  bool ok = true;
  for (size_t l = 0; l < c.L && ok; ++l) {
    const LayerJobs j = layer_jobs(e, l);
    ok = plan(j.qkv, 3, kEpiStore, false) && plan(&j.o, 1, kEpiResidual, true) &&
         plan(&j.gu, 1, kEpiSwiglu, true) && plan(&j.dn, 1, kEpiResidual, true);
  }
  const GemvJob lm = lm_job(e);
  ok = ok && plan(&lm, 1, kEpiStore, false);
  if (!ok) {
    e->staged_why = "a product has no matrix-core plan (unquantized matrices or shapes)";
    return EF_HIP_OK;
  }
  const size_t Kb = std::max(c.D, c.F);
  const int bpad = stage_bpad(B);
  const size_t ta = stage_table_bytes(static_cast<int>(c.D), B), tb = stage_table_bytes(static_cast<int>(Kb), B);
  EFH_RC(dev_alloc(e, &e->ta4, ta));
  EFH_RC(dev_alloc(e, &e->ta8, ta));
  EFH_RC(dev_alloc(e, &e->tb4, tb));
  EFH_RC(dev_alloc(e, &e->tb8, tb));
  EFH_RC(dev_alloc(e, &e->ta_s, c.D / 32 * bpad));
  EFH_RC(dev_alloc(e, &e->tb_s, Kb / 32 * bpad));
  EFH_RC(dev_alloc(e, &e->ta_ssp, c.D / 32 * bpad));
  EFH_RC(dev_alloc(e, &e->tb_ssp, static_cast<size_t>(bpad)));
  for (auto [p, n] : {std::pair<void*, size_t>{e->ta4, ta}, {e->ta8, ta}, {e->tb4, tb}, {e->tb8, tb},
                      {e->ta_s, c.D / 32 * bpad * 4}, {e->tb_s, Kb / 32 * bpad * 4},
                      {e->ta_ssp, c.D / 32 * bpad * 8}})
    EFH_HIP(hipMemsetAsync(p, 0, n, e->stream));
  if (need > e->gemv_ws_bytes) {
    void* gw = nullptr;
    EFH_HIP(hipMalloc(&gw, need));
    e->allocs.push_back(gw);
    e->gemv_ws = gw;
    e->gemv_ws_bytes = need;
  }
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->bpad = bpad;
  e->staged = true;
  e->staged_why.clear();
  return EF_HIP_OK;
}

// The layers of a several-sequence step over staged tables.
int enqueue_staged_layers(ef_hip_engine e, unsigned groups, bool split) {
  const ef_hip_model_config& c = e->c;
  const int B = e->B;
  const size_t D = c.D, F = c.F, kvd = e->kvd, S = e->max_seq;
  hipStream_t s = e->stream;
  const MfmaStage sa = table_set(e, true), sb = table_set(e, false);
  if (groups & kGEmbed) {
    const ef_hip_layer& w0 = e->layers[0];
    const AEmit em = table_emit(e, true, {w0.wq, w0.wk, w0.wv}, w0.attn_norm_dev, D);
    EFH_RC(launch_embed_at(e->embed, e->hist, static_cast<long>(S), e->pos, B, e->x, static_cast<long>(D), s,
                           e->cos_t, e->sin_t, static_cast<int>(c.hd / 2), e->rope_now, &em));
  }
  AttnArgs a = attn_args(e, split);
  const bool group_attn = attention_uses_group(a, B);
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = e->layers[l];
    const LayerJobs j = layer_jobs(e, l);
    if (groups & kGQkv)
      EFH_RC(launch_gemv_mfma_staged(j.qkv, 3, kEpiStore, sa, B, D, e->gemv_ws, e->gemv_ws_bytes, s));
    a.kcache = e->kc + l * B * S * kvd;
    a.vcache = e->vc + l * B * S * kvd;
    a.em = group_attn ? table_emit(e, false, {w.wo}, nullptr, D) : AEmit{};
    if (groups & kGAttn) {
      EFH_RC(launch_attention(a, B, s));
      if (!group_attn) {
        MfmaStage pb = sb;
        pb.ssp = e->tb_ssp;  // written by the preparation, unused by the product
        EFH_RC(launch_stage_tables(e->ctx, D, static_cast<int>(D), B, nullptr, pb, s));
      }
    }
    if (groups & kGOproj) {
      const AEmit em = table_emit(e, true, {w.w_gate, w.w_up}, w.ffn_norm_dev, D);
      EFH_RC(launch_gemv_mfma_staged(&j.o, 1, kEpiResidual, sb, B, D, e->gemv_ws, e->gemv_ws_bytes, s, &em));
    }
    if (groups & kGGateUp) {
      const AEmit em = table_emit(e, false, {w.w_down}, nullptr, F);
      EFH_RC(launch_gemv_mfma_staged(&j.gu, 1, kEpiSwiglu, sa, B, F, e->gemv_ws, e->gemv_ws_bytes, s, &em));
    }
    if (groups & kGDown) {
      const bool last = l + 1 == c.L;
      const ef_hip_layer& nx = e->layers[last ? l : l + 1];
      const AEmit em = last ? table_emit(e, true, {e->lm_head}, e->final_norm, D)
                            : table_emit(e, true, {nx.wq, nx.wk, nx.wv}, nx.attn_norm_dev, D);
      EFH_RC(launch_gemv_mfma_staged(&j.dn, 1, kEpiResidual, sb, B, D, e->gemv_ws, e->gemv_ws_bytes, s, &em));
    }
  }
  return EF_HIP_OK;
}

int enqueue_step(ef_hip_engine e, int mode, unsigned groups = kAllGroups) {
  const ef_hip_model_config& c = e->c;
  const int B = e->B;
  const size_t D = c.D, F = c.F, kvd = e->kvd, S = e->max_seq;
  hipStream_t s = e->stream;
  if (e->staged) {
    EFH_RC(enqueue_staged_layers(e, groups, (mode & kSplit) != 0));
    return enqueue_tail(e, mode, groups, true);
  }
  if (groups & kGEmbed)
    EFH_RC(launch_embed_at(e->embed, e->hist, static_cast<long>(S), e->pos, B, e->x, static_cast<long>(D), s,
                           e->cos_t, e->sin_t, static_cast<int>(c.hd / 2), e->rope_now));
  AttnArgs a = attn_args(e, (mode & kSplit) != 0);
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = e->layers[l];
    const GemvJob qkv[3] = {{w.wq, nullptr, e->x, e->q, D, D},
                            {w.wk, nullptr, e->x, e->knew, D, kvd},
                            {w.wv, nullptr, e->x, e->vnew, D, kvd}};
    if (groups & kGQkv)
      EFH_RC(launch_gemv(qkv, 3, kEpiStore, w.attn_norm_dev, c.eps, B, D, D, s, e->gemv_ws, e->gemv_ws_bytes));
    a.kcache = e->kc + l * B * S * kvd;
    a.vcache = e->vc + l * B * S * kvd;
    if (groups & kGAttn) EFH_RC(launch_attention(a, B, s));
    const GemvJob o{w.wo, nullptr, e->ctx, e->x, D, D};
    if (groups & kGOproj)
      EFH_RC(launch_gemv(&o, 1, kEpiResidual, nullptr, 0.0f, B, D, D, s, e->gemv_ws, e->gemv_ws_bytes));
    const GemvJob gu{w.w_gate, w.w_up, e->x, e->act, D, F};
    if (groups & kGGateUp)
      EFH_RC(launch_gemv(&gu, 1, kEpiSwiglu, w.ffn_norm_dev, c.eps, B, D, F, s, e->gemv_ws, e->gemv_ws_bytes));
    const GemvJob dn{w.w_down, nullptr, e->act, e->x, F, D};
    if (groups & kGDown)
      EFH_RC(launch_gemv(&dn, 1, kEpiResidual, nullptr, 0.0f, B, F, D, s, e->gemv_ws, e->gemv_ws_bytes));
  }
  return enqueue_tail(e, mode, groups);
}

// After the layers: final RMSNorm + lm_head, then the token pick and the step bookkeeping, or
// only the position advance (a prompt position whose logits are not needed).  staged_in: the last
// down projection staged lm_head's input tables (the staged step; not after a prefill).
int enqueue_tail(ef_hip_engine e, int mode, unsigned groups, bool staged_in) {
  const ef_hip_model_config& c = e->c;
  const int B = e->B;
  const size_t D = c.D, V = c.V, S = e->max_seq;
  hipStream_t s = e->stream;
  if ((mode & kLogits) && (groups & kGLmHead)) {
    const GemvJob lm{e->lm_head, nullptr, e->x, e->logits, D, V};
    if (staged_in) {
      EFH_RC(launch_gemv_mfma_staged(&lm, 1, kEpiStore, table_set(e, true), B, V, e->gemv_ws, e->gemv_ws_bytes, s));
    } else {
      EFH_RC(launch_gemv(&lm, 1, kEpiStore, e->final_norm, c.eps, B, D, V, s, e->gemv_ws, e->gemv_ws_bytes));
    }
  }
  if (!(groups & kGPick)) return EF_HIP_OK;
  if (mode & (kGreedy | kSample)) {
    if (mode & kGreedy) {
      StepArgs f{e->next_tok, e->hist, static_cast<long>(S), e->hist_len, e->out_tokens, static_cast<long>(S),
                 e->n_prompt, e->pos, e->step_counter};
      EFH_RC(launch_argmax_finish(e->logits, static_cast<int>(V), static_cast<long>(V), B, f, s));
    } else {
      const bool eos = (mode & kEos) != 0;
      EFH_RC(launch_sample(e->logits, static_cast<int>(V), B, static_cast<long>(V), e->scfg, e->hist, e->hist_len,
                           static_cast<long>(S), e->rng, e->next_tok, e->sample_ws, s, e->eos_id,
                           eos ? e->eos_cur : nullptr));
      EFH_RC(launch_finish_step(e->next_tok, B, e->hist, static_cast<long>(S), e->hist_len, e->out_tokens,
                                static_cast<long>(S), e->n_prompt, e->pos, s, eos ? e->eos_cur : nullptr,
                                eos ? e->eos_out : nullptr));
    }
  } else if (mode & kAdvance) {
    EFH_RC(launch_advance(e->pos, s));
  }
  return EF_HIP_OK;
}

// Batched prefill of positions *pos .. *pos + n - 1 of every sequence (tokens already in the
// history): every product runs once over all B * n rows (the matrix-core GEMV), RoPE + cache
// writes for all rows, then causal attention per (head, row) over the cache; the last row of each
// sequence becomes the decode state x, the position moves to the last prompt position and the
// tail runs as for a decode step there.  Results equal the one-position-at-a-time path to the
// GEMV's rounding.
int enqueue_prefill(ef_hip_engine e, int n, int mode) {
  const ef_hip_model_config& c = e->c;
  const int B = e->B, R = B * n;
  const size_t D = c.D, F = c.F, kvd = e->kvd, S = e->max_seq;
  hipStream_t s = e->stream;
  EFH_RC(launch_embed_rows(e->embed, e->hist, static_cast<long>(S), e->pos, n, R, e->pf_x, static_cast<long>(D), s));
  PrefillArgs pa{};
  pa.n = n;
  AttnArgs& a = pa.a;
  a.q = e->pf_q;
  a.knew = e->pf_k;
  a.vnew = e->pf_v;
  a.cos_t = e->cos_t;
  a.sin_t = e->sin_t;
  a.pos_dev = e->pos;
  a.ctx = e->pf_ctx;
  a.ldq = static_cast<long>(D);
  a.H = static_cast<int>(c.H);
  a.KV = static_cast<int>(c.KV);
  a.hd = static_cast<int>(c.hd);
  a.max_seq = static_cast<int>(S);
  a.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.hd)));  // src/kernels.cpp:158
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = e->layers[l];
    const GemvJob qkv[3] = {{w.wq, nullptr, e->pf_x, e->pf_q, D, D},
                            {w.wk, nullptr, e->pf_x, e->pf_k, D, kvd},
                            {w.wv, nullptr, e->pf_x, e->pf_v, D, kvd}};
    EFH_RC(launch_gemv(qkv, 3, kEpiStore, w.attn_norm_dev, c.eps, R, D, D, s, e->pf_ws, e->pf_ws_bytes));
    a.kcache = e->kc + l * B * S * kvd;
    a.vcache = e->vc + l * B * S * kvd;
    EFH_RC(launch_prefill_attention(pa, R, s));
    const GemvJob o{w.wo, nullptr, e->pf_ctx, e->pf_x, D, D};
    EFH_RC(launch_gemv(&o, 1, kEpiResidual, nullptr, 0.0f, R, D, D, s, e->pf_ws, e->pf_ws_bytes));
    const GemvJob gu{w.w_gate, w.w_up, e->pf_x, e->pf_act, D, F};
    EFH_RC(launch_gemv(&gu, 1, kEpiSwiglu, w.ffn_norm_dev, c.eps, R, D, F, s, e->pf_ws, e->pf_ws_bytes));
    const GemvJob dn{w.w_down, nullptr, e->pf_act, e->pf_x, F, D};
    EFH_RC(launch_gemv(&dn, 1, kEpiResidual, nullptr, 0.0f, R, F, D, s, e->pf_ws, e->pf_ws_bytes));
  }
  if (mode & kAllLogits) {  // teacher-forced scoring: final RMSNorm + lm_head on every row
    const GemvJob lm{e->lm_head, nullptr, e->pf_x, e->pf_logits, D, c.V};
    return launch_gemv(&lm, 1, kEpiStore, e->final_norm, c.eps, R, D, c.V, s, e->pf_ws, e->pf_ws_bytes);
  }
  if (n > 1) EFH_RC(launch_advance_by(e->pos, n - 1, s));
  // the last prompt row of every sequence becomes the decode state
  EFH_RC(launch_copy_rows(e->pf_x + (n - 1) * D, static_cast<long>(n * D), e->x, static_cast<long>(D),
                          static_cast<int>(D), B, s));
  return enqueue_tail(e, mode);
}

// Buffers and GEMV workspace for prefill launches of up to `rows` rows.
int ensure_prefill(ef_hip_engine e, size_t rows) {
  if (rows <= e->pf_rows) return EF_HIP_OK;
  const ef_hip_model_config& c = e->c;
  const size_t kvd = e->kvd;
  float* bufs[6] = {};
  const size_t sizes[6] = {rows * c.D, rows * c.D, rows * kvd, rows * kvd, rows * c.D, rows * c.F};
  for (int i = 0; i < 6; ++i) {
    if (hipMalloc(&bufs[i], sizes[i] * sizeof(float)) != hipSuccess) {
      for (int k = 0; k < i; ++k) (void)hipFree(bufs[k]);
      return fail(EF_HIP_ENOMEM, "engine prefill buffers");
    }
  }
  size_t need = 0;
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = e->layers[l];
    const GemvJob qkv[3] = {{w.wq, nullptr, bufs[0], bufs[1], c.D, c.D},
                            {w.wk, nullptr, bufs[0], bufs[2], c.D, kvd},
                            {w.wv, nullptr, bufs[0], bufs[3], c.D, kvd}};
    const GemvJob o{w.wo, nullptr, bufs[4], bufs[0], c.D, c.D};
    const GemvJob gu{w.w_gate, w.w_up, bufs[0], bufs[5], c.D, c.F};
    const GemvJob dn{w.w_down, nullptr, bufs[5], bufs[0], c.F, c.D};
    // every row count a launch may use (a last chunk is shorter): the plan depends on
    // min(rows, gemv_mfma_max_rows()) only; row counts up to 128 one by one, then every multiple
    // of a 16-row tile (within a tile count the workspace grows with the rows), and the full count
    const int cap = static_cast<int>(std::min<size_t>(rows, gemv_mfma_max_rows()));
    std::vector<int> counts;
    for (int r = 2; r <= std::min(cap, 128); ++r) counts.push_back(r);
    for (int r = 144; r <= cap; r += 16) counts.push_back(r);
    counts.push_back(cap);
    counts.push_back(static_cast<int>(rows));
    for (const int r : counts) {
      const GemvJob lm{e->lm_head, nullptr, bufs[0], nullptr, c.D, c.V};
      need = std::max({need, gemv_mfma_workspace_bytes(qkv, 3, kEpiStore, r, c.D),
                       gemv_mfma_workspace_bytes(&o, 1, kEpiResidual, r, c.D),
                       gemv_mfma_workspace_bytes(&gu, 1, kEpiSwiglu, r, c.D),
                       gemv_mfma_workspace_bytes(&dn, 1, kEpiResidual, r, c.F),
                       gemv_mfma_workspace_bytes(&lm, 1, kEpiStore, r, c.D)});
    }
  }
  void* ws = nullptr;
  if (need > 0 && hipMalloc(&ws, need) != hipSuccess) {
    for (float* b : bufs) (void)hipFree(b);
    return fail(EF_HIP_ENOMEM, "engine prefill GEMV workspace");
  }
  // replace the old buffers (their graphs hold the old addresses)
  EFH_HIP(hipStreamSynchronize(e->stream));
  for (auto it = e->graphs.begin(); it != e->graphs.end();) {
    if (it->first & kPrefill) {
      e->retired.push_back(it->second);
      it = e->graphs.erase(it);
    } else {
      ++it;
    }
  }
  for (float* old : {e->pf_x, e->pf_q, e->pf_k, e->pf_v, e->pf_ctx, e->pf_act})
    if (old) (void)hipFree(old);
  if (e->pf_ws) (void)hipFree(e->pf_ws);
  e->pf_x = bufs[0];
  e->pf_q = bufs[1];
  e->pf_k = bufs[2];
  e->pf_v = bufs[3];
  e->pf_ctx = bufs[4];
  e->pf_act = bufs[5];
  e->pf_ws = ws;
  e->pf_ws_bytes = need;
  e->pf_rows = rows;
  return EF_HIP_OK;
}

int graph_for(ef_hip_engine e, int mode, hipGraphExec_t* out) {
  auto it = e->graphs.find(mode);
  if (it != e->graphs.end()) {
    *out = it->second;
    return EF_HIP_OK;
  }
  EFH_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  const int rc = (mode & kPrefill) ? enqueue_prefill(e, mode >> 8, mode & 0xEF) : enqueue_step(e, mode);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(e->stream, &g);
  if (rc != EF_HIP_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (ec != hipSuccess) return fail_hip(ec, "hipStreamEndCapture");
  hipGraphExec_t ex = nullptr;
  const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ei != hipSuccess) return fail_hip(ei, "hipGraphInstantiate");
  e->graphs[mode] = ex;
  *out = ex;
  return EF_HIP_OK;
}

// The step mode for a decode step at position pos: with the split bit from kSplitFrom on.
int at_pos(ef_hip_engine e, int mode, size_t pos) {
  return e->attn_part != nullptr && pos >= kSplitFrom ? mode | kSplit : mode;
}

// Bounds the retired executables (a long chat that keeps changing sampler settings): past 256, the
// older half is destroyed after the stream has drained.
int trim_retired(ef_hip_engine e) {
  if (e->retired.size() <= 256) return EF_HIP_OK;
  EFH_HIP(hipStreamSynchronize(e->stream));
  const size_t half = e->retired.size() / 2;
  for (size_t i = 0; i < half; ++i) EFH_HIP(hipGraphExecDestroy(e->retired[i]));
  e->retired.erase(e->retired.begin(), e->retired.begin() + static_cast<long>(half));
  return EF_HIP_OK;
}

// Drops every cached graph whose mode has any of `bits` (their captured arguments are stale).
int drop_graphs_with(ef_hip_engine e, int bits) {
  EFH_HIP(hipStreamSynchronize(e->stream));
  for (auto it = e->graphs.begin(); it != e->graphs.end();) {
    if (it->first & bits) {
      e->retired.push_back(it->second);
      it = e->graphs.erase(it);
    } else {
      ++it;
    }
  }
  return trim_retired(e);
}

// Sampler settings and RNG states are captured into the graphs that sample.
int set_sampler(ef_hip_engine e, const ef_hip_sampler_config& cfg, void* rng) {
  const bool same = e->rng == rng && e->scfg.temperature == cfg.temperature && e->scfg.top_k == cfg.top_k &&
                    e->scfg.top_p == cfg.top_p && e->scfg.repetition_penalty == cfg.repetition_penalty;
  if (!same) EFH_RC(drop_graphs_with(e, kSample));
  e->scfg = cfg;
  e->rng = rng;
  return EF_HIP_OK;
}

int run_step(ef_hip_engine e, int mode) {
  hipGraphExec_t g;
  EFH_RC(graph_for(e, mode, &g));
  EFH_HIP(hipGraphLaunch(g, e->stream));
  return EF_HIP_OK;
}

// Positions [*pos, *pos + n) of every sequence in chunks of at most kPrefillRows rows; `last_mode`
// is the tail of the final chunk (earlier chunks only advance the position).  With instantiate
// set, only builds the graphs (so a timed region launches nothing new).
int run_prefill(ef_hip_engine e, size_t n, int last_mode, bool instantiate) {
  size_t rows = kPrefillRows;
  if (const char* v = std::getenv("EF_HIP_PREFILL_ROWS")) rows = std::max<long>(1, std::atol(v));  // test knob
  const size_t chunk = std::max<size_t>(1, rows / static_cast<size_t>(e->B));
  EFH_RC(ensure_prefill(e, static_cast<size_t>(e->B) * std::min(chunk, n)));
  for (size_t done = 0; done < n;) {
    const size_t k = std::min(chunk, n - done);
    const int mode = kPrefill | (done + k == n ? last_mode : kAdvance) | static_cast<int>(k << 8);
    hipGraphExec_t g;
    EFH_RC(graph_for(e, mode, &g));
    if (!instantiate) EFH_HIP(hipGraphLaunch(g, e->stream));
    done += k;
  }
  return EF_HIP_OK;
}

bool batched_prefill_enabled() {
  const char* v = std::getenv("EF_HIP_PREFILL");
  return v == nullptr || std::strcmp(v, "serial") != 0;
}

}  // namespace
void engine_set_owner(ef_hip_engine e, std::atomic<int>* refs) { e->owner_refs = refs; }
int launch_nll(const float* logits, int V, long ld, const int32_t* targets, int n, double* nll, hipStream_t s);

}  // namespace efh

using namespace efh;

extern "C" {

int ef_hip_engine_create(const ef_hip_model_config* cfg, const ef_hip_layer* layers, ef_hip_weight embed,
                         ef_hip_weight lm_head, const float* final_norm, size_t max_seq, int batch,
                         ef_hip_engine* out) {
  EFH_RC(require_ready());
  EFH_CHECK(cfg && layers && out && final_norm, "engine_create: null argument");
  const ef_hip_model_config& c = *cfg;
  EFH_CHECK(c.D > 0 && c.F > 0 && c.H > 0 && c.KV > 0 && c.hd > 0 && c.V > 0 && c.L > 0, "engine_create: zero dim");
  EFH_CHECK(c.H * c.hd == c.D && c.H % c.KV == 0 && c.hd % 4 == 0 && c.hd <= 256,
            "engine_create: need H*hd == D, H % KV == 0, hd a multiple of 4 up to 256");
  EFH_CHECK(max_seq > 0 && max_seq <= c.max_pos, "engine_create: max_seq must be in [1, max_position_embeddings]");
  EFH_CHECK(max_seq <= 12000 && attention_lds_bytes(static_cast<int>(c.hd), static_cast<int>(max_seq)) <=
                                    std::max<size_t>(ctx().lds_per_block, 65536),
            "engine_create: max_seq too large (attention scores and staged rows are held in LDS)");
  EFH_CHECK(batch >= 1 && batch <= 1024, "engine_create: batch must be in [1, 1024]");
  EFH_CHECK(c.V < 0x7FFFFFFF, "engine_create: vocab too large");
  const size_t kvd = c.KV * c.hd;
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = layers[l];
    EFH_RC(check_matrix(w.wq, c.D, c.D, "q_proj"));
    EFH_RC(check_matrix(w.wk, kvd, c.D, "k_proj"));
    EFH_RC(check_matrix(w.wv, kvd, c.D, "v_proj"));
    EFH_RC(check_matrix(w.wo, c.D, c.D, "o_proj"));
    EFH_RC(check_matrix(w.w_gate, c.F, c.D, "gate_proj"));
    EFH_RC(check_matrix(w.w_up, c.F, c.D, "up_proj"));
    EFH_RC(check_matrix(w.w_down, c.D, c.F, "down_proj"));
    EFH_CHECK(w.w_gate->qtype == w.w_up->qtype, "gate_proj and up_proj must share a storage type");
    EFH_CHECK(w.attn_norm_dev && w.ffn_norm_dev, "engine_create: null norm weights");
  }
  EFH_RC(check_matrix(lm_head, c.V, c.D, "lm_head"));
  EFH_RC(check_matrix(embed, c.V, c.D, "embed_tokens"));
  // Batched products (several sequences, or a prefill's positions) read packed matrices from a
  // tile-order copy; make them now, before any graph is captured.
  auto tile = [](ef_hip_weight w) {
    return w->qtype == EF_QTYPE_Q4_0 || w->qtype == EF_QTYPE_Q8_0 ? ensure_tiled(w, ctx().stream) : EF_HIP_OK;
  };
  for (size_t l = 0; l < c.L; ++l) {
    const ef_hip_layer& w = layers[l];
    for (ef_hip_weight m : {w.wq, w.wk, w.wv, w.wo, w.w_gate, w.w_up, w.w_down}) EFH_RC(tile(m));
  }
  EFH_RC(tile(lm_head));

  auto* e = new ef_hip_engine_s;
  e->c = c;
  e->layers.assign(layers, layers + c.L);
  e->embed = embed;
  e->lm_head = lm_head;
  e->final_norm = final_norm;
  e->max_seq = max_seq;
  e->kvd = kvd;
  e->B = batch;
  auto cleanup_fail = [&](int rc) {
    for (void* p : e->allocs) (void)hipFree(p);
    if (e->stage) (void)hipHostFree(e->stage);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
    return rc;
  };
  const size_t B = static_cast<size_t>(batch), S = max_seq;
  int rc = EF_HIP_OK;
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
    return cleanup_fail(fail(EF_HIP_ERUNTIME, "engine stream"));
  if ((rc = dev_alloc(e, &e->x, B * c.D)) || (rc = dev_alloc(e, &e->q, B * c.D)) ||
      (rc = dev_alloc(e, &e->knew, B * kvd)) || (rc = dev_alloc(e, &e->vnew, B * kvd)) ||
      (rc = dev_alloc(e, &e->ctx, B * c.D)) || (rc = dev_alloc(e, &e->act, B * c.F)) ||
      (rc = dev_alloc(e, &e->logits, B * c.V)) || (rc = dev_alloc(e, &e->hidden, B * c.D)) ||
      (rc = dev_alloc(e, &e->kc, c.L * B * S * kvd)) || (rc = dev_alloc(e, &e->vc, c.L * B * S * kvd)) ||
      (rc = dev_alloc(e, &e->cos_t, S * c.hd / 2)) || (rc = dev_alloc(e, &e->sin_t, S * c.hd / 2)) ||
      (rc = dev_alloc(e, &e->rope_now, c.hd)) ||
      (rc = dev_alloc(e, &e->hist, B * S)) || (rc = dev_alloc(e, &e->hist_len, B)) ||
      (rc = dev_alloc(e, &e->next_tok, B)) || (rc = dev_alloc(e, &e->pos, 1)) ||
      (rc = dev_alloc(e, &e->n_prompt, 1)) || (rc = dev_alloc(e, &e->out_tokens, B * S)) ||
      (rc = dev_alloc(e, &e->step_counter, 1)) || (rc = dev_alloc(e, &e->eos_cur, B)) ||
      (rc = dev_alloc(e, &e->eos_out, B * S)) || (rc = dev_alloc(e, &e->tok_dev, B * S + 8))) {
    return cleanup_fail(rc);
  }
  void* ws = nullptr;
  if (hipMalloc(&ws, sample_workspace_stride(static_cast<int>(c.V)) * B) != hipSuccess)
    return cleanup_fail(fail(EF_HIP_ENOMEM, "engine sampler workspace"));
  e->allocs.push_back(ws);
  e->sample_ws = ws;
  {
    int splits = 1, span = 0;
    size_t part = 0;
    if (attention_split_plan(static_cast<int>(c.H), static_cast<int>(c.KV), static_cast<int>(c.hd),
                             static_cast<int>(S), batch, &splits, &span, &part) &&
        !attention_uses_group(attn_args(e, false), batch)) {
      if ((rc = dev_alloc(e, &e->attn_part, part))) return cleanup_fail(rc);
      e->attn_splits = splits;
      e->attn_span = span;
    }
  }
  if (B > 1) {  // the largest workspace any of the step's batched GEMVs plans for
    size_t need = 0;
    for (size_t l = 0; l < c.L; ++l) {
      const ef_hip_layer& w = e->layers[l];
      const GemvJob qkv[3] = {{w.wq, nullptr, e->x, e->q, c.D, c.D},
                              {w.wk, nullptr, e->x, e->knew, c.D, kvd},
                              {w.wv, nullptr, e->x, e->vnew, c.D, kvd}};
      const GemvJob o{w.wo, nullptr, e->ctx, e->x, c.D, c.D};
      const GemvJob gu{w.w_gate, w.w_up, e->x, e->act, c.D, c.F};
      const GemvJob dn{w.w_down, nullptr, e->act, e->x, c.F, c.D};
      need = std::max({need, gemv_mfma_workspace_bytes(qkv, 3, kEpiStore, B, c.D),
                       gemv_mfma_workspace_bytes(&o, 1, kEpiResidual, B, c.D),
                       gemv_mfma_workspace_bytes(&gu, 1, kEpiSwiglu, B, c.D),
                       gemv_mfma_workspace_bytes(&dn, 1, kEpiResidual, B, c.F)});
    }
    const GemvJob lm{e->lm_head, nullptr, e->x, e->logits, c.D, c.V};
    need = std::max(need, gemv_mfma_workspace_bytes(&lm, 1, kEpiStore, B, c.D));
    if (need > 0) {
      void* gw = nullptr;
      if (hipMalloc(&gw, need) != hipSuccess) return cleanup_fail(fail(EF_HIP_ENOMEM, "engine GEMV workspace"));
      e->allocs.push_back(gw);
      e->gemv_ws = gw;
      e->gemv_ws_bytes = need;
    }
  }
  if (hipHostMalloc(reinterpret_cast<void**>(&e->stage), (B * S + 8) * sizeof(int32_t), hipHostMallocDefault) !=
      hipSuccess)
    return cleanup_fail(fail(EF_HIP_ENOMEM, "engine pinned staging"));
  // RoPE tables exactly as kern::RopeTable builds them (src/kernels.cpp:113-131): float pow / cos /
  // sin from the host C library, so the device sees the reference's bits.
  const size_t half = c.hd / 2;
  std::vector<float> inv(half), ct(S * half), st(S * half);
  for (size_t i = 0; i < half; ++i) {
    const float expo = static_cast<float>(2 * i) / static_cast<float>(c.hd);
    inv[i] = 1.0f / std::pow(c.rope_theta, expo);
  }
  for (size_t p = 0; p < S; ++p) {
    for (size_t i = 0; i < half; ++i) {
      const float ang = static_cast<float>(p) * inv[i];
      ct[p * half + i] = std::cos(ang);
      st[p * half + i] = std::sin(ang);
    }
  }
  hipError_t he = hipMemcpyAsync(e->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice, e->stream);
  if (he == hipSuccess) he = hipMemcpyAsync(e->sin_t, st.data(), st.size() * 4, hipMemcpyHostToDevice, e->stream);
  if (he == hipSuccess) he = hipMemsetAsync(e->kc, 0, c.L * B * S * kvd * 4, e->stream);
  if (he == hipSuccess) he = hipMemsetAsync(e->vc, 0, c.L * B * S * kvd * 4, e->stream);
  if (he == hipSuccess) he = hipMemsetAsync(e->hist, 0, B * S * 4, e->stream);
  if (he == hipSuccess) he = hipMemsetAsync(e->pos, 0, 4, e->stream);
  if (he == hipSuccess) he = hipMemsetAsync(e->step_counter, 0, 4, e->stream);
  if (he == hipSuccess) he = hipStreamSynchronize(e->stream);
  if (he != hipSuccess) return cleanup_fail(fail_hip(he, "engine init"));
  if ((rc = build_staged(e)) != EF_HIP_OK) return cleanup_fail(rc);
  e->magic = kEngineMagic;
  *out = e;
  return EF_HIP_OK;
}

int ef_hip_engine_destroy(ef_hip_engine e) {
  EFH_RC(check_engine(e));
  e->magic = 0;
  (void)hipStreamSynchronize(e->stream);
  for (auto& kv : e->graphs) (void)hipGraphExecDestroy(kv.second);
  for (hipGraphExec_t g : e->retired) (void)hipGraphExecDestroy(g);
  for (void* p : e->allocs) (void)hipFree(p);
  for (float* p : {e->pf_x, e->pf_q, e->pf_k, e->pf_v, e->pf_ctx, e->pf_act})
    if (p) (void)hipFree(p);
  if (e->pf_ws) (void)hipFree(e->pf_ws);
  if (e->pf_logits) (void)hipFree(e->pf_logits);
  if (e->stage) (void)hipHostFree(e->stage);
  (void)hipStreamDestroy(e->stream);
  if (e->owner_refs != nullptr) e->owner_refs->fetch_sub(1);
  delete e;
  return EF_HIP_OK;
}

int ef_hip_engine_forward(ef_hip_engine e, const int32_t* tokens, size_t pos, int compute_logits) {
  EFH_RC(check_engine(e));
  EFH_CHECK(tokens != nullptr, "engine_forward: null tokens");
  for (int b = 0; b < e->B; ++b) {  // src/model.cpp:185-195
    if (tokens[b] < 0 || static_cast<size_t>(tokens[b]) >= e->c.V)
      return fail(EF_HIP_EINVAL, "forward: token id " + std::to_string(tokens[b]) + " is outside [0, " +
                                     std::to_string(e->c.V) + ")");
  }
  if (pos >= e->max_seq)
    return fail(EF_HIP_EINVAL, "forward: position " + std::to_string(pos) + " exceeds the KV-cache capacity " +
                                   std::to_string(e->max_seq));
  if (pos > e->cached)
    return fail(EF_HIP_EINVAL, "forward: position " + std::to_string(pos) + " skips ahead of the " +
                                   std::to_string(e->cached) + " cached tokens");
  EFH_HIP(hipStreamSynchronize(e->stream));  // the pinned staging buffer is reused below
  for (int b = 0; b < e->B; ++b) e->stage[b] = tokens[b];
  e->stage[e->B] = static_cast<int32_t>(pos);
  EFH_RC(put_tokens(e, pos, 1));
  EFH_HIP(hipMemcpyAsync(e->pos, e->tok_dev + e->B, 4, hipMemcpyDeviceToDevice, e->stream));
  EFH_RC(run_step(e, at_pos(e, compute_logits ? kLogits : 0, pos)));
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->cached = pos + 1;
  return EF_HIP_OK;
}

int ef_hip_engine_prefill(ef_hip_engine e, const int32_t* tokens, size_t n, size_t pos, int compute_logits) {
  EFH_RC(check_engine(e));
  EFH_CHECK(tokens != nullptr && n >= 1, "engine_prefill: null tokens or n = 0");
  for (size_t i = 0; i < n * static_cast<size_t>(e->B); ++i) {
    if (tokens[i] < 0 || static_cast<size_t>(tokens[i]) >= e->c.V)
      return fail(EF_HIP_EINVAL, "prefill: token id " + std::to_string(tokens[i]) + " is outside [0, " +
                                     std::to_string(e->c.V) + ")");
  }
  if (pos + n > e->max_seq)
    return fail(EF_HIP_EINVAL, "prefill: positions up to " + std::to_string(pos + n - 1) +
                                   " exceed the KV-cache capacity " + std::to_string(e->max_seq));
  if (pos > e->cached)
    return fail(EF_HIP_EINVAL, "prefill: position " + std::to_string(pos) + " skips ahead of the " +
                                   std::to_string(e->cached) + " cached tokens");
  const int B = e->B;
  EFH_HIP(hipStreamSynchronize(e->stream));  // the pinned staging buffer is reused below
  for (size_t i = 0; i < n * static_cast<size_t>(B); ++i) e->stage[i] = tokens[i];
  EFH_RC(put_tokens(e, pos, n));
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->stage[0] = static_cast<int32_t>(pos);
  EFH_HIP(hipMemcpyAsync(e->pos, e->stage, 4, hipMemcpyHostToDevice, e->stream));
  EFH_RC(run_prefill(e, n, compute_logits ? kLogits : 0, false));
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->cached = pos + n;
  return EF_HIP_OK;
}

int ef_hip_engine_logits(ef_hip_engine e, const float** logits) {
  EFH_RC(check_engine(e));
  EFH_CHECK(logits != nullptr, "engine_logits: null out pointer");
  *logits = e->logits;
  return EF_HIP_OK;
}

int ef_hip_engine_hidden(ef_hip_engine e, const float** hidden) {
  EFH_RC(check_engine(e));
  EFH_CHECK(hidden != nullptr, "engine_hidden: null out pointer");
  EFH_RC(launch_rmsnorm(e->x, e->final_norm, e->c.eps, static_cast<int>(e->c.D), static_cast<long>(e->c.D), e->B,
                        e->hidden, e->stream));
  EFH_HIP(hipStreamSynchronize(e->stream));
  *hidden = e->hidden;
  return EF_HIP_OK;
}

int ef_hip_engine_generate(ef_hip_engine e, const int32_t* prompt, size_t n_prompt, size_t n,
                           const ef_hip_sampler_config* cfg, void* rng, int32_t* tokens_out, double* prefill_s,
                           double* decode_s) {
  EFH_RC(check_engine(e));
  EFH_CHECK(prompt && tokens_out, "engine_generate: null argument");
  if (n_prompt == 0) return fail(EF_HIP_EINVAL, "generate: empty prompt");  // src/model.cpp:280
  EFH_CHECK(n >= 1, "generate: n must be >= 1");
  if (n_prompt + n > e->max_seq)
    return fail(EF_HIP_EINVAL, "generate: prompt (" + std::to_string(n_prompt) + ") + max_new (" + std::to_string(n) +
                                   ") exceeds the KV-cache capacity " + std::to_string(e->max_seq));
  const int B = e->B;
  const size_t S = e->max_seq;
  for (size_t i = 0; i < n_prompt * B; ++i) {
    if (prompt[i] < 0 || static_cast<size_t>(prompt[i]) >= e->c.V)
      return fail(EF_HIP_EINVAL, "generate: prompt token " + std::to_string(prompt[i]) + " out of range");
  }
  int pick = kGreedy;
  if (cfg != nullptr) {
    EFH_CHECK(cfg->temperature <= 0.0f || rng != nullptr, "generate: sampling needs rng states");
    EFH_RC(set_sampler(e, *cfg, rng));
    pick = kSample;
  }
  // history <- prompt, hist_len <- n_prompt, position 0
  EFH_HIP(hipStreamSynchronize(e->stream));  // the pinned staging buffer is reused below
  for (int b = 0; b < B; ++b) {
    for (size_t p = 0; p < n_prompt; ++p) e->stage[b * n_prompt + p] = prompt[b * n_prompt + p];
  }
  EFH_RC(put_tokens(e, 0, n_prompt));
  EFH_HIP(hipStreamSynchronize(e->stream));
  for (int b = 0; b < B; ++b) e->stage[b] = static_cast<int32_t>(n_prompt);
  e->stage[B] = 0;
  e->stage[B + 1] = static_cast<int32_t>(n_prompt);
  EFH_HIP(hipMemcpyAsync(e->hist_len, e->stage, B * 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipMemcpyAsync(e->pos, e->stage + B, 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipMemcpyAsync(e->n_prompt, e->stage + B + 1, 4, hipMemcpyHostToDevice, e->stream));
  // The prompt: one batched prefill (every prompt position of every sequence through each
  // product at once) or, with EF_HIP_PREFILL=serial, the reference's one position at a time
  // (src/model.cpp:290).  Graphs are instantiated before the clock starts.
  const bool batched = n_prompt >= 2 && batched_prefill_enabled();
  // step graphs for positions below and from kSplitFrom (the same graph when the engine does not
  // split), instantiated before the clock starts
  hipGraphExec_t g_pre[2] = {nullptr, nullptr}, g_dec[2];
  if (batched) {
    EFH_RC(run_prefill(e, n_prompt, kLogits | pick, true));
  } else {
    EFH_RC(graph_for(e, kAdvance, &g_pre[0]));
    EFH_RC(graph_for(e, at_pos(e, kAdvance, S), &g_pre[1]));
  }
  EFH_RC(graph_for(e, kLogits | pick, &g_dec[0]));
  EFH_RC(graph_for(e, at_pos(e, kLogits | pick, S), &g_dec[1]));
  auto pre_at = [&](size_t p) { return g_pre[at_pos(e, 0, p) != 0]; };
  auto dec_at = [&](size_t p) { return g_dec[at_pos(e, 0, p) != 0]; };
  EFH_HIP(hipStreamSynchronize(e->stream));
  using Clock = std::chrono::steady_clock;
  const auto t0 = Clock::now();
  if (batched) {
    EFH_RC(run_prefill(e, n_prompt, kLogits | pick, false));  // ends with logits and the first pick
  } else {
    for (size_t p = 0; p + 1 < n_prompt; ++p) EFH_HIP(hipGraphLaunch(pre_at(p), e->stream));
    EFH_HIP(hipGraphLaunch(dec_at(n_prompt - 1), e->stream));  // last prompt position: logits and the first pick
  }
  EFH_HIP(hipStreamSynchronize(e->stream));
  const auto t1 = Clock::now();
  for (size_t k = 1; k < n; ++k) EFH_HIP(hipGraphLaunch(dec_at(n_prompt - 1 + k), e->stream));
  EFH_HIP(hipStreamSynchronize(e->stream));
  const auto t2 = Clock::now();
  // [B][S] -> [B][n] on the device, then one contiguous copy to the caller
  EFH_RC(launch_copy_rows(e->out_tokens, static_cast<long>(S), e->tok_dev, static_cast<long>(n), static_cast<int>(n),
                          B, e->stream));
  EFH_HIP(hipMemcpyAsync(tokens_out, e->tok_dev, n * B * 4, hipMemcpyDeviceToHost, e->stream));
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->cached = n_prompt + n - 1;
  e->chat_ids.clear();
  if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
  if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
  return EF_HIP_OK;
}

int ef_hip_engine_profile(ef_hip_engine e, const ef_hip_sampler_config* cfg, void* rng, int reps, double* ms_out) {
  EFH_RC(check_engine(e));
  EFH_CHECK(ms_out != nullptr && reps >= 1 && reps <= 100000, "engine_profile: null output or reps not in [1, 1e5]");
  EFH_CHECK(e->cached >= 1, "engine_profile: no cached position (run forward, prefill or generate first)");
  int pick = kGreedy;
  if (cfg != nullptr && cfg->temperature > 0.0f) {
    EFH_CHECK(rng != nullptr, "engine_profile: sampling needs rng states");
    EFH_RC(set_sampler(e, *cfg, rng));
    pick = kSample;
  }
  // every group runs at position P (its token and cache rows are in bounds); only the pick group
  // moves the position, and it is put back after each group
  const int32_t P = static_cast<int32_t>(std::min(e->cached, e->max_seq - 1));
  const int mode = at_pos(e, kLogits | pick, static_cast<size_t>(P));
  auto set_pos = [&]() -> int {
    EFH_HIP(hipStreamSynchronize(e->stream));
    e->stage[0] = P;
    EFH_HIP(hipMemcpyAsync(e->pos, e->stage, 4, hipMemcpyHostToDevice, e->stream));
    EFH_HIP(hipStreamSynchronize(e->stream));
    return EF_HIP_OK;
  };
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  EFH_HIP(hipEventCreate(&ev0));
  if (hipEventCreate(&ev1) != hipSuccess) {
    (void)hipEventDestroy(ev0);
    return fail(EF_HIP_ERUNTIME, "engine_profile: hipEventCreate");
  }
  int rc = EF_HIP_OK;
  for (int g = 0; g < EF_HIP_PROF_GROUPS && rc == EF_HIP_OK; ++g) {
    hipGraphExec_t ex = nullptr;
    rc = set_pos();
    if (rc != EF_HIP_OK) break;
    if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
      rc = fail(EF_HIP_ERUNTIME, "engine_profile: hipStreamBeginCapture");
      break;
    }
    // the group's launches kInGraph times in one graph, so one graph launch's host-side cost is
    // spread over as many steps' worth of work (a step graph pays it once per step)
    constexpr int kInGraph = 8;
    for (int k = 0; k < kInGraph && rc == EF_HIP_OK; ++k) rc = enqueue_step(e, mode, 1u << g);
    hipGraph_t gr = nullptr;
    const hipError_t ec = hipStreamEndCapture(e->stream, &gr);
    if (rc == EF_HIP_OK && ec != hipSuccess) rc = fail_hip(ec, "hipStreamEndCapture");
    if (rc == EF_HIP_OK) {
      const hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
      if (ei != hipSuccess) rc = fail_hip(ei, "hipGraphInstantiate");
    }
    if (gr) (void)hipGraphDestroy(gr);
    float ms = 0.0f;
    if (rc == EF_HIP_OK) {
      hipError_t he = hipSuccess;
      for (int w = 0; w < 3 && he == hipSuccess; ++w) he = hipGraphLaunch(ex, e->stream);  // warm-up
      if (he == hipSuccess) he = hipEventRecord(ev0, e->stream);
      for (int r = 0; r < reps && he == hipSuccess; ++r) he = hipGraphLaunch(ex, e->stream);
      if (he == hipSuccess) he = hipEventRecord(ev1, e->stream);
      if (he == hipSuccess) he = hipEventSynchronize(ev1);
      if (he == hipSuccess) he = hipEventElapsedTime(&ms, ev0, ev1);
      if (he != hipSuccess) rc = fail_hip(he, "engine_profile: timed launches");
    }
    if (ex) e->retired.push_back(ex);
    ms_out[g] = static_cast<double>(ms) / (static_cast<double>(reps) * kInGraph);
  }
  (void)hipEventDestroy(ev0);
  (void)hipEventDestroy(ev1);
  if (rc == EF_HIP_OK) rc = set_pos();
  e->chat_ids.clear();
  return rc;
}

int ef_hip_engine_tables(ef_hip_engine e, int* on, const char** why) {
  EFH_RC(check_engine(e));
  EFH_CHECK(on != nullptr, "engine_tables: null output");
  *on = e->staged ? 1 : 0;
  if (why != nullptr) *why = e->staged_why.c_str();
  return EF_HIP_OK;
}

int ef_hip_engine_reset(ef_hip_engine e) {
  EFH_RC(check_engine(e));
  e->chat_ids.clear();
  e->cached = 0;
  return EF_HIP_OK;
}

int ef_hip_engine_score(ef_hip_engine e, const int32_t* ids, size_t n, size_t first, double* nll_host,
                        float* logits_dev) {
  EFH_RC(check_engine(e));
  EFH_CHECK(ids && nll_host, "engine_score: null argument");
  EFH_CHECK(e->B == 1, "engine_score: scores one sequence (engine batch 1)");
  EFH_CHECK(n >= 2 && first + 1 < n, "engine_score: need n >= 2 and first < n - 1");
  EFH_CHECK(n - 1 <= e->max_seq, "engine_score: sequence longer than the KV cache");
  for (size_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || static_cast<size_t>(ids[i]) >= e->c.V)
      return fail(EF_HIP_EINVAL, "score: token id " + std::to_string(ids[i]) + " out of range");
  }
  const size_t V = e->c.V, m = n - 1;
  size_t rows = 1024;  // [rows][V] logits per launch: 128 MB at V = 32000
  if (const char* v = std::getenv("EF_HIP_PREFILL_ROWS"))  // test knob: smaller launches
    rows = std::min<size_t>(rows, static_cast<size_t>(std::max<long>(1, std::atol(v))));
  const size_t chunk = std::min(rows, m);
  EFH_RC(ensure_prefill(e, chunk));
  if (e->pf_logit_rows < chunk) {
    if (e->pf_logits) (void)hipFree(e->pf_logits);
    e->pf_logits = nullptr;
    e->pf_logit_rows = 0;
    EFH_RC(drop_graphs_with(e, kAllLogits));
    EFH_HIP(hipMalloc(&e->pf_logits, chunk * V * sizeof(float)));
    e->pf_logit_rows = chunk;
  }
  int32_t* targets = nullptr;
  double* nll = nullptr;
  EFH_HIP(hipMallocAsync(reinterpret_cast<void**>(&targets), n * sizeof(int32_t), e->stream));
  EFH_HIP(hipMallocAsync(reinterpret_cast<void**>(&nll), n * sizeof(double), e->stream));
  EFH_HIP(hipStreamSynchronize(e->stream));
  for (size_t i = 0; i < n; ++i) e->stage[i] = ids[i];
  EFH_HIP(hipMemcpyAsync(e->hist, e->stage, n * 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipMemcpyAsync(targets, e->stage, n * 4, hipMemcpyHostToDevice, e->stream));
  int rc = EF_HIP_OK;
  for (size_t c0 = 0; c0 < m && rc == EF_HIP_OK; c0 += chunk) {
    const size_t k = std::min(chunk, m - c0);
    EFH_HIP(hipStreamSynchronize(e->stream));  // the pinned slot below is reused per chunk
    e->stage[n] = static_cast<int32_t>(c0);
    EFH_HIP(hipMemcpyAsync(e->pos, e->stage + n, 4, hipMemcpyHostToDevice, e->stream));
    rc = run_step(e, kPrefill | kAllLogits | static_cast<int>(k << 8));
    if (rc != EF_HIP_OK) break;
    // rows of this chunk at positions >= first: targets are the next ids
    const size_t lo = std::max(first, c0), hi = c0 + k;
    if (lo < hi) {
      rc = launch_nll(e->pf_logits + (lo - c0) * V, static_cast<int>(V), static_cast<long>(V), targets + lo + 1,
                      static_cast<int>(hi - lo), nll + (lo - first), e->stream);
      if (rc == EF_HIP_OK && logits_dev != nullptr &&
          hipMemcpyAsync(logits_dev + (lo - first) * V, e->pf_logits + (lo - c0) * V, (hi - lo) * V * sizeof(float),
                         hipMemcpyDeviceToDevice, e->stream) != hipSuccess)
        rc = fail(EF_HIP_ERUNTIME, "score: logits copy");
    }
  }
  if (rc == EF_HIP_OK &&
      hipMemcpyAsync(nll_host, nll, (m - first) * sizeof(double), hipMemcpyDeviceToHost, e->stream) != hipSuccess)
    rc = fail(EF_HIP_ERUNTIME, "score: nll copy");
  (void)hipFreeAsync(targets, e->stream);
  (void)hipFreeAsync(nll, e->stream);
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->cached = std::max(e->cached, m);
  e->chat_ids.clear();
  return rc;
}

// The token-level loop of ChatSession::reply (src/chat.cpp:174-259): reuse of the cached prefix
// (longest common prefix with the ids whose K / V the cache holds, at least the last prompt token
// recomputed), batched prefill of the rest, then sample / P(EOS) / stop checks per step.  Steps
// run on the device in windows of steps_per_check graph launches; the host then applies the
// reference's stop checks to the window's tokens in order.  Steps launched past a stop only write
// cache positions the next turn recomputes, and the RNG states are restored to the window's start
// and advanced by the draws the reference makes (one per sampled step), so a conversation samples
// the same ids as the reference's Sampler.
int ef_hip_engine_reply(ef_hip_engine e, const int32_t* ids, size_t n_ids, const ef_hip_sampler_config* cfg,
                        void* rng, const ef_hip_reply_options* o, int32_t* reply_out, double* eos_p_out,
                        ef_hip_reply_stats* st) {
  EFH_RC(check_engine(e));
  EFH_CHECK(ids && cfg && o && reply_out, "engine_reply: null argument");
  EFH_CHECK(e->B == 1, "engine_reply: a chat session is one sequence (engine batch 1)");
  EFH_CHECK(n_ids >= 1, "engine_reply: empty prompt");
  EFH_CHECK(o->max_new > 0, "chat: max_new must be > 0");
  const size_t S = e->max_seq;
  if (n_ids >= S)
    return fail(EF_HIP_EINVAL, "message is too long for the " + std::to_string(S) + "-token context");
  for (size_t i = 0; i < n_ids; ++i) {
    if (ids[i] < 0 || static_cast<size_t>(ids[i]) >= e->c.V)
      return fail(EF_HIP_EINVAL, "reply: token id " + std::to_string(ids[i]) + " out of range");
  }
  const bool sampled = cfg->temperature > 0.0f;
  EFH_CHECK(!sampled || rng != nullptr, "engine_reply: sampling needs rng states");
  EFH_RC(set_sampler(e, *cfg, rng));
  if (e->eos_id != o->eos_id) {
    EFH_RC(drop_graphs_with(e, kEos));
    e->eos_id = o->eos_id;
  }
  if (sampled && e->rng_snap == nullptr) EFH_RC(dev_alloc(e, reinterpret_cast<uint8_t**>(&e->rng_snap), kRngStateBytes));
  ef_hip_reply_stats r{};
  r.prompt_tokens = n_ids;
  size_t lcp = 0;
  while (lcp < e->chat_ids.size() && lcp < n_ids && e->chat_ids[lcp] == ids[lcp]) ++lcp;
  if (lcp == n_ids) --lcp;
  lcp = std::min(lcp, e->cached);
  r.reused_tokens = lcp;
  r.prefill_tokens = n_ids - lcp;
  // history <- ids, hist_len <- n_ids, n_prompt <- n_ids, position <- lcp
  EFH_HIP(hipStreamSynchronize(e->stream));
  for (size_t i = 0; i < n_ids; ++i) e->stage[i] = ids[i];
  EFH_HIP(hipMemcpyAsync(e->hist, e->stage, n_ids * 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipStreamSynchronize(e->stream));
  e->stage[0] = static_cast<int32_t>(n_ids);
  e->stage[1] = static_cast<int32_t>(lcp);
  EFH_HIP(hipMemcpyAsync(e->hist_len, e->stage, 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipMemcpyAsync(e->n_prompt, e->stage, 4, hipMemcpyHostToDevice, e->stream));
  EFH_HIP(hipMemcpyAsync(e->pos, e->stage + 1, 4, hipMemcpyHostToDevice, e->stream));
  const int mode = kLogits | kSample | kEos;
  const size_t n_pre = n_ids - lcp;
  const bool batched = n_pre >= 2 && batched_prefill_enabled();
  hipGraphExec_t g_dec[2];
  if (batched) EFH_RC(run_prefill(e, n_pre, mode, true));
  EFH_RC(graph_for(e, mode, &g_dec[0]));
  EFH_RC(graph_for(e, at_pos(e, mode, S), &g_dec[1]));
  auto dec_at = [&](size_t p) { return g_dec[at_pos(e, 0, p) != 0]; };
  const size_t max_new = std::min(o->max_new, S - n_ids);
  const size_t window = static_cast<size_t>(std::max(1, o->steps_per_check));
  std::vector<int32_t> toks(max_new);
  std::vector<double> peos(max_new);
  auto snapshot = [&]() -> int {
    if (sampled) EFH_HIP(hipMemcpyAsync(e->rng_snap, rng, kRngStateBytes, hipMemcpyDeviceToDevice, e->stream));
    return EF_HIP_OK;
  };
  using Clock = std::chrono::steady_clock;
  EFH_HIP(hipStreamSynchronize(e->stream));
  const auto t0 = Clock::now();
  EFH_RC(snapshot());
  if (batched) {
    EFH_RC(run_prefill(e, n_pre, mode, false));  // ends with the first pick
  } else {
    for (size_t p = lcp; p + 1 < n_ids; ++p) EFH_RC(run_step(e, at_pos(e, kAdvance, p)));
    EFH_HIP(hipGraphLaunch(dec_at(n_ids - 1), e->stream));
  }
  EFH_HIP(hipStreamSynchronize(e->stream));
  const auto t1 = Clock::now();
  size_t picks = 1, w0 = 0, steps = 0, generated = 0, forwarded = 0;
  int reason = 0;
  while (reason == 0) {
    const size_t w1 = std::min(max_new, w0 + window);
    for (; picks < w1; ++picks) EFH_HIP(hipGraphLaunch(dec_at(n_ids - 1 + picks), e->stream));
    EFH_HIP(hipMemcpyAsync(toks.data() + w0, e->out_tokens + w0, (w1 - w0) * 4, hipMemcpyDeviceToHost, e->stream));
    EFH_HIP(hipMemcpyAsync(peos.data() + w0, e->eos_out + w0, (w1 - w0) * 8, hipMemcpyDeviceToHost, e->stream));
    EFH_HIP(hipStreamSynchronize(e->stream));
    for (size_t k = w0; k < w1 && reason == 0; ++k) {  // src/chat.cpp:220-246
      steps = k + 1;
      if (peos[k] > r.eos_p_max) {
        r.eos_p_max = peos[k];
        r.eos_p_max_step = k;
      }
      if (toks[k] == o->eos_id) {
        reason = EF_HIP_STOP_EOS;
      } else if (o->eos_min_p > 0.0f && peos[k] >= static_cast<double>(o->eos_min_p)) {
        reason = EF_HIP_STOP_EOS_MIN_P;
      } else {
        reply_out[generated++] = toks[k];
        if (k + 1 == max_new) {
          reason = max_new < o->max_new ? EF_HIP_STOP_CONTEXT : EF_HIP_STOP_MAX_NEW;
        } else {
          ++forwarded;
        }
      }
    }
    if (reason != 0 && sampled && steps < w1) {  // steps w0 .. steps-1 happened in the reference
      EFH_HIP(hipMemcpyAsync(rng, e->rng_snap, kRngStateBytes, hipMemcpyDeviceToDevice, e->stream));
      EFH_RC(launch_rng_discard(rng, 1, static_cast<int>(steps - w0), e->stream));
    }
    w0 = w1;
    if (reason == 0) EFH_RC(snapshot());
  }
  EFH_HIP(hipStreamSynchronize(e->stream));
  const auto t2 = Clock::now();
  if (eos_p_out != nullptr) std::copy(peos.begin(), peos.begin() + steps, eos_p_out);
  e->chat_ids.assign(ids, ids + n_ids);
  e->chat_ids.insert(e->chat_ids.end(), reply_out, reply_out + forwarded);
  e->cached = e->chat_ids.size();
  r.generated = generated;
  r.steps = steps;
  r.reason = reason;
  r.prefill_s = std::chrono::duration<double>(t1 - t0).count();
  r.decode_s = std::chrono::duration<double>(t2 - t1).count();
  if (st != nullptr) *st = r;
  return EF_HIP_OK;
}

}  // extern "C"
