/* EdgeForge on MI355X: C-ABI of the HIP quantized-decode hot path (libedgeforge_hip.so).
 *
 * Plain C types only (pointers, sizes, ints).  Every entry point returns an int status: 0 is OK,
 * negative values are the EF_HIP_E* codes below, and ef_hip_last_error() gives the message of the
 * calling thread's last failure.  Device pointers ("*_dev") are HIP device addresses on the
 * current device; "stream" is a hipStream_t (NULL = the library's default stream of the device).
 *
 * Each declaration names the reference interface it replaces (paths relative to the EdgeForge
 * repository root).  The C++ signatures of the reference are kept one level up, by the host shim
 * in edgeforge_amd/host (ef::kern::matvec / matvec_jobs, ef::Sampler), which calls these.
 */
#ifndef EF_HIP_H
#define EF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------------- */
#define EF_HIP_OK 0
#define EF_HIP_EINVAL (-1)  /* bad argument: shape, type, null pointer, size limit             */
#define EF_HIP_ERUNTIME (-2) /* a HIP runtime call failed                                      */
#define EF_HIP_ENODEV (-3)  /* no usable gfx950 device                                          */
#define EF_HIP_ENOMEM (-4)  /* device allocation failed                                         */
#define EF_HIP_ESTATE (-5)  /* library not initialised / handle already released                */

/* Storage types, numbered as ef::QType (include/ef/quant.h:35). */
#define EF_QTYPE_F32 0
#define EF_QTYPE_F16 1
#define EF_QTYPE_BF16 2
#define EF_QTYPE_Q8_0 3
#define EF_QTYPE_Q4_0 4

/* ---- context (no reference counterpart: the reference is CPU-only; these replace the process-global
 *      backend switch kern::set_backend, src/qkernels.cpp:80-99) ------------------------------ */
int ef_hip_init(int device);
int ef_hip_shutdown(void);
const char* ef_hip_last_error(void);
int ef_hip_device_name(char* buf, size_t cap);
int ef_hip_version(int* major, int* minor);

/* ---- device memory and streams (plumbing for callers without their own allocator) ----------- */
int ef_hip_malloc(void** dev, size_t bytes);
int ef_hip_free(void* dev);
int ef_hip_memcpy_h2d(void* dst_dev, const void* src_host, size_t bytes, void* stream);
int ef_hip_memcpy_d2h(void* dst_host, const void* src_dev, size_t bytes, void* stream);
int ef_hip_memcpy_d2d(void* dst_dev, const void* src_dev, size_t bytes, void* stream);
int ef_hip_memset(void* dev, int value, size_t bytes, void* stream);
int ef_hip_stream_create(void** stream);
int ef_hip_stream_destroy(void* stream);
int ef_hip_stream_sync(void* stream);
/* *kind = 1 when p is device memory, 2 for pinned host memory, 0 otherwise (pageable host). */
int ef_hip_pointer_kind(const void* p, int* kind);
/* HIP events, for timing kernels on the stream they run on. */
int ef_hip_event_create(void** ev);
int ef_hip_event_destroy(void* ev);
int ef_hip_event_record(void* ev, void* stream);
int ef_hip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---- weights ----------------------------------------------------------------------------------
 * Replaces ef::WeightView (include/ef/qkernels.h:28-34): a row-major [rows][cols] matrix in one of
 * the storage types above (row bytes as src/quant.cpp:136-149; Q4_0/Q8_0 need cols % 32 == 0).
 * register_host uploads the bytes once; register_device wraps device bytes the caller owns (no
 * copy).  The handle is what the GEMV entry points take.
 * Batched products (batch >= 2) of a Q4_0 / Q8_0 handle read a tile-order copy of its bytes, made
 * on the handle's first batched call (or at engine creation) and freed with the handle; batch 1
 * reads the bytes in place.  A caller that rewrites a handle's bytes after its first batched use
 * (ef_hip_quantize into the same buffer, a copy) calls ef_hip_weight_refresh, which rewrites the
 * copy in place on `stream`, stream-ordered after the write, without allocating (graphs captured
 * over the handle stay valid); without it batched products keep using the former bytes. */
typedef struct ef_hip_weight_s* ef_hip_weight;
int ef_hip_weight_register_host(const void* host_bytes, int qtype, size_t rows, size_t cols, ef_hip_weight* out);
int ef_hip_weight_register_device(const void* dev_bytes, int qtype, size_t rows, size_t cols, ef_hip_weight* out);
int ef_hip_weight_release(ef_hip_weight w);
int ef_hip_weight_refresh(ef_hip_weight w, void* stream);
int ef_hip_weight_info(ef_hip_weight w, int* qtype, size_t* rows, size_t* cols, const void** dev_bytes);
int ef_hip_row_bytes(int qtype, size_t cols, size_t* out); /* src/quant.cpp:136-149 */

/* ---- GEMV ------------------------------------------------------------------------------------
 * y[b][r] = sum_c W[r][c] * x[b][c] for b < batch, r < rows (FP32 activations, FP32 result).
 * Replaces kern::matvec (include/ef/qkernels.h:66, src/qkernels.cpp:275-278) and, with batch > 1,
 * the loop over independent sequences the reference would run.  ldx / ldy are the row strides
 * (in floats) of x and y.  All five storage types, as kern::matvec_rows (src/qkernels.cpp:213-269):
 * Q4_0 / Q8_0 read the 18 / 34-byte blocks (in place at batch 1, from the handle's tile-order copy
 * at batch >= 2; cols % 32 == 0, cols <= 14336); F32 / F16 /
 * BF16 rows take any cols up to 16320.  Results agree with
 * the reference's FP32 kernels to the rounding of a different summation order (the dot products
 * are reproducible: the same inputs give the same bits on every call). */
int ef_hip_matvec(ef_hip_weight W, const float* x_dev, float* y_dev, int batch, size_t ldx, size_t ldy, void* stream);

/* Several products in one launch, one per job (kern::matvec_jobs + kern::MatvecJob,
 * include/ef/qkernels.h:70-75, src/qkernels.cpp:280-297).  Each job has its own x / y; every job's
 * rows are computed exactly as ef_hip_matvec would. */
typedef struct {
  float* y_dev;
  ef_hip_weight W;
  const float* x_dev;
} ef_hip_job;
int ef_hip_matvec_jobs(const ef_hip_job* jobs, size_t n_jobs, int batch, size_t ldx, size_t ldy, void* stream);

/* Fused epilogues of the products Transformer::forward chains (src/model.cpp:227-262):
 *  - residual:  y += W x            (matvec + kern::add_inplace, model.cpp:247-249, 260-262)
 *  - swiglu:    y  = silu(G x) * (U x)  (matvec_jobs{gate,up} + kern::swiglu, model.cpp:255-258)
 *  - rmsnorm on the input: x' = w * (x * rsqrt(mean(x^2) + eps)) computed per launch before the
 *    product (kern::rmsnorm, src/kernels.cpp:69-75, model.cpp:227,253,269).  norm_w_dev NULL = off. */
int ef_hip_matvec_residual(ef_hip_weight W, const float* x_dev, float* y_dev, int batch, size_t ldx, size_t ldy,
                           void* stream);
int ef_hip_matvec_swiglu(ef_hip_weight G, ef_hip_weight U, const float* x_dev, const float* norm_w_dev, float eps,
                         float* y_dev, int batch, size_t ldx, size_t ldy, void* stream);
int ef_hip_matvec_jobs_rmsnorm(const ef_hip_job* jobs, size_t n_jobs, const float* norm_w_dev, float eps, int batch,
                               size_t ldx, size_t ldy, void* stream);

/* Row r of W as FP32 (kern::row_f32, include/ef/qkernels.h:78): exact for F32/F16/BF16,
 * dequantized for Q4_0/Q8_0.  One row per batch entry, ids on the device. */
int ef_hip_rows_f32(ef_hip_weight W, const int32_t* ids_dev, int batch, float* out_dev, size_t ldo, void* stream);

/* ---- quantizer (src/quant.cpp:26-99 q4_group, :151-175) ----------------------------------------
 * Packs a row-major FP32 [rows][cols] matrix on the device into Q4_0 / Q8_0 / BF16 / F16 / F32
 * rows; byte-identical to the reference's quantize_row (search = the reference's Q4 scale search). */
int ef_hip_quantize(int qtype, const float* w_dev, size_t rows, size_t cols, int search, void* out_dev, void* stream);

/* ---- synthetic inputs (no reference counterpart: the reference reads real checkpoints) -------
 * out[i] = mean + scale * z_i, z_i ~ N(0,1) from Philox4x32-10 and Box-Muller; deterministic in
 * (seed, offset, i).  Builds the benchmark's random-init weights and activations on the device. */
int ef_hip_fill_normal(float* out_dev, size_t n, uint64_t seed, uint64_t offset, float mean, float scale,
                       void* stream);

/* ---- sampler ----------------------------------------------------------------------------------
 * ef::SamplerConfig (include/ef/sampler.h:13-19) and Sampler::sample (src/sampler.cpp:13-70) for
 * `batch` independent sequences: logits [batch][ld] on the device; history [batch][hist_ld] int32
 * with hist_len[batch] valid entries (device); one std::mt19937_64 state per sequence in rng_dev
 * (created by ef_hip_rng_seed), advanced by one draw exactly when temperature > 0, as the
 * reference does.  Token ids are bit-identical to the reference's on identical logits. */
typedef struct {
  float temperature;
  int top_k;
  float top_p;
  float repetition_penalty;
  uint64_t seed;
} ef_hip_sampler_config;
size_t ef_hip_rng_state_bytes(void); /* per sequence */
int ef_hip_rng_seed(void* rng_dev, const uint64_t* seeds_host, int batch, void* stream);
/* ws_dev: ef_hip_sample_workspace_bytes(vocab, batch) bytes of device scratch, or NULL for the
 * library's own scratch (then calls that overlap on one device must not run concurrently). */
size_t ef_hip_sample_workspace_bytes(size_t vocab, int batch);
int ef_hip_sample(const float* logits_dev, size_t vocab, int batch, size_t ld, const ef_hip_sampler_config* cfg,
                  const int32_t* hist_dev, const int32_t* hist_len_dev, size_t hist_ld, void* rng_dev,
                  int32_t* out_dev, void* ws_dev, void* stream);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): ef_hip_sample with the
 * library's own fixed scratch, a 16 MiB device array per GPU held until the process ends, and no
 * allocation of any kind.  Sizes whose workspace (ef_hip_sample_workspace_bytes) exceeds 16 MiB are
 * rejected with EF_HIP_EINVAL (at vocab 32000: at most 18 sequences per call).  Every call on one
 * GPU shares that scratch: calls that overlap on one GPU (other streams, other threads) race. */
int ef_hip_sample_noalloc(const float* logits_dev, size_t vocab, int batch, size_t ld, const ef_hip_sampler_config* cfg,
                          const int32_t* hist_dev, const int32_t* hist_len_dev, size_t hist_ld, void* rng_dev,
                          int32_t* out_dev, void* stream);
/* kern::argmax (src/kernels.cpp:105-111): first maximum wins. */
int ef_hip_argmax(const float* x_dev, size_t n, int batch, size_t ld, int32_t* out_dev, void* stream);
/* The sampler's softmax-term function (std::exp in src/sampler.cpp:46) over n device doubles:
 * y[i] = exp(x[i]) computed as the sampling kernels compute it, so that a caller can compare the
 * device's exp with the host libm the reference links. */
int ef_hip_sampler_exp(const double* x_dev, double* y_dev, size_t n, void* stream);

/* ---- profiling (the reference's per-op timing, src/bench_decode.cpp:164-231) -------------------
 * Runs `launches` GEMVs back to back on `stream` as one captured HIP graph (launch overhead
 * excluded, as in the decode engine's step graphs), cycling over n_weights weight handles (so the
 * matrices come from HBM, not the 256 MB Infinity Cache), bracketed by HIP events on that stream;
 * *avg_ms is the mean time per launch (for batch > 1 a launch is the fragment preparation and the
 * matrix-core GEMV).  `stream` must be capturable (not the null stream).  epi: 0 = y = W x, 1 = y += W x, 2 = y = silu(W x)*(W2 x)
 * (W2 then holds n_weights up matrices); norm_w_dev as in ef_hip_matvec_swiglu. */
int ef_hip_profile_matvec(int epi, const ef_hip_weight* W, const ef_hip_weight* W2, size_t n_weights,
                          const float* x_dev, const float* norm_w_dev, float eps, float* y_dev, int batch,
                          int launches, void* stream, float* avg_ms);

/* Achievable HBM read bandwidth (membench, include/ef/membench.h:21-54, src/membench.cpp): sums a
 * buffer of pattern words w[i] = i * 0x9E3779B97F4A7C15 + 0x0123456789ABCDEF `passes` times per run
 * on every CU and checks the sum against the closed form; decimal GB/s of the timed runs.  The
 * buffer is rounded down to a whole sweep of the grid (buffer_bytes in the result). */
typedef struct {
  uint64_t buffer_bytes; /* default in the reference: 1 GiB */
  int runs, passes, warmup_runs;
} ef_hip_membench_options;
typedef struct {
  uint64_t buffer_bytes;
  int passes;
  uint64_t bytes_per_run;
  double best_gbps, median_gbps, worst_gbps;
  uint64_t checksum, expected_checksum;
  int checksum_ok; /* every run, warm-up included, matched */
} ef_hip_membench_result;
int ef_hip_membench(const ef_hip_membench_options* options, ef_hip_membench_result* result);
uint64_t ef_hip_membench_expected_pass_sum(uint64_t words); /* membench.h:51 */

/* ---- decode engine ----------------------------------------------------------------------------
 * Transformer::forward (src/model.cpp:184-276) on the device for `batch` independent sequences
 * that share weights, with an FP32 KV cache [L][batch][max_seq][KV*hd] and a per-step HIP graph.
 * Weights are registered handles; norms and the BF16 embedding are device arrays.  Limits: hd a
 * multiple of 4 up to 256, max_seq up to 12000 (attention keeps scores and staged rows in LDS). */
typedef struct {
  size_t D, F, H, KV, hd, V, L, max_pos;
  float eps, rope_theta;
} ef_hip_model_config;

typedef struct {
  ef_hip_weight wq, wk, wv, wo, w_gate, w_up, w_down;
  const float* attn_norm_dev;
  const float* ffn_norm_dev;
} ef_hip_layer;

typedef struct ef_hip_engine_s* ef_hip_engine;
int ef_hip_engine_create(const ef_hip_model_config* cfg, const ef_hip_layer* layers, ef_hip_weight embed,
                         ef_hip_weight lm_head, const float* final_norm_dev, size_t max_seq, int batch,
                         ef_hip_engine* out);
int ef_hip_engine_destroy(ef_hip_engine e);
/* One forward at position pos for all sequences: tokens[batch] (host).  Logits [batch][V] stay on
 * the device (ef_hip_engine_logits); compute_logits = 0 skips the lm_head, as prefill does. */
int ef_hip_engine_forward(ef_hip_engine e, const int32_t* tokens_host, size_t pos, int compute_logits);
/* Positions pos .. pos+n-1 of every sequence at once: tokens[batch][n] (host).  Equivalent to n
 * forward calls (src/model.cpp:290 feeds the prompt one position at a time), with every product
 * run once over all batch * n rows on the matrix cores and causal attention over the cache; logits
 * (compute_logits) and the hidden state are those of position pos+n-1. */
int ef_hip_engine_prefill(ef_hip_engine e, const int32_t* tokens_host, size_t n, size_t pos, int compute_logits);
int ef_hip_engine_logits(ef_hip_engine e, const float** logits_dev);
int ef_hip_engine_hidden(ef_hip_engine e, const float** hidden_dev); /* final-norm output [batch][D] */
/* The reference decode protocol (src/bench_decode.cpp:30-49, generate_greedy src/model.cpp:278-304)
 * run on the device: prompt [batch][n_prompt] one position at a time (logits only at the last),
 * then n tokens per sequence picked by argmax (cfg NULL or temperature <= 0) or by the sampler
 * (rng_dev as in ef_hip_sample; the history is the prompt plus the tokens picked so far).  The
 * prompt goes through ef_hip_engine_prefill's batched path (environment EF_HIP_PREFILL=serial
 * selects the reference's one-position-at-a-time order instead).
 * tokens_out [batch][n] host.  Each step is one HIP graph launch; timings in seconds. */
int ef_hip_engine_generate(ef_hip_engine e, const int32_t* prompt_host, size_t n_prompt, size_t n,
                           const ef_hip_sampler_config* cfg, void* rng_dev, int32_t* tokens_out,
                           double* prefill_s, double* decode_s);

/* Where the time of a decode step goes (the reference's ForwardProfile and run_profile,
 * include/ef/model.h:89-94, src/bench_decode.cpp:164-231; its 13 buckets merged where this build
 * fuses the ops into one kernel).  Each group's launches of one step (every layer's, in step order,
 * the same kernels and arguments as the step graph) are captured as their own HIP graph and
 * replayed `reps` times between HIP events on the engine's stream, at the last cached position;
 * ms_out[g] gets the mean milliseconds per step of group g.  cfg / rng_dev as in generate: the
 * pick group is the sampler (cfg with temperature > 0) or argmax.  The position is restored after
 * each group; the RNG states advance and history entries past the cached positions are
 * overwritten.  Needs at least one cached position (forward, prefill or generate first). */
#define EF_HIP_PROF_EMBED 0     /* Embed */
#define EF_HIP_PROF_QKV 1       /* AttnNorm + QKV (+ the batched path's activation preparation) */
#define EF_HIP_PROF_ATTENTION 2 /* Rope + Attention (cache write included) */
#define EF_HIP_PROF_OPROJ 3     /* OProj + Residual */
#define EF_HIP_PROF_GATE_UP 4   /* FfnNorm + GateUp + SwiGLU */
#define EF_HIP_PROF_DOWN 5      /* Down + Residual */
#define EF_HIP_PROF_LM_HEAD 6   /* FinalNorm + LmHead */
#define EF_HIP_PROF_PICK 7      /* argmax or the sampler, and the step bookkeeping */
#define EF_HIP_PROF_GROUPS 8
int ef_hip_engine_profile(ef_hip_engine e, const ef_hip_sampler_config* cfg, void* rng_dev, int reps, double* ms_out);

/* A several-sequence engine runs its decode step over producer-staged inputs: the embedding lookup,
 * the KV-group attention and the o / gate-up / down products write the next product's matrix-core
 * input tables (block-scaled fp16 hi + lo pairs, with the RMSNorm's per-block partial sums) as they
 * store their outputs, so no product runs a preparation launch.  *on = 1 when this engine does;
 * *why (owned by the engine) says why not otherwise: one sequence, an unquantized matrix, no
 * matrix-core plan for a product, or EF_HIP_DECODE_TABLES=prep at engine creation (the
 * per-product preparation, kept for comparison).  No counterpart in the reference (a CPU build has
 * no kernel boundaries); it lets a caller see which step path runs. */
int ef_hip_engine_tables(ef_hip_engine e, int* on, const char** why);

/* ---- quality of a quantized model (eval-quant, src/eval_quant.cpp) ---------------------------------
 * compare_dist (src/eval_quant.cpp:48-96) over n positions of device logits: KL(P_ref || P_ours) in
 * double, top-1 agreement, the reference confident (its top-1 probability >= 0.5), ours finite;
 * kl_host (optional) gets each position's KL, agg the DistAgg totals in position order. */
typedef struct {
  size_t n, top1, confident, confident_top1, nonfinite;
  double kl_sum, kl_max, kl_mean;
} ef_hip_dist_stats;
int ef_hip_compare_dist(const float* ref_dev, const float* ours_dev, size_t V, size_t n, size_t ld_ref, size_t ld_ours,
                        double* kl_host, ef_hip_dist_stats* agg, void* stream);
/* neg_log_prob (src/eval_quant.cpp:100-102): nll[p] = log_sum_exp(logits_p) - logits_p[target_p]. */
int ef_hip_neg_log_prob(const float* logits_dev, size_t V, size_t n, size_t ld, const int32_t* targets_dev,
                        double* nll_dev, void* stream);

/* ---- chat turns ----------------------------------------------------------------------------------
 * The token-level loop of ef::ChatSession::reply (include/ef/chat.h:99-105, src/chat.cpp:174-259)
 * on an engine of batch 1: ids is the rendered conversation (the tokenizer and chat template stay
 * on the caller's side).  The longest common prefix with the ids whose K / V the engine holds is
 * reused (at least the last id is recomputed), the rest is prefilled in one batched pass, then each
 * step samples (cfg; greedy when temperature <= 0), records P(eos_id) under softmax of the raw
 * logits (prob_of, src/chat.cpp:35-42, fused into the sampler kernel), and stops as the reference:
 * the EOS id, P(EOS) >= eos_min_p (when > 0), or max_new / the context limit.  reply_out gets the
 * generated ids (at most max_new), eos_p_out (optional) P(EOS) of every step.  Role-marker and
 * repetition stops work on decoded text and stay with the caller.  Consecutive calls continue the
 * conversation (the RNG states advance exactly as the reference's Sampler). */
#define EF_HIP_STOP_NONE 0
#define EF_HIP_STOP_EOS 1        /* StopReason order, include/ef/chat.h */
#define EF_HIP_STOP_EOS_MIN_P 2
#define EF_HIP_STOP_MAX_NEW 5
#define EF_HIP_STOP_CONTEXT 6
typedef struct {
  size_t max_new;       /* ChatOptions::max_new */
  int32_t eos_id;       /* Tokenizer::eos_id (-1: none) */
  float eos_min_p;      /* StopConfig::eos_min_p (0: off) */
  int steps_per_check;  /* decode steps launched between host checks (>= 1) */
} ef_hip_reply_options;
typedef struct {        /* TurnStats (include/ef/chat.h) */
  size_t prompt_tokens, reused_tokens, prefill_tokens, generated, steps;
  int reason;           /* EF_HIP_STOP_* */
  double prefill_s, decode_s, eos_p_max;
  size_t eos_p_max_step;
} ef_hip_reply_stats;
int ef_hip_engine_reply(ef_hip_engine e, const int32_t* ids_host, size_t n_ids, const ef_hip_sampler_config* cfg,
                        void* rng_dev, const ef_hip_reply_options* options, int32_t* reply_out, double* eos_p_out,
                        ef_hip_reply_stats* stats);
/* ChatSession::reset (src/chat.cpp:143-148): forget the cached ids (the next turn prefills all). */
int ef_hip_engine_reset(ef_hip_engine e);
/* Teacher-forced scoring of one sequence (engine batch 1; eval-quant's text chunk loop,
 * src/eval_quant.cpp:383-399): ids[0 .. n-2] at positions 0 .. n-2 in batched prefills with the
 * logits of every position (the lm_head on the matrix cores), nll_host[p - first] =
 * neg_log_prob(logits_p, ids[p+1]) for p in [first, n-1); logits_dev (optional) receives those
 * positions' logits, [(n-1-first)][V]. */
int ef_hip_engine_score(ef_hip_engine e, const int32_t* ids_host, size_t n, size_t first, double* nll_host,
                        float* logits_dev);

/* ---- .efq model files -------------------------------------------------------------------------
 * ef::QuantFile (include/ef/qfile.h:95-124).  ef_hip_efq_open maps a file and validates it as
 * QuantFile::open / parse_efq do (src/qfile.cpp:125-243): magic, version, header length, strict
 * JSON header, config.json fields (src/model_config.cpp:72-131), per-tensor type / shape / bytes /
 * 64-byte alignment / bounds / overlap, exactly the tensors the config needs, and every tensor's
 * type re-derived from the header's quantization policy.  ef_hip_efq_parse does the same over a
 * caller's buffer (parse_efq; the buffer must outlive the handle).  Host-only: neither needs a GPU
 * or ef_hip_init.  A rejected file gives EF_HIP_EINVAL and the reader's message (the reference's
 * wording: "bad magic", "past the end", "64-byte aligned", "header says", "policy gives", ...). */
typedef struct ef_hip_efq_s* ef_hip_efq;
typedef struct {
  const char* name;        /* valid while the handle lives */
  const char* rule;        /* policy rule that chose the type: layers, lm_head, embed, norm, override, fallback-bf16 */
  int qtype;
  int ndim;                /* 1 (norms) or 2 */
  size_t rows, cols;       /* a 1-D tensor has rows = 1 */
  uint64_t offset, bytes;  /* absolute file offset and size */
  double rel_rmse, max_abs_err;
  const void* host_data;   /* the tensor's bytes in the mapping */
} ef_hip_efq_tensor;
int ef_hip_efq_open(const char* path, ef_hip_efq* out);            /* QuantFile::open, qfile.h:98 */
int ef_hip_efq_parse(const void* bytes, size_t size, ef_hip_efq* out); /* parse_efq, qfile.h:133 */
int ef_hip_efq_close(ef_hip_efq f);
int ef_hip_efq_config(ef_hip_efq f, ef_hip_model_config* cfg, int* tie_word_embeddings, int64_t* bos_token_id,
                      int64_t* eos_token_id);                      /* QuantFile::config, qfile.h:103 */
int ef_hip_efq_tensor_count(ef_hip_efq f, size_t* n);              /* QuantFile::tensors, qfile.h:105 */
int ef_hip_efq_tensor_info(ef_hip_efq f, size_t i, ef_hip_efq_tensor* out);
int ef_hip_efq_find(ef_hip_efq f, const char* name, size_t* index); /* QuantFile::find / at, qfile.h:106 */
int ef_hip_efq_bytes_per_token(ef_hip_efq f, uint64_t* out);        /* QuantFile::bytes_per_token, qfile.h:112 */
/* QuantFile::policy, qfile.h:104 (layers / lm_head / embed types, override count, policy name). */
int ef_hip_efq_policy(ef_hip_efq f, int* layers, int* lm_head, int* embed, size_t* n_overrides, char* name,
                      size_t name_cap);

/* ---- a model from an .efq file on the device ------------------------------------------------
 * Model::load_efq (src/model.cpp:66-111): every tensor of the file copied once into one device
 * arena in the file's own layout (64-byte aligned tensors), matrices as weight handles over it,
 * norms as FP32 device arrays, the embedding as the lm_head when tie_word_embeddings is set.
 * ef_hip_model_upload takes an open file (which may be closed afterwards).  Engines made by
 * ef_hip_model_engine_create use the model's weights: destroy them before ef_hip_model_free
 * (which otherwise returns EF_HIP_ESTATE). */
typedef struct ef_hip_model_s* ef_hip_model;
int ef_hip_model_load_efq(const char* path, ef_hip_model* out);
int ef_hip_model_upload(ef_hip_efq f, ef_hip_model* out);
int ef_hip_model_free(ef_hip_model m);
int ef_hip_model_config_get(ef_hip_model m, ef_hip_model_config* cfg, int* tie_word_embeddings,
                            int64_t* eos_token_id);                 /* Model::config, model.h:54 */
int ef_hip_model_description(ef_hip_model m, char* buf, size_t cap); /* Model::description, model.h:65 */
int ef_hip_model_bytes_per_token(ef_hip_model m, uint64_t* out);    /* model.h:63 */
int ef_hip_model_layer(ef_hip_model m, size_t l, ef_hip_layer* out); /* Model::layer, model.h:58 */
int ef_hip_model_tensors(ef_hip_model m, ef_hip_weight* embed, ef_hip_weight* lm_head,
                         const float** final_norm_dev);             /* model.h:55-57 */
/* Transformer(model, max_seq) (include/ef/model.h:101, src/model.cpp:153) for `batch` sequences. */
int ef_hip_model_engine_create(ef_hip_model m, size_t max_seq, int batch, ef_hip_engine* out);

#ifdef __cplusplus
}
#endif
#endif
