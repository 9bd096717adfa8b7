/* EdgeForge CPU oracle: a plain-C restatement of the reference's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker or the timed CPU baseline.  The product path
 * (edgeforge_amd) never links, imports or falls back to it.
 *
 * Every function names the reference file:line it restates (paths relative to the EdgeForge
 * repository root).  Parity of each function is pinned in tests/test_oracle_*.py against the
 * reference's own known-answer tests, against the reference sources compiled into oracle/_ref
 * (when that library is present), and against closed forms / brute force.  No function here is
 * "parity unpinned".
 *
 * Numerics follow the reference build: -O3 -ffp-contract=off, scalar kernels in the exact
 * summation order of src/qkernels.cpp, AVX2 kernels in the exact lane/FMA order of the reference's
 * AVX2 backend, so both backends are bit-identical to the reference's.
 */
#ifndef EFO_H
#define EFO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- storage types (include/ef/quant.h:22-35) ------------------------------------------------ */
enum { EFO_F32 = 0, EFO_F16 = 1, EFO_BF16 = 2, EFO_Q8_0 = 3, EFO_Q4_0 = 4 };
#define EFO_QK 32
#define EFO_Q4_BLOCK 18
#define EFO_Q8_BLOCK 34

/* ---- 16-bit floats (include/ef/fp16.h:28-91) ------------------------------------------------- */
float efo_fp16_to_f32(uint16_t h);
uint16_t efo_f32_to_fp16(float f);
float efo_bf16_to_f32(uint16_t h);
uint16_t efo_f32_to_bf16(float f);
void efo_fp16_to_f32_n(const uint16_t* h, float* out, size_t n);
void efo_f32_to_fp16_n(const float* f, uint16_t* out, size_t n);
void efo_f32_to_bf16_n(const float* f, uint16_t* out, size_t n);

/* ---- block codec (src/quant.cpp:136-249) ----------------------------------------------------- */
/* Returns 0 and the row byte count in *out, or -1 when a block type gets cols % 32 != 0. */
int efo_row_bytes(int qtype, uint64_t cols, uint64_t* out);
void efo_quantize_block_q4_0(const float* x, uint8_t* out18, int search);
void efo_quantize_block_q8_0(const float* x, uint8_t* out34);
void efo_dequantize_block_q4_0(const uint8_t* b18, float* out);
void efo_dequantize_block_q8_0(const uint8_t* b34, float* out);
int efo_quantize_row(int qtype, const float* x, size_t n, uint8_t* out, int search);
int efo_dequantize_row(int qtype, const uint8_t* in, size_t n, float* out);
/* rows x cols matrix, row-major, rows quantized independently; uses up to `threads` threads. */
int efo_quantize_matrix(int qtype, const float* w, size_t rows, size_t cols, uint8_t* out, int search, int threads);
void efo_fake_quant_q4_group(const float* x, size_t n, float* out, int search);

/* ---- packed GEMV (src/qkernels.cpp) ---------------------------------------------------------- */
enum { EFO_BACKEND_SCALAR = 0, EFO_BACKEND_AVX2 = 1 };
float efo_dot_q4_0(const uint8_t* row, const float* x, size_t n);
float efo_dot_q8_0(const uint8_t* row, const float* x, size_t n);
float efo_dot_q4_0_avx2(const uint8_t* row, const float* x, size_t n);
float efo_dot_q8_0_avx2(const uint8_t* row, const float* x, size_t n);
float efo_dot_bf16_avx2(const uint16_t* w, const float* x, size_t n);
float efo_dot_f32_avx2(const float* w, const float* x, size_t n);
float efo_dot_f32(const float* a, const float* b, size_t n);
void efo_matvec_f32(float* y, const float* W, const float* x, size_t rows, size_t cols);
void efo_matvec_bf16(float* y, const uint16_t* W, const float* x, size_t rows, size_t cols);

typedef struct efo_pool efo_pool;
efo_pool* efo_pool_create(unsigned threads);
void efo_pool_destroy(efo_pool* p);
unsigned efo_pool_size(const efo_pool* p);
typedef void (*efo_range_fn)(void* ctx, size_t chunk, size_t begin, size_t end);
void efo_pool_parallel_for(efo_pool* p, size_t n, efo_range_fn fn, void* ctx, size_t min_chunk);
size_t efo_pool_chunk_begin(size_t n, unsigned chunks, unsigned c);

typedef struct {
  int qtype;
  const uint8_t* data;
  size_t rows, cols;
} efo_weight;

typedef struct {
  float* y;
  const efo_weight* W;
  const float* x;
} efo_job;

void efo_matvec_rows(int backend, float* y, const efo_weight* W, const float* x, size_t begin, size_t end);
void efo_matvec_jobs(int backend, const efo_job* jobs, size_t n_jobs, efo_pool* pool);
void efo_matvec(int backend, float* y, const efo_weight* W, const float* x, efo_pool* pool);
void efo_row_f32(float* out, const efo_weight* W, size_t r);

/* ---- FP32 glue kernels (src/kernels.cpp) ----------------------------------------------------- */
void efo_add_inplace(float* x, const float* y, size_t n);
void efo_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps);
void efo_softmax_inplace(float* x, size_t n);
float efo_silu(float x);
void efo_swiglu(float* out, const float* gate, const float* up, size_t n);
void efo_embedding_bf16(float* out, const uint16_t* table, size_t token, size_t dim);
size_t efo_argmax(const float* x, size_t n);
/* cos/sin tables [max_pos][head_dim/2] and inv_freq[head_dim/2] */
void efo_rope_table(float* inv_freq, float* cos_t, float* sin_t, size_t max_pos, size_t head_dim, float theta);
void efo_rope_apply(float* x, size_t n_heads, size_t head_dim, const float* cos_row, const float* sin_row);
void efo_attention_heads(float* out, const float* q, const float* k_cache, const float* v_cache, size_t n_pos,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float* scores, size_t h_begin,
                         size_t h_end);

/* ---- sampler (include/ef/sampler.h, src/sampler.cpp) ----------------------------------------- */
typedef struct {
  uint64_t mt[312];
  int idx;
} efo_mt64;
void efo_mt64_seed(efo_mt64* g, uint64_t seed);
uint64_t efo_mt64_next(efo_mt64* g);
double efo_canonical_double(efo_mt64* g); /* std::uniform_real_distribution<double>(0,1) on libstdc++ */

typedef struct {
  float temperature;
  int top_k;
  float top_p;
  float repetition_penalty;
  uint64_t seed;
} efo_sampler_config;

typedef struct efo_sampler efo_sampler;
efo_sampler* efo_sampler_create(const efo_sampler_config* cfg);
void efo_sampler_destroy(efo_sampler* s);
/* Returns the token id, or -1 for vocab == 0 (the reference throws). */
int32_t efo_sampler_sample(efo_sampler* s, const float* logits, size_t vocab, const int32_t* history, size_t n_hist);
/* Debug view of the last call: the kept candidate ids (sorted) and their final probabilities. */
size_t efo_sampler_last_keep(const efo_sampler* s, int32_t* ids, double* probs, size_t cap);
double efo_sampler_last_r(const efo_sampler* s);
/* y[i] = exp(x[i]) through the host libm's exp, the call the softmax terms use (std::exp,
 * src/sampler.cpp:46): the host side of the device exp(double) sweep. */
void efo_exp_array(const double* x, double* y, size_t n);

/* ---- transformer (include/ef/model.h, src/model.cpp:153-304) --------------------------------- */
typedef struct {
  size_t D, F, H, KV, hd, V, L, max_pos;
  float eps, rope_theta;
} efo_config;

typedef struct {
  efo_weight wq, wk, wv, wo, w_gate, w_up, w_down;
  const float* attn_norm;
  const float* ffn_norm;
} efo_layer;

typedef struct {
  efo_config cfg;
  efo_weight embed;   /* BF16 (or any type) [V][D] */
  efo_weight lm_head; /* [V][D] */
  const float* final_norm;
  const efo_layer* layers; /* [L] */
} efo_model;

typedef struct efo_transformer efo_transformer;
efo_transformer* efo_transformer_create(const efo_model* m, size_t max_seq, efo_pool* pool, int backend);
void efo_transformer_destroy(efo_transformer* t);
/* Returns the logits [V] or NULL (compute_logits == 0); NULL with *err != 0 on a bad token/pos. */
const float* efo_transformer_forward(efo_transformer* t, int32_t token, size_t pos, int compute_logits, int* err);
size_t efo_transformer_cached(const efo_transformer* t);
/* Final RMSNorm output of the last forward (the lm_head input). */
const float* efo_transformer_hidden(const efo_transformer* t);
/* Reference decode protocol (src/bench_decode.cpp:30-49): prompt one token at a time, then n greedy
 * steps.  tokens[n]; logits (optional) [n][V]; seconds of prefill / decode. */
int efo_run_once(const efo_model* m, const int32_t* prompt, size_t n_prompt, size_t n, efo_pool* pool, int backend,
                 int32_t* tokens, float* logits, double* prefill_s, double* decode_s);

#ifdef __cplusplus
}
#endif
#endif
