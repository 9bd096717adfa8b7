/* EdgeForge CPU oracle (test infrastructure only): FP32 glue kernels and the Llama decode step
 * with a KV cache, plus the reference's decode-benchmark protocol.
 *
 * Restates src/kernels.cpp:65-174, src/model.cpp:153-304 and src/bench_decode.cpp:30-49. */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "efo.h"

void efo_add_inplace(float* x, const float* y, size_t n) { /* src/kernels.cpp:65-67 */
  for (size_t i = 0; i < n; ++i) x[i] += y[i];
}

/* Sum of squares in double, HF order w * (x * rsqrt) (src/kernels.cpp:69-75). */
void efo_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  const double mean = n ? ss / (double)n : 0.0;
  const float inv = (float)(1.0 / sqrt(mean + (double)eps));
  for (size_t i = 0; i < n; ++i) out[i] = w[i] * (x[i] * inv);
}

/* Max-subtracted softmax, float exp, double sum; an all -inf row becomes zeros
 * (src/kernels.cpp:77-92). */
void efo_softmax_inplace(float* x, size_t n) {
  if (n == 0) return;
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = x[i] > mx ? x[i] : mx;
  if (mx == -INFINITY) {
    memset(x, 0, n * sizeof(float));
    return;
  }
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - mx);
    sum += (double)x[i];
  }
  const float inv = (float)(1.0 / sum);
  for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

float efo_silu(float x) { return x / (1.0f + expf(-x)); } /* src/kernels.cpp:94 */

void efo_swiglu(float* out, const float* gate, const float* up, size_t n) { /* :96-98 */
  for (size_t i = 0; i < n; ++i) out[i] = efo_silu(gate[i]) * up[i];
}

void efo_embedding_bf16(float* out, const uint16_t* table, size_t token, size_t dim) { /* :100-103 */
  for (size_t i = 0; i < dim; ++i) out[i] = efo_bf16_to_f32(table[token * dim + i]);
}

size_t efo_argmax(const float* x, size_t n) { /* first maximum wins (src/kernels.cpp:105-111) */
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

/* inv_freq[i] = 1 / theta^(2i/hd) and angle = float(pos) * inv_freq[i], all FP32
 * (src/kernels.cpp:113-131). */
void efo_rope_table(float* inv_freq, float* cos_t, float* sin_t, size_t max_pos, size_t head_dim, float theta) {
  const size_t half = head_dim / 2;
  for (size_t i = 0; i < half; ++i) inv_freq[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
  for (size_t p = 0; p < max_pos; ++p)
    for (size_t i = 0; i < half; ++i) {
      const float ang = (float)p * inv_freq[i];
      cos_t[p * half + i] = cosf(ang);
      sin_t[p * half + i] = sinf(ang);
    }
}

/* Half-split rotation of dims (i, i + hd/2) (src/kernels.cpp:133-146). */
void efo_rope_apply(float* x, size_t n_heads, size_t head_dim, const float* c, const float* s) {
  const size_t half = head_dim / 2;
  for (size_t h = 0; h < n_heads; ++h) {
    float* v = x + h * head_dim;
    for (size_t i = 0; i < half; ++i) {
      const float a = v[i], b = v[i + half];
      v[i] = a * c[i] - b * s[i];
      v[i + half] = b * c[i] + a * s[i];
    }
  }
}

/* GQA attention of one query position over n_pos cached positions, heads [h_begin, h_end)
 * (src/kernels.cpp:153-174): query head h reads KV head h / (H / KV). */
void efo_attention_heads(float* out, const float* q, const float* kc, const float* vc, size_t n_pos, size_t H,
                         size_t KV, size_t hd, float* scores, size_t h_begin, size_t h_end) {
  const size_t group = H / KV, kvd = KV * hd;
  const float scale = (float)(1.0 / sqrt((double)hd));
  for (size_t h = h_begin; h < h_end; ++h) {
    const size_t g = h / group;
    const float* qh = q + h * hd;
    for (size_t t = 0; t < n_pos; ++t) scores[t] = efo_dot_f32(qh, kc + t * kvd + g * hd, hd) * scale;
    efo_softmax_inplace(scores, n_pos);
    float* oh = out + h * hd;
    memset(oh, 0, hd * sizeof(float));
    for (size_t t = 0; t < n_pos; ++t) {
      const float pt = scores[t];
      const float* vt = vc + t * kvd + g * hd;
      for (size_t d = 0; d < hd; ++d) oh[d] += pt * vt[d];
    }
  }
}

/* ---- transformer (src/model.cpp:153-276) ---------------------------------------------------- */
struct efo_transformer {
  const efo_model* m;
  efo_pool* pool;
  int backend;
  size_t max_seq, cached;
  float *inv_freq, *cos_t, *sin_t;
  float *k_cache, *v_cache; /* [L][max_seq][KV*hd] */
  float *x, *h, *q, *ctx, *o, *gate, *up, *scores, *logits;
};

efo_transformer* efo_transformer_create(const efo_model* m, size_t max_seq, efo_pool* pool, int backend) {
  const efo_config* c = &m->cfg;
  if (max_seq == 0 || max_seq > c->max_pos) return NULL; /* src/model.cpp:164-168 throw */
  efo_transformer* t = (efo_transformer*)calloc(1, sizeof(efo_transformer));
  t->m = m;
  t->pool = pool;
  t->backend = backend;
  t->max_seq = max_seq;
  const size_t half = c->hd / 2, kvd = c->KV * c->hd;
  t->inv_freq = (float*)malloc(half * sizeof(float));
  t->cos_t = (float*)malloc(max_seq * half * sizeof(float));
  t->sin_t = (float*)malloc(max_seq * half * sizeof(float));
  efo_rope_table(t->inv_freq, t->cos_t, t->sin_t, max_seq, c->hd, c->rope_theta);
  t->k_cache = (float*)calloc(c->L * max_seq * kvd, sizeof(float));
  t->v_cache = (float*)calloc(c->L * max_seq * kvd, sizeof(float));
  t->x = (float*)malloc(c->D * sizeof(float));
  t->h = (float*)malloc(c->D * sizeof(float));
  t->q = (float*)malloc(c->D * sizeof(float));
  t->ctx = (float*)malloc(c->D * sizeof(float));
  t->o = (float*)malloc(c->D * sizeof(float));
  t->gate = (float*)malloc(c->F * sizeof(float));
  t->up = (float*)malloc(c->F * sizeof(float));
  t->scores = (float*)malloc(max_seq * efo_pool_size(pool) * sizeof(float));
  t->logits = (float*)malloc(c->V * sizeof(float));
  return t;
}

void efo_transformer_destroy(efo_transformer* t) {
  if (!t) return;
  free(t->inv_freq);
  free(t->cos_t);
  free(t->sin_t);
  free(t->k_cache);
  free(t->v_cache);
  free(t->x);
  free(t->h);
  free(t->q);
  free(t->ctx);
  free(t->o);
  free(t->gate);
  free(t->up);
  free(t->scores);
  free(t->logits);
  free(t);
}

size_t efo_transformer_cached(const efo_transformer* t) { return t->cached; }
const float* efo_transformer_hidden(const efo_transformer* t) { return t->h; }

typedef struct {
  efo_transformer* t;
  const float* kl;
  const float* vl;
  size_t n_pos;
} attn_ctx;

static void attn_body(void* vctx, size_t chunk, size_t hb, size_t he) {
  const attn_ctx* a = (const attn_ctx*)vctx;
  const efo_config* c = &a->t->m->cfg;
  efo_attention_heads(a->t->ctx, a->t->q, a->kl, a->vl, a->n_pos, c->H, c->KV, c->hd,
                      a->t->scores + chunk * a->t->max_seq, hb, he);
}

const float* efo_transformer_forward(efo_transformer* t, int32_t token, size_t pos, int compute_logits, int* err) {
  const efo_model* m = t->m;
  const efo_config* c = &m->cfg;
  if (err) *err = 0;
  if (token < 0 || (size_t)token >= c->V || pos >= t->max_seq || pos > t->cached) { /* :185-195 */
    if (err) *err = 1;
    return NULL;
  }
  const size_t kvd = c->KV * c->hd, half = c->hd / 2;
  float* x = t->x;
  float* h = t->h;
  efo_row_f32(x, &m->embed, (size_t)token);
  const float* cr = t->cos_t + pos * half;
  const float* sr = t->sin_t + pos * half;
  for (size_t l = 0; l < c->L; ++l) {
    const efo_layer* w = &m->layers[l];
    float* kl = t->k_cache + l * t->max_seq * kvd;
    float* vl = t->v_cache + l * t->max_seq * kvd;
    float* kp = kl + pos * kvd;
    float* vp = vl + pos * kvd;
    efo_rmsnorm(h, x, w->attn_norm, c->D, c->eps);
    const efo_job qkv[3] = {{t->q, &w->wq, h}, {kp, &w->wk, h}, {vp, &w->wv, h}};
    efo_matvec_jobs(t->backend, qkv, 3, t->pool);
    efo_rope_apply(t->q, c->H, c->hd, cr, sr);
    efo_rope_apply(kp, c->KV, c->hd, cr, sr);
    attn_ctx a = {t, kl, vl, pos + 1};
    if (t->pool && efo_pool_size(t->pool) > 1)
      efo_pool_parallel_for(t->pool, c->H, attn_body, &a, 4);
    else
      attn_body(&a, 0, 0, c->H);
    efo_matvec(t->backend, t->o, &w->wo, t->ctx, t->pool);
    efo_add_inplace(x, t->o, c->D);
    efo_rmsnorm(h, x, w->ffn_norm, c->D, c->eps);
    const efo_job gu[2] = {{t->gate, &w->w_gate, h}, {t->up, &w->w_up, h}};
    efo_matvec_jobs(t->backend, gu, 2, t->pool);
    efo_swiglu(t->gate, t->gate, t->up, c->F);
    efo_matvec(t->backend, t->o, &w->w_down, t->gate, t->pool);
    efo_add_inplace(x, t->o, c->D);
  }
  t->cached = pos + 1;
  efo_rmsnorm(h, x, m->final_norm, c->D, c->eps);
  if (!compute_logits) return NULL;
  efo_matvec(t->backend, t->logits, &m->lm_head, h, t->pool);
  return t->logits;
}

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Prompt one token at a time (logits only at its last position), then n greedy steps; the
 * n-th token is picked without a further forward (src/bench_decode.cpp:30-49). */
int efo_run_once(const efo_model* m, const int32_t* prompt, size_t n_prompt, size_t n, efo_pool* pool, int backend,
                 int32_t* tokens, float* logits, double* prefill_s, double* decode_s) {
  if (n_prompt == 0) return -1;
  efo_transformer* t = efo_transformer_create(m, n_prompt + n, pool, backend);
  if (!t) return -1;
  const size_t V = m->cfg.V;
  int err = 0;
  const double t0 = now_s();
  const float* lg = NULL;
  for (size_t p = 0; p < n_prompt; ++p) {
    lg = efo_transformer_forward(t, prompt[p], p, p + 1 == n_prompt, &err);
    if (err) goto fail;
  }
  const double t1 = now_s();
  for (size_t k = 0; k < n; ++k) {
    if (logits) memcpy(logits + k * V, lg, V * sizeof(float));
    tokens[k] = (int32_t)efo_argmax(lg, V);
    if (k + 1 < n) {
      lg = efo_transformer_forward(t, tokens[k], n_prompt + k, 1, &err);
      if (err) goto fail;
    }
  }
  if (prefill_s) *prefill_s = t1 - t0;
  if (decode_s) *decode_s = now_s() - t1;
  efo_transformer_destroy(t);
  return 0;
fail:
  efo_transformer_destroy(t);
  return -1;
}
