/* EdgeForge CPU oracle (test infrastructure only): the next-token sampler and the random number
 * generator it draws from.
 *
 * Restates include/ef/sampler.h:13-35 and src/sampler.cpp:13-70.  The generator is
 * std::mt19937_64 (fully specified by ISO C++ [rand.predef]); the draw is libstdc++'s
 * std::uniform_real_distribution<double>(0, 1), i.e. generate_canonical<double, 53> with one
 * 64-bit word: double(u) / 2^64, mapped to nextafter(1, 0) if it rounds up to 1. */
#define _GNU_SOURCE
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "efo.h"

/* ---- std::mt19937_64 ------------------------------------------------------------------------ */
#define MT_N 312
#define MT_M 156

void efo_mt64_seed(efo_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < MT_N; ++i) g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
  g->idx = MT_N;
}

static void mt_refill(efo_mt64* g) {
  const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL, a = 0xB5026F5AA96619E9ULL;
  for (int i = 0; i < MT_N; ++i) {
    const uint64_t y = (g->mt[i] & upper) | (g->mt[(i + 1) % MT_N] & lower);
    g->mt[i] = g->mt[(i + MT_M) % MT_N] ^ (y >> 1) ^ ((y & 1ULL) ? a : 0ULL);
  }
  g->idx = 0;
}

uint64_t efo_mt64_next(efo_mt64* g) {
  if (g->idx >= MT_N) mt_refill(g);
  uint64_t y = g->mt[g->idx++];
  y ^= (y >> 29) & 0x5555555555555555ULL;
  y ^= (y << 17) & 0x71D67FFFEDA60000ULL;
  y ^= (y << 37) & 0xFFF7EEE000000000ULL;
  y ^= y >> 43;
  return y;
}

double efo_canonical_double(efo_mt64* g) {
  const double r = (double)efo_mt64_next(g) / 18446744073709551616.0;
  return r >= 1.0 ? nextafter(1.0, 0.0) : r;
}

/* ---- sampler -------------------------------------------------------------------------------- */
struct efo_sampler {
  efo_sampler_config cfg;
  efo_mt64 rng;
  float* work;
  int32_t* idx;
  double* prob;
  unsigned char* seen;
  size_t cap;
  size_t last_keep;
  double last_r;
};

efo_sampler* efo_sampler_create(const efo_sampler_config* cfg) {
  efo_sampler* s = (efo_sampler*)calloc(1, sizeof(efo_sampler));
  s->cfg = *cfg;
  efo_mt64_seed(&s->rng, cfg->seed);
  s->last_r = -1.0;
  return s;
}

void efo_sampler_destroy(efo_sampler* s) {
  if (!s) return;
  free(s->work);
  free(s->idx);
  free(s->prob);
  free(s->seen);
  free(s);
}

/* Strict total order of the reference comparator: higher logit first, then lower id. */
static inline int ahead(const float* w, int32_t a, int32_t b) { return w[a] != w[b] ? w[a] > w[b] : a < b; }

static int cmp_ids(const void* pa, const void* pb, void* work) {
  const int32_t a = *(const int32_t*)pa, b = *(const int32_t*)pb;
  if (a == b) return 0;
  return ahead((const float*)work, a, b) ? -1 : 1;
}

/* The k best ids of [0, V) in order, via a bounded heap whose root is the worst kept id. */
static void top_k_ids(const float* w, size_t V, size_t k, int32_t* out) {
  size_t n = 0;
  for (size_t i = 0; i < V; ++i) {
    const int32_t id = (int32_t)i;
    if (n < k) { /* sift up: parent must be the worse one */
      size_t c = n++;
      out[c] = id;
      while (c > 0) {
        const size_t p = (c - 1) / 2;
        if (!ahead(w, out[p], out[c])) break;
        const int32_t t = out[p];
        out[p] = out[c];
        out[c] = t;
        c = p;
      }
    } else if (ahead(w, id, out[0])) { /* replace the worst and sift down */
      out[0] = id;
      size_t c = 0;
      for (;;) {
        const size_t l = 2 * c + 1, r = l + 1;
        size_t worst = c;
        if (l < k && ahead(w, out[worst], out[l])) worst = l;
        if (r < k && ahead(w, out[worst], out[r])) worst = r;
        if (worst == c) break;
        const int32_t t = out[c];
        out[c] = out[worst];
        out[worst] = t;
        c = worst;
      }
    }
  }
  qsort_r(out, k, sizeof(int32_t), cmp_ids, (void*)w);
}

int32_t efo_sampler_sample(efo_sampler* s, const float* logits, size_t vocab, const int32_t* history, size_t n_hist) {
  if (vocab == 0) return -1; /* src/sampler.cpp:14 throws */
  if (s->cap < vocab) {
    free(s->work);
    free(s->idx);
    free(s->prob);
    free(s->seen);
    s->work = (float*)malloc(vocab * sizeof(float));
    s->idx = (int32_t*)malloc(vocab * sizeof(int32_t));
    s->prob = (double*)malloc(vocab * sizeof(double));
    s->seen = (unsigned char*)malloc(vocab);
    s->cap = vocab;
  }
  float* w = s->work;
  memcpy(w, logits, vocab * sizeof(float));
  const float pen = s->cfg.repetition_penalty;
  if (pen != 1.0f) { /* each unique in-range history id once (src/sampler.cpp:16-24) */
    memset(s->seen, 0, vocab);
    for (size_t i = 0; i < n_hist; ++i) {
      const int32_t t = history[i];
      if (t < 0 || (size_t)t >= vocab || s->seen[t]) continue;
      s->seen[t] = 1;
      w[t] = w[t] > 0.0f ? w[t] / pen : w[t] * pen;
    }
  }
  s->last_keep = 0;
  s->last_r = -1.0;
  if (s->cfg.temperature <= 0.0f) return (int32_t)efo_argmax(w, vocab); /* :25, no draw */

  for (size_t i = 0; i < vocab; ++i) w[i] /= s->cfg.temperature;
  size_t keep = vocab;
  if (s->cfg.top_k > 0 && (size_t)s->cfg.top_k < vocab) {
    keep = (size_t)s->cfg.top_k;
    top_k_ids(w, vocab, keep, s->idx);
  } else {
    for (size_t i = 0; i < vocab; ++i) s->idx[i] = (int32_t)i;
    qsort_r(s->idx, vocab, sizeof(int32_t), cmp_ids, (void*)w);
  }
  /* softmax over the kept ids in double, left-to-right sum (src/sampler.cpp:42-49) */
  double* p = s->prob;
  const float mx = w[s->idx[0]];
  double sum = 0.0;
  for (size_t i = 0; i < keep; ++i) {
    p[i] = exp((double)(w[s->idx[i]] - mx));
    sum += p[i];
  }
  for (size_t i = 0; i < keep; ++i) p[i] /= sum;
  if (s->cfg.top_p < 1.0f) { /* nucleus cut and renormalisation (src/sampler.cpp:50-61) */
    double cum = 0.0;
    size_t n = 0;
    while (n < keep) {
      cum += p[n++];
      if (cum >= (double)s->cfg.top_p) break;
    }
    keep = n > 1 ? n : 1;
    double s2 = 0.0;
    for (size_t i = 0; i < keep; ++i) s2 += p[i];
    for (size_t i = 0; i < keep; ++i) p[i] /= s2;
  }
  const double r = efo_canonical_double(&s->rng); /* :62-63 */
  s->last_keep = keep;
  s->last_r = r;
  double cum = 0.0;
  for (size_t i = 0; i < keep; ++i) { /* :64-69 */
    cum += p[i];
    if (r < cum) return s->idx[i];
  }
  return s->idx[keep - 1];
}

size_t efo_sampler_last_keep(const efo_sampler* s, int32_t* ids, double* probs, size_t cap) {
  const size_t n = s->last_keep < cap ? s->last_keep : cap;
  for (size_t i = 0; i < n; ++i) {
    if (ids) ids[i] = s->idx[i];
    if (probs) probs[i] = s->prob[i];
  }
  return s->last_keep;
}

double efo_sampler_last_r(const efo_sampler* s) { return s->last_r; }

void efo_exp_array(const double* x, double* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = exp(x[i]);
}
