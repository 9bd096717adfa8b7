/* EdgeForge CPU oracle (test infrastructure only): packed Q4_0 / Q8_0 dot products in the
 * reference's two summation orders (scalar and AVX2), the row dispatch, the multi-job GEMV and the
 * persistent thread pool that splits rows across cores.
 *
 * Restates src/qkernels.cpp:21-305, src/kernels.cpp:25-63 and src/threadpool.cpp:18-73 /
 * include/ef/threadpool.h:37-54.  Built with -ffp-contract=off so the scalar order is literal. */
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "efo.h"

static inline float scale_at(const uint8_t* p) { return efo_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Fixed pairwise reduction of the 32 lane sums (src/qkernels.cpp:28-32). */
static float reduce32(const float* lo, const float* hi) {
  float s[8];
  for (int j = 0; j < 8; ++j) s[j] = (lo[j] + lo[j + 8]) + (hi[j] + hi[j + 8]);
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* Scalar order (src/qkernels.cpp:39-65): lane j accumulates d * (float(code - 8) * x) for weight
 * j of every block; lanes 0-15 hold the low nibbles, 16-31 the high nibbles.  No FMA. */
float efo_dot_q4_0(const uint8_t* row, const float* x, size_t n) {
  float lo[16] = {0}, hi[16] = {0};
  const size_t nb = n / EFO_QK;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + b * EFO_Q4_BLOCK;
    const float* xb = x + b * EFO_QK;
    const float d = scale_at(blk);
    for (int j = 0; j < 16; ++j) {
      const float p_lo = (float)((blk[2 + j] & 15) - 8) * xb[j];
      const float p_hi = (float)((blk[2 + j] >> 4) - 8) * xb[j + 16];
      lo[j] += d * p_lo;
      hi[j] += d * p_hi;
    }
  }
  return reduce32(lo, hi);
}

float efo_dot_q8_0(const uint8_t* row, const float* x, size_t n) {
  float lo[16] = {0}, hi[16] = {0};
  const size_t nb = n / EFO_QK;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + b * EFO_Q8_BLOCK;
    const float* xb = x + b * EFO_QK;
    const float d = scale_at(blk);
    for (int j = 0; j < 16; ++j) {
      const float p_lo = (float)(int8_t)blk[2 + j] * xb[j];
      const float p_hi = (float)(int8_t)blk[18 + j] * xb[j + 16];
      lo[j] += d * p_lo;
      hi[j] += d * p_hi;
    }
  }
  return reduce32(lo, hi);
}

/* ---- AVX2 order (src/qkernels.cpp:115-208) --------------------------------------------------
 * Per block, 8 lanes: s = w[0:8]*x[0:8]; s = fma(w[8:16], x[8:16], s); then weights 16..23 and
 * 24..31 the same way; acc = fma(d, s, acc).  Even blocks go to one accumulator, odd blocks to a
 * second; the two are added lane-wise and reduced as ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)). */
static inline float lanes8_reduce(__m256 v) {
  const __m128 q = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1)); /* v_i + v_{i+4} */
  const __m128 p = _mm_add_ps(q, _mm_movehl_ps(q, q));                                  /* q0+q2, q1+q3 */
  return _mm_cvtss_f32(_mm_add_ss(p, _mm_movehdup_ps(p)));
}

static inline __m256 bytes8_to_ps(__m128i b) { return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b)); }

/* Four 8-weight slices (already widened to signed bytes: w0..15 in a, w16..31 in b) against x. */
static inline __m256 block_fma(__m128i a, __m128i b, const float* x, float d, __m256 acc) {
  __m256 s = _mm256_mul_ps(bytes8_to_ps(a), _mm256_loadu_ps(x));
  s = _mm256_fmadd_ps(bytes8_to_ps(_mm_srli_si128(a, 8)), _mm256_loadu_ps(x + 8), s);
  s = _mm256_fmadd_ps(bytes8_to_ps(b), _mm256_loadu_ps(x + 16), s);
  s = _mm256_fmadd_ps(bytes8_to_ps(_mm_srli_si128(b, 8)), _mm256_loadu_ps(x + 24), s);
  return _mm256_fmadd_ps(_mm256_set1_ps(d), s, acc);
}

static inline __m256 q4_blk(const uint8_t* blk, const float* x, __m256 acc) {
  const __m128i raw = _mm_loadu_si128((const __m128i*)(blk + 2));
  const __m128i nib = _mm_set1_epi8(15), bias = _mm_set1_epi8(8);
  const __m128i lo = _mm_sub_epi8(_mm_and_si128(raw, nib), bias);
  const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(raw, 4), nib), bias);
  return block_fma(lo, hi, x, scale_at(blk), acc);
}

static inline __m256 q8_blk(const uint8_t* blk, const float* x, __m256 acc) {
  const __m128i a = _mm_loadu_si128((const __m128i*)(blk + 2));
  const __m128i b = _mm_loadu_si128((const __m128i*)(blk + 18));
  return block_fma(a, b, x, scale_at(blk), acc);
}

float efo_dot_q4_0_avx2(const uint8_t* row, const float* x, size_t n) {
  const size_t nb = n / EFO_QK;
  __m256 even = _mm256_setzero_ps(), odd = _mm256_setzero_ps();
  size_t b = 0;
  for (; b + 1 < nb; b += 2) {
    even = q4_blk(row + b * EFO_Q4_BLOCK, x + b * EFO_QK, even);
    odd = q4_blk(row + (b + 1) * EFO_Q4_BLOCK, x + (b + 1) * EFO_QK, odd);
  }
  if (b < nb) even = q4_blk(row + b * EFO_Q4_BLOCK, x + b * EFO_QK, even);
  return lanes8_reduce(_mm256_add_ps(even, odd));
}

float efo_dot_q8_0_avx2(const uint8_t* row, const float* x, size_t n) {
  const size_t nb = n / EFO_QK;
  __m256 even = _mm256_setzero_ps(), odd = _mm256_setzero_ps();
  size_t b = 0;
  for (; b + 1 < nb; b += 2) {
    even = q8_blk(row + b * EFO_Q8_BLOCK, x + b * EFO_QK, even);
    odd = q8_blk(row + (b + 1) * EFO_Q8_BLOCK, x + (b + 1) * EFO_QK, odd);
  }
  if (b < nb) even = q8_blk(row + b * EFO_Q8_BLOCK, x + b * EFO_QK, even);
  return lanes8_reduce(_mm256_add_ps(even, odd));
}

/* BF16 row: 2 accumulators over 16-wide steps, scalar tail (src/qkernels.cpp:182-194). */
float efo_dot_bf16_avx2(const uint16_t* w, const float* x, size_t n) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  size_t i = 0;
  for (; i + 16 <= n; i += 16) {
    const __m256i u0 = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i*)(w + i)));
    const __m256i u1 = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i*)(w + i + 8)));
    a0 = _mm256_fmadd_ps(_mm256_castsi256_ps(_mm256_slli_epi32(u0, 16)), _mm256_loadu_ps(x + i), a0);
    a1 = _mm256_fmadd_ps(_mm256_castsi256_ps(_mm256_slli_epi32(u1, 16)), _mm256_loadu_ps(x + i + 8), a1);
  }
  float s = lanes8_reduce(_mm256_add_ps(a0, a1));
  for (; i < n; ++i) s += efo_bf16_to_f32(w[i]) * x[i];
  return s;
}

/* F32 row: 4 accumulators over 32-wide steps, scalar tail (src/qkernels.cpp:196-208). */
float efo_dot_f32_avx2(const float* w, const float* x, size_t n) {
  __m256 a[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  size_t i = 0;
  for (; i + 32 <= n; i += 32)
    for (int k = 0; k < 4; ++k) a[k] = _mm256_fmadd_ps(_mm256_loadu_ps(w + i + 8 * k), _mm256_loadu_ps(x + i + 8 * k), a[k]);
  float s = lanes8_reduce(_mm256_add_ps(_mm256_add_ps(a[0], a[1]), _mm256_add_ps(a[2], a[3])));
  for (; i < n; ++i) s += w[i] * x[i];
  return s;
}

/* FP32 / BF16 reference rows: 8 partial sums, pairwise combination (src/kernels.cpp:27-43). */
static float dot8(const float* w, const uint16_t* wb, const float* x, size_t n) {
  float a[8] = {0};
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int k = 0; k < 8; ++k) a[k] += (wb ? efo_bf16_to_f32(wb[i + k]) : w[i + k]) * x[i + k];
  for (; i < n; ++i) a[0] += (wb ? efo_bf16_to_f32(wb[i]) : w[i]) * x[i];
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

float efo_dot_f32(const float* a, const float* b, size_t n) { return dot8(a, NULL, b, n); }
void efo_matvec_f32(float* y, const float* W, const float* x, size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; ++r) y[r] = dot8(W + r * cols, NULL, x, cols);
}
void efo_matvec_bf16(float* y, const uint16_t* W, const float* x, size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; ++r) y[r] = dot8(NULL, W + r * cols, x, cols);
}

static float dot_f16_plain(const uint8_t* p, const float* x, size_t n) { /* src/qkernels.cpp:228-236 */
  float acc = 0.0f;
  for (size_t c = 0; c < n; ++c) acc += efo_fp16_to_f32((uint16_t)(p[2 * c] | (p[2 * c + 1] << 8))) * x[c];
  return acc;
}

/* Rows [begin, end) of y = W x with one backend (src/qkernels.cpp:213-269). */
void efo_matvec_rows(int backend, float* y, const efo_weight* W, const float* x, size_t begin, size_t end) {
  if (begin >= end) return;
  uint64_t rb = 0;
  if (efo_row_bytes(W->qtype, W->cols, &rb)) return;
  for (size_t r = begin; r < end; ++r) {
    const uint8_t* row = W->data + r * rb;
    float v = 0.0f;
    switch (W->qtype) {
      case EFO_Q4_0: v = backend == EFO_BACKEND_AVX2 ? efo_dot_q4_0_avx2(row, x, W->cols) : efo_dot_q4_0(row, x, W->cols); break;
      case EFO_Q8_0: v = backend == EFO_BACKEND_AVX2 ? efo_dot_q8_0_avx2(row, x, W->cols) : efo_dot_q8_0(row, x, W->cols); break;
      case EFO_BF16:
        v = backend == EFO_BACKEND_AVX2 ? efo_dot_bf16_avx2((const uint16_t*)row, x, W->cols)
                                        : dot8(NULL, (const uint16_t*)row, x, W->cols);
        break;
      case EFO_F32:
        v = backend == EFO_BACKEND_AVX2 ? efo_dot_f32_avx2((const float*)row, x, W->cols) : dot8((const float*)row, NULL, x, W->cols);
        break;
      case EFO_F16: v = dot_f16_plain(row, x, W->cols); break;
    }
    y[r] = v;
  }
}

/* ---- persistent thread pool (src/threadpool.cpp, include/ef/threadpool.h:37-54) ------------- */
struct efo_pool {
  unsigned size;
  pthread_t* th;
  pthread_mutex_t mu;
  pthread_cond_t cv;
  _Atomic unsigned long long gen;
  _Atomic unsigned pending;
  _Atomic int stop;
  size_t job_n;
  unsigned job_chunks;
  efo_range_fn job_fn;
  void* job_ctx;
};

typedef struct {
  efo_pool* p;
  unsigned id;
} pool_arg;

size_t efo_pool_chunk_begin(size_t n, unsigned chunks, unsigned c) { return (size_t)((uint64_t)n * c / chunks); }

static void* pool_worker(void* arg) {
  efo_pool* p = ((pool_arg*)arg)->p;
  const unsigned id = ((pool_arg*)arg)->id;
  free(arg);
  unsigned long long seen = 0;
  for (;;) {
    unsigned long long g = atomic_load_explicit(&p->gen, memory_order_acquire);
    for (int spin = 0; g == seen && spin < 20000; ++spin) {
      _mm_pause();
      g = atomic_load_explicit(&p->gen, memory_order_acquire);
    }
    if (g == seen) {
      pthread_mutex_lock(&p->mu);
      while ((g = atomic_load_explicit(&p->gen, memory_order_acquire)) == seen) pthread_cond_wait(&p->cv, &p->mu);
      pthread_mutex_unlock(&p->mu);
    }
    if (atomic_load_explicit(&p->stop, memory_order_relaxed)) return NULL;
    seen = g;
    if (id < p->job_chunks)
      p->job_fn(p->job_ctx, id, efo_pool_chunk_begin(p->job_n, p->job_chunks, id),
                efo_pool_chunk_begin(p->job_n, p->job_chunks, id + 1));
    atomic_fetch_sub_explicit(&p->pending, 1, memory_order_release);
  }
}

efo_pool* efo_pool_create(unsigned threads) {
  efo_pool* p = (efo_pool*)calloc(1, sizeof(efo_pool));
  p->size = threads ? threads : 1;
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->cv, NULL);
  p->th = (pthread_t*)calloc(p->size, sizeof(pthread_t));
  for (unsigned i = 1; i < p->size; ++i) {
    pool_arg* a = (pool_arg*)malloc(sizeof(pool_arg));
    a->p = p;
    a->id = i;
    pthread_create(&p->th[i], NULL, pool_worker, a);
  }
  return p;
}

void efo_pool_destroy(efo_pool* p) {
  if (!p) return;
  pthread_mutex_lock(&p->mu);
  atomic_store_explicit(&p->stop, 1, memory_order_relaxed);
  atomic_fetch_add_explicit(&p->gen, 1, memory_order_release);
  pthread_mutex_unlock(&p->mu);
  pthread_cond_broadcast(&p->cv);
  for (unsigned i = 1; i < p->size; ++i) pthread_join(p->th[i], NULL);
  pthread_mutex_destroy(&p->mu);
  pthread_cond_destroy(&p->cv);
  free(p->th);
  free(p);
}

unsigned efo_pool_size(const efo_pool* p) { return p ? p->size : 1; }

/* C = min(size, ceil(n / min_chunk)) contiguous chunks; the caller runs chunk 0 and waits for
 * every worker to acknowledge the job (include/ef/threadpool.h:37-49, src/threadpool.cpp:36-51). */
void efo_pool_parallel_for(efo_pool* p, size_t n, efo_range_fn fn, void* ctx, size_t min_chunk) {
  if (n == 0) return;
  if (min_chunk == 0) min_chunk = 1;
  size_t want = (n + min_chunk - 1) / min_chunk;
  if (want < 1) want = 1;
  const unsigned size = efo_pool_size(p);
  const unsigned chunks = (unsigned)(want < size ? want : size);
  if (chunks <= 1) {
    fn(ctx, 0, 0, n);
    return;
  }
  p->job_n = n;
  p->job_chunks = chunks;
  p->job_fn = fn;
  p->job_ctx = ctx;
  atomic_store_explicit(&p->pending, p->size - 1, memory_order_relaxed);
  pthread_mutex_lock(&p->mu);
  atomic_fetch_add_explicit(&p->gen, 1, memory_order_release);
  pthread_mutex_unlock(&p->mu);
  pthread_cond_broadcast(&p->cv);
  fn(ctx, 0, 0, efo_pool_chunk_begin(n, chunks, 1));
  while (atomic_load_explicit(&p->pending, memory_order_acquire) != 0) _mm_pause();
}

/* ---- multi-job GEMV (src/qkernels.cpp:272-297) ----------------------------------------------
 * The rows of all jobs form one index space; each chunk maps back onto the jobs it overlaps. */
typedef struct {
  int backend;
  const efo_job* jobs;
  size_t n_jobs;
} jobs_ctx;

static void jobs_body(void* vctx, size_t chunk, size_t b, size_t e) {
  (void)chunk;
  const jobs_ctx* c = (const jobs_ctx*)vctx;
  size_t first = 0;
  for (size_t j = 0; j < c->n_jobs; ++j) {
    const size_t rows = c->jobs[j].W->rows;
    const size_t lo = b > first ? b : first, hi = e < first + rows ? e : first + rows;
    if (lo < hi) efo_matvec_rows(c->backend, c->jobs[j].y, c->jobs[j].W, c->jobs[j].x, lo - first, hi - first);
    first += rows;
  }
}

void efo_matvec_jobs(int backend, const efo_job* jobs, size_t n_jobs, efo_pool* pool) {
  size_t total = 0;
  for (size_t j = 0; j < n_jobs; ++j) total += jobs[j].W->rows;
  jobs_ctx c = {backend, jobs, n_jobs};
  if (!pool || efo_pool_size(pool) <= 1) {
    jobs_body(&c, 0, 0, total);
    return;
  }
  efo_pool_parallel_for(pool, total, jobs_body, &c, 32);
}

void efo_matvec(int backend, float* y, const efo_weight* W, const float* x, efo_pool* pool) {
  const efo_job j = {y, W, x};
  efo_matvec_jobs(backend, &j, 1, pool);
}

/* Row r as FP32: BF16 widening or exact dequantization (src/qkernels.cpp:299-305). */
void efo_row_f32(float* out, const efo_weight* W, size_t r) {
  uint64_t rb = 0;
  if (efo_row_bytes(W->qtype, W->cols, &rb)) return;
  efo_dequantize_row(W->qtype, W->data + r * rb, W->cols, out);
}
