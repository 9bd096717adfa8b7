/* EdgeForge CPU oracle (test infrastructure only): 16-bit float conversions and the Q4_0 / Q8_0
 * block codec, including the reference's scale-search quantizer.
 *
 * Restates include/ef/fp16.h:28-91 and src/quant.cpp:15-256. */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "efo.h"

static inline uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float float_of(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* bf16 -> f32 is the 16-bit shift (include/ef/fp16.h:28-30). */
float efo_bf16_to_f32(uint16_t h) { return float_of((uint32_t)h << 16); }

/* Round to nearest even; NaN truncated with the quiet bit forced (include/ef/fp16.h:32-40). */
uint16_t efo_f32_to_bf16(float f) {
  uint32_t u = bits_of(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* Exact binary16 -> binary32 with subnormals, inf and NaN payloads (include/ef/fp16.h:44-67).
 * A subnormal m * 2^-24 is normalised by counting the shifts that bring the leading 1 to bit 10. */
float efo_fp16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 31u;
  uint32_t m = h & 1023u;
  if (e == 31u) return float_of(sign | 0x7F800000u | (m << 13));
  if (e != 0u) return float_of(sign | ((e + 112u) << 23) | (m << 13));
  if (m == 0u) return float_of(sign);
  uint32_t shifts = 0;
  while (!(m & 1024u)) {
    m <<= 1;
    ++shifts;
  }
  return float_of(sign | ((113u - shifts) << 23) | ((m & 1023u) << 13));
}

/* binary32 -> binary16, round to nearest even, overflow to inf, quiet NaN keeps its top payload
 * bits (include/ef/fp16.h:69-91). */
uint16_t efo_f32_to_fp16(float f) {
  const uint32_t u = bits_of(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 1023u));
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* |f| >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                   /* result is subnormal or zero */
    if (a <= 0x33000000u) return sign;                     /* <= 2^-25: ties-to-even gives 0 */
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t sh = 126u - (a >> 23); /* 14..24 */
    uint32_t r = mant >> sh;
    const uint32_t rest = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rest > half || (rest == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  const uint32_t x = a - 0x38000000u; /* exponent rebias 127 -> 15 */
  return (uint16_t)(sign | ((x + 0xFFFu + ((x >> 13) & 1u)) >> 13));
}

void efo_fp16_to_f32_n(const uint16_t* h, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = efo_fp16_to_f32(h[i]);
}
void efo_f32_to_fp16_n(const float* f, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = efo_f32_to_fp16(f[i]);
}
void efo_f32_to_bf16_n(const float* f, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = efo_f32_to_bf16(f[i]);
}

/* ---- codec ---------------------------------------------------------------------------------- */

int efo_row_bytes(int qtype, uint64_t cols, uint64_t* out) { /* src/quant.cpp:136-149 */
  switch (qtype) {
    case EFO_F32: *out = cols * 4; return 0;
    case EFO_F16:
    case EFO_BF16: *out = cols * 2; return 0;
    case EFO_Q8_0:
    case EFO_Q4_0:
      if (cols % EFO_QK) return -1;
      *out = cols / EFO_QK * (qtype == EFO_Q8_0 ? EFO_Q8_BLOCK : EFO_Q4_BLOCK);
      return 0;
    default: return -1;
  }
}

static float round_to_fp16(float d) { return efo_fp16_to_f32(efo_f32_to_fp16(d)); } /* src/quant.cpp:20 */

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Codes for scale d (already fp16-rounded), and the squared reconstruction error in double. */
static double q4_codes_for(const float* x, size_t n, float d, uint8_t* codes) {
  const float inv = 1.0f / d;
  double sse = 0.0;
  for (size_t j = 0; j < n; ++j) {
    const int c = clampi((int)nearbyintf(x[j] * inv) + 8, 0, 15);
    codes[j] = (uint8_t)c;
    const double err = (double)x[j] - (double)((float)(c - 8) * d);
    sse += err * err;
  }
  return sse;
}

/* One symmetric 4-bit group (src/quant.cpp:26-99): candidate scales signed_max/-8 and, with the
 * search, amax/{7, 7.25, 7.5, 7.75, 8}; each is rounded to fp16 first and scored by SSE in
 * double; the first strictly best wins.  Then up to two least-squares refinements d = Σxc/Σc²
 * (kept only while the error strictly drops).  An all-zero, non-finite or fp16-underflowing
 * group gives d = 0 and codes 8. */
static float q4_group(const float* x, size_t n, int search, uint8_t* q) {
  float amax = 0.0f, smax = 0.0f;
  for (size_t j = 0; j < n; ++j) {
    const float a = fabsf(x[j]);
    if (a > amax) {
      amax = a;
      smax = x[j];
    }
  }
  if (!(amax > 0.0f) || !isfinite(amax)) {
    memset(q, 8, n);
    return 0.0f;
  }
  float cands[6];
  int nc = 0;
  cands[nc++] = smax / -8.0f;
  if (search) {
    static const float div[5] = {7.0f, 7.25f, 7.5f, 7.75f, 8.0f};
    for (int i = 0; i < 5; ++i) cands[nc++] = amax / div[i];
  }
  uint8_t trial[256];
  float best = 0.0f;
  double best_sse = -1.0;
  for (int c = 0; c < nc; ++c) {
    float v = cands[c];
    v = v < -65504.0f ? -65504.0f : (v > 65504.0f ? 65504.0f : v);
    const float d = round_to_fp16(v);
    if (d == 0.0f) continue;
    const double sse = q4_codes_for(x, n, d, trial);
    if (best_sse < 0.0 || sse < best_sse) {
      best_sse = sse;
      best = d;
      memcpy(q, trial, n);
    }
  }
  if (best_sse < 0.0) {
    memset(q, 8, n);
    return 0.0f;
  }
  if (!search) return best;
  for (int round = 0; round < 2; ++round) {
    double num = 0.0, den = 0.0;
    for (size_t j = 0; j < n; ++j) {
      const double c = (double)((int)q[j] - 8);
      num += (double)x[j] * c;
      den += c * c;
    }
    if (den == 0.0) break;
    double ls = num / den;
    ls = ls < -65504.0 ? -65504.0 : (ls > 65504.0 ? 65504.0 : ls);
    const float d = round_to_fp16((float)ls);
    if (d == 0.0f || d == best) break;
    const double sse = q4_codes_for(x, n, d, trial);
    if (!(sse < best_sse)) break;
    best_sse = sse;
    best = d;
    memcpy(q, trial, n);
  }
  return best;
}

/* Q4_0 block: fp16 d, then byte j = code j | code (j+16) << 4 (src/quant.cpp:151-156). */
void efo_quantize_block_q4_0(const float* x, uint8_t* out, int search) {
  uint8_t q[EFO_QK];
  const uint16_t d = efo_f32_to_fp16(q4_group(x, EFO_QK, search, q));
  out[0] = (uint8_t)(d & 0xFF);
  out[1] = (uint8_t)(d >> 8);
  for (int j = 0; j < 16; ++j) out[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

/* w[j] = (lo nibble of byte j - 8) d, w[j+16] = (hi nibble - 8) d (src/quant.cpp:158-164). */
void efo_dequantize_block_q4_0(const uint8_t* b, float* out) {
  const float d = efo_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  for (int j = 0; j < 16; ++j) {
    out[j] = (float)((b[2 + j] & 15) - 8) * d;
    out[j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
  }
}

/* Q8_0: d = fp16(amax / 127) (capped at 65504), codes nearbyint(x / d) in [-127, 127]
 * (src/quant.cpp:166-175). */
void efo_quantize_block_q8_0(const float* x, uint8_t* out) {
  float amax = 0.0f;
  for (int j = 0; j < EFO_QK; ++j) amax = fmaxf(amax, fabsf(x[j]));
  float d = 0.0f;
  if (amax > 0.0f && isfinite(amax)) d = round_to_fp16(fminf(amax / 127.0f, 65504.0f));
  const uint16_t h = efo_f32_to_fp16(d);
  out[0] = (uint8_t)(h & 0xFF);
  out[1] = (uint8_t)(h >> 8);
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  for (int j = 0; j < EFO_QK; ++j) out[2 + j] = (uint8_t)(int8_t)clampi((int)nearbyintf(x[j] * inv), -127, 127);
}

void efo_dequantize_block_q8_0(const uint8_t* b, float* out) { /* src/quant.cpp:177-180 */
  const float d = efo_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  for (int j = 0; j < EFO_QK; ++j) out[j] = (float)(int8_t)b[2 + j] * d;
}

int efo_quantize_row(int qtype, const float* x, size_t n, uint8_t* out, int search) { /* :182-217 */
  uint64_t rb;
  if (efo_row_bytes(qtype, n, &rb)) return -1;
  switch (qtype) {
    case EFO_F32: memcpy(out, x, n * 4); return 0;
    case EFO_F16:
      for (size_t i = 0; i < n; ++i) {
        const uint16_t h = efo_f32_to_fp16(x[i]);
        memcpy(out + 2 * i, &h, 2);
      }
      return 0;
    case EFO_BF16:
      for (size_t i = 0; i < n; ++i) {
        const uint16_t h = efo_f32_to_bf16(x[i]);
        memcpy(out + 2 * i, &h, 2);
      }
      return 0;
    case EFO_Q4_0:
      for (size_t b = 0; b < n / EFO_QK; ++b) efo_quantize_block_q4_0(x + b * EFO_QK, out + b * EFO_Q4_BLOCK, search);
      return 0;
    case EFO_Q8_0:
      for (size_t b = 0; b < n / EFO_QK; ++b) efo_quantize_block_q8_0(x + b * EFO_QK, out + b * EFO_Q8_BLOCK);
      return 0;
  }
  return -1;
}

int efo_dequantize_row(int qtype, const uint8_t* in, size_t n, float* out) { /* :219-249 */
  uint64_t rb;
  if (efo_row_bytes(qtype, n, &rb)) return -1;
  switch (qtype) {
    case EFO_F32: memcpy(out, in, n * 4); return 0;
    case EFO_F16:
    case EFO_BF16:
      for (size_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, in + 2 * i, 2);
        out[i] = qtype == EFO_F16 ? efo_fp16_to_f32(h) : efo_bf16_to_f32(h);
      }
      return 0;
    case EFO_Q4_0:
      for (size_t b = 0; b < n / EFO_QK; ++b) efo_dequantize_block_q4_0(in + b * EFO_Q4_BLOCK, out + b * EFO_QK);
      return 0;
    case EFO_Q8_0:
      for (size_t b = 0; b < n / EFO_QK; ++b) efo_dequantize_block_q8_0(in + b * EFO_Q8_BLOCK, out + b * EFO_QK);
      return 0;
  }
  return -1;
}

void efo_fake_quant_q4_group(const float* x, size_t n, float* out, int search) { /* :251-256 */
  uint8_t q[256];
  const size_t m = n < 256 ? n : 256;
  const float d = q4_group(x, m, search, q);
  for (size_t j = 0; j < m; ++j) out[j] = (float)(q[j] - 8) * d;
}

/* Row-parallel matrix quantization (each row is independent, so the bytes do not depend on the
 * thread count; the reference's writer has the same property, src/quantizer.cpp:38-60). */
typedef struct {
  int qtype, search;
  const float* w;
  size_t rows, cols, rb;
  uint8_t* out;
  int nthreads, tid;
} qm_task;

static void* qm_worker(void* arg) {
  const qm_task* t = (const qm_task*)arg;
  const size_t lo = t->rows * (size_t)t->tid / (size_t)t->nthreads;
  const size_t hi = t->rows * (size_t)(t->tid + 1) / (size_t)t->nthreads;
  for (size_t r = lo; r < hi; ++r) efo_quantize_row(t->qtype, t->w + r * t->cols, t->cols, t->out + r * t->rb, t->search);
  return NULL;
}

int efo_quantize_matrix(int qtype, const float* w, size_t rows, size_t cols, uint8_t* out, int search, int threads) {
  uint64_t rb;
  if (efo_row_bytes(qtype, cols, &rb)) return -1;
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  qm_task task[64];
  for (int i = 0; i < threads; ++i) {
    task[i] = (qm_task){qtype, search, w, rows, cols, (size_t)rb, out, threads, i};
    if (i > 0) pthread_create(&th[i], NULL, qm_worker, &task[i]);
  }
  qm_worker(&task[0]);
  for (int i = 1; i < threads; ++i) pthread_join(th[i], NULL);
  return 0;
}
