// Launchers of the decode-step glue kernels (glue.hip).
#pragma once

#include "afrag.h"
#include "common.h"

namespace efh {

struct AttnArgs {
  const float* q;       // [batch][ldq] un-roped queries (H * hd)
  const float* knew;    // [batch][KV * hd] un-roped keys of the current position
  const float* vnew;    // [batch][KV * hd]
  float* kcache;        // this layer: [batch][max_seq][KV * hd] (roped keys)
  float* vcache;        // this layer: [batch][max_seq][KV * hd]
  const float* cos_t;   // [max_seq][hd / 2]
  const float* sin_t;
  const int32_t* pos_dev;
  const float* rope_now;  // cos then sin rows (hd / 2 each) at *pos_dev, or null (decode only)
  float* ctx;           // [batch][ldq]
  long ldq;
  int H, KV, hd, max_seq;
  float scale;          // float(1 / sqrt(hd))
  int pre_vrows;        // set by launch_attention: the first chunk's V rows have their own LDS
  int chunk;            // set by launch_attention: rows of the LDS staging buffer (>= 64)
  AEmit em;             // KV-group kernel: ctx also staged as the o-projection's tables (afrag.h)
  // Position-split decode (attention_split_kernel, then attention_combine_kernel): `splits`
  // workgroups per (sequence, KV group), each over `span` positions; part holds their partial
  // results.  part == nullptr: no split.
  float* part;
  int splits, span;
  int split_hpw;  // set by launch_attention: query heads per split workgroup (all of a group's, or half)
};

// Prefill of n positions per sequence at once: rows r = b * n + i hold position *pos_dev + i of
// sequence b; q / knew / vnew / ctx are [rows][...] with the strides of AttnArgs.
struct PrefillArgs {
  AttnArgs a;
  int n;
};
int launch_prefill_attention(const PrefillArgs& a, int rows, hipStream_t s);  // RoPE + cache write, then attention
int launch_embed_rows(const ef_hip_weight_s* W, const int32_t* hist, long hist_ld, const int32_t* pos_dev, int n,
                      int rows, float* out, long ldo, hipStream_t s);
int launch_advance_by(int32_t* pos_dev, int n, hipStream_t s);

// With rope_now, also copies the cos / sin table rows at *pos_dev there (half floats each).
int launch_embed_at(const ef_hip_weight_s* W, const int32_t* hist, long hist_ld, const int32_t* pos_dev, int batch,
                    float* out, long ldo, hipStream_t s, const float* cos_t = nullptr, const float* sin_t = nullptr,
                    int half = 0, float* rope_now = nullptr, const AEmit* em = nullptr);
size_t attention_lds_bytes(int hd, int max_seq);
// The position split for a decode step of `batch` sequences: whether it applies (hd = 64, at most 8
// query heads per KV head, more than one 64-position chunk of cache) and its splits / span (the
// smallest multiple of 64 positions that needs no more splits than the combine takes: 64 up to
// 2048 positions at 8 heads per KV head).  part_floats: the workspace it needs.
bool attention_split_plan(int H, int KV, int hd, int max_seq, int batch, int* splits, int* span, size_t* part_floats);
int launch_attention(const AttnArgs& a, int batch, hipStream_t s);
// Whether launch_attention runs the KV-group kernel (the one that can stage ctx as tables).
bool attention_uses_group(const AttnArgs& a, int batch);
int launch_rmsnorm(const float* x, const float* w, float eps, int n, long ld, int batch, float* out, hipStream_t s);
// With out_eos: eos_p[b] is stored beside the picked token (the chat loop's per-step P(EOS)).
int launch_finish_step(const int32_t* next, int batch, int32_t* hist, long hist_ld, int32_t* hist_len, int32_t* out,
                       long out_ld, const int32_t* n_prompt_dev, int32_t* pos_dev, hipStream_t s,
                       const double* eos_p = nullptr, double* out_eos = nullptr);
int launch_advance(int32_t* pos_dev, hipStream_t s);
// dst[r][0..n) = src[r][0..n) for rows r (4-byte words; strides lds / ldd in words), as a kernel:
// it touches only those words (a strided 2D runtime copy may treat pitch x height as its extent).
int launch_copy_rows(const void* src, long lds, void* dst, long ldd, int n, int rows, hipStream_t s);

}  // namespace efh
