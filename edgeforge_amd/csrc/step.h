// Persistent decode step (step.hip): one cooperative launch of one 1024-thread workgroup per CU
// runs the embedding lookup and every layer of a one-sequence decode step, its phases separated by
// grid barriers instead of kernel boundaries.
#pragma once

#include "common.h"

namespace efh {

constexpr int kStepThreads = 512;
// Static LDS of the step kernel: two weight regions (each phase's rows of this workgroup, fetched
// one or two phases ahead), the staged activation and its norm weights.
constexpr int kStepRegion0 = 64 * 1024;
constexpr int kStepRegion1 = 32 * 1024;
constexpr int kStepMaxK = 6144;      // longest activation a phase stages
constexpr int kStepMaxNormK = 2048;  // longest activation with a fused RMSNorm

enum StepPhaseKind : int { kPhaseGemv = 0, kPhaseAttention = 1 };

// One matrix of a GEMV phase; its rows are rows [row0, row0 + rows) of the phase.
struct StepJob {
  const uint8_t* W;
  const uint8_t* W2;  // the up projection of a SwiGLU phase (same shape as W)
  float* y;
  int rows, row_bytes, qtype, row0;
};

struct StepPhase {
  int kind;
  int epi;     // kEpiStore / kEpiResidual / kEpiSwiglu
  int K;       // activation length
  int n_jobs;  // 1..3
  int rows;    // rows of all jobs
  int rpw;     // rows per workgroup
  int region;  // LDS region of this phase's weights (0 or 1)
  int own;     // 1: the phase fetches its own weights (nothing fetched them earlier)
  int pf;      // phase whose weights this phase fetches when it ends (-1: none)
  int embed;   // 1: the activation is the embedding row of the step's token (written to x too)
  const float* x;
  const float* norm_w;  // fused RMSNorm weights or null
  float eps;
  float* kc;  // attention: this layer's cache rows [max_seq][KV * hd]
  float* vc;
  StepJob job[3];
};

struct PersistentArgs {
  const StepPhase* phases;
  int n_phases;
  const int32_t* pos_dev;
  const int32_t* hist;  // the step's token is hist[*pos_dev]
  const uint8_t* embed;
  int embed_qtype;
  long embed_rows, embed_rb;
  float* x;  // residual stream [D]
  int D;
  const float* q;  // attention inputs (the q/k/v phase's outputs) and output
  const float* knew;
  const float* vnew;
  float* ctx;
  const float* cos_t;
  const float* sin_t;
  int H, KV, hd, max_seq;
  float scale;
  unsigned* sync;  // kStepSyncWords words: epoch, error, arrival flags
};

constexpr int kStepMaxGroups = 1024;
constexpr size_t kStepSyncWords = 64 + 16 * kStepMaxGroups;

// Why a model / engine cannot take the persistent step (empty when it can).
std::string step_unsupported(const StepPhase* phases, int n_phases, int groups, int hd, int H, int KV, int max_seq,
                             int D);
// Workgroups of one launch: one per CU.
int step_groups();
// Why the device cannot run the step kernel's grid at once (empty when it can).
std::string step_launch_unsupported();
int launch_step(const PersistentArgs& a, hipStream_t s);

}  // namespace efh
