// Parameters of the attention prologue and range guard kernels.
#pragma once

#include "common.h"
#include "ktimer.h"

namespace alg {

struct PrepParams {
  const void* q; const void* k; const void* v;
  void* q_s;
  float* part;      // (nblocks, 3) partial maxima
  size_t rows;      // B*H*T
  int D;
  float alpha;
  int want_guard;
};

struct GuardParams {
  const float* part; int nblocks;
  const float* sink_logit; int sink_count;  // broadcast to H (count 1 or H), or nullptr
  float* sink_out; int H;
  float c;
  int* flag;
  float q2k2_bound;   // (bound/1.01)^2
  float sink_bound;   // bound/1.01
  float v_bound;      // min(1e8, 1e37/((T+has_sink)(2 bound+1)^n))
  int want_guard;
};

// Fused prologue (QK RMS norm + gain, Cayley rotation, q pre-scale, guard maxima).
struct QkPrologueParams {
  const void* q; const void* k; const void* v;  // raw projections in `layout`
  const float* q_gain; const float* k_gain;     // (D,) or nullptr (no gain)
  const float* cos; const float* sin;           // (T, D/2) or nullptr (no rotation)
  void* q_s; void* k_r;                         // outputs in `layout`
  float* tau_q; float* tau_k;                   // (B, H, T) 1/rms per row
  float* part;                                  // (nblocks, 3) guard maxima
  int B, H, T, D;
  int layout;                                   // 0: (B, H, T, D), 1: (B, T, H, D)
  float eps, alpha;
  int want_guard;
};

struct QkPrologueBwdParams {
  const void* q; const void* k;                 // raw projections in `layout`
  const float* q_gain; const float* k_gain;
  const float* cos; const float* sin;
  const float* tau_q; const float* tau_k;
  const void* dq_r; const void* dk_r;           // cotangents of the rotated rows, in `layout`
  void* dq; void* dk;                           // outputs in `layout`
  float* gpart;                                 // (2, D, nblocks) gain-gradient partials
  int B, H, T, D;
  int layout;
};

}  // namespace alg
