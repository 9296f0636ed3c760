// Parameters of the fused-head kernels.
#pragma once

#include "common.h"
#include "ktimer.h"

namespace alg {

struct HeadParams {
  const bf16* h;        // (N, d)
  const bf16* E;        // (V, d), already in h's dtype (fused_head.py:168)
  const int* targets;   // (N,)
  int N, d, V, Npad;
  int log2n;
  float inv_c, c, clamp;
  float* partial;       // (nvt, N) per-vocab-tile row sums
  float* stat;          // (N,)
  float* zt;            // (N,)
  float* pt;            // (N,)
  float* obj_part;      // (nblocks,)
  float* obj;           // (1,)
  const float* g;       // (1,) cotangent of the objective
  bf16* dzt;            // (V, Npad) workspace
  bf16* dh;             // (N, d)
  void* dE;             // (V, d) bf16 or f32
  int dE_f32;
};

}  // namespace alg
