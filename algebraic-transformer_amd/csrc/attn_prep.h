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

}  // namespace alg
