// Parameters and variant selection shared by the attention kernels.
#pragma once

#include "common.h"
#include "ktimer.h"

namespace alg {

// Variants of the asinh-power kernel (src/algebraic/kernels/flash.py:59-73, 732-760, 850-852):
//   INRANGE  unshifted, unclipped, stat = 1/Z (the guarded "low" variant, bounded_scores)
//   CLIPPED  unshifted with x = min(s, clamp) (range_guard=False defaults); stat 1/Z or Z^(-1/n)
//   SHIFTED  running-max accumulation (the guarded "high" fallback or explicit shift=True)
enum AttnMode { MODE_INRANGE = 0, MODE_CLIPPED = 1, MODE_SHIFTED = 2 };

struct AttnFwdParams {
  const void* q;       // (B,H,T,D) pre-scaled queries q_s = round(q * alpha)
  const void* k;       // (B,H,T,D)
  const void* v;       // (B,H,T,D)
  const float* sink;   // (H,) sink logit / c, or nullptr
  const int* flag;     // device guard flag (nonzero = in range) or nullptr (always run)
  void* o;             // (B,H,T,D) output in the input dtype
  float* o_precise;    // (B,H,T,D) f32 output (SHIFTED with precise output) or nullptr
  float* stat;         // (B,H,T) f32 row statistic
  int B, H, T;
  int log2n;           // n = 2^log2n
  float clamp;         // CLIPPED: positive-score clamp
  int fast_rho;        // SHIFTED: fast rho for the weights
  int inv_stat;        // CLIPPED: 1 -> stat = 1/Z, 0 -> stat = Z^(-1/n)
};

struct AttnBwdParams {
  const void* q;       // q_s
  const void* k;
  const void* v;
  const void* o;       // forward output in the input dtype (di source in range)
  const float* o_precise;  // f32 forward output (di source when shifted) or nullptr
  const void* dO;      // (B,H,T,D) upstream cotangent in the input dtype
  const float* stat;   // (B,H,T)
  const float* sink;   // (H,) or nullptr
  const int* flag;
  float* di;           // (B,H,T) f32, written by the pre kernel
  float* dq_acc;       // (B,H,T,D) f32 accumulator (workspace)
  float* sink_part;    // (B*H*nblk) f32 partial sums of mass*di (workspace)
  void* dq;            // (B,H,T,D) output
  void* dk;
  void* dv;
  float* dbeta;        // (H,) gradient w.r.t. sink/c
  int B, H, T;
  int log2n;
  float clamp;
  int fast_rho;
  int inv_stat;
  int mode;            // AttnMode selected by the host when flag is nullptr
  float dq_scale;      // chain-rule factor applied after the slope (alpha), or 1
};

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// LDS row padding (elements) of the bf16 tiles: row pitch = width + pad, chosen against
// bank conflicts of the row-fragment and transposed (ds_read_b64_tr_b16) reads.
#ifndef ALG_FWD_PAD
#define ALG_FWD_PAD 8
#endif
#ifndef ALG_BWD_PAD
#define ALG_BWD_PAD 8
#endif
#ifndef ALG_BWD_SPAD
#define ALG_BWD_SPAD 8
#endif

}  // namespace alg
