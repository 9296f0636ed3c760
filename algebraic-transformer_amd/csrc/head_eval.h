// Helpers of the streamed evaluation head shared by the bf16 and f32 head kernels: the argmax
// order and the weights relative to a group's largest logit (src/algebraic/evaluation.py:13-23,
// src/algebraic/benchmarking.py:178-188).
#pragma once

#include "common.h"

namespace alg {

// Marks an empty running argmax (no vocabulary index seen yet).
constexpr int EVAL_NO_INDEX = 0x7fffffff;

// Argmax order over increasing vocabulary indices (jnp.argmax): the first NaN wins, else the
// first of the largest values. (z, i) replaces the running (zm, im) when it comes first in that
// order; the running value starts empty (EVAL_NO_INDEX).
__device__ __forceinline__ bool eval_better(float z, int i, float zm, int im) {
  if (im == EVAL_NO_INDEX) return true;
  if (zm != zm) return z != z && i < im;
  if (z != z) return true;
  return z > zm || (z == zm && i < im);
}

// Stable rho (reciprocal form below zero) with the hardware reciprocal: rho(x) = e^asinh(x).
__device__ __forceinline__ float eval_rho(float x) {
  const float rad = __builtin_fmaf(x, x, 1.0f);
  const float t = __builtin_fmaf(rad, rsq(rad), __builtin_fabsf(x));
  return x >= 0.0f ? t : __builtin_amdgcn_rcpf(t);
}

// Factor that moves a sum of weights relative to logit za onto logit zb >= za:
// (rho(za/c) rho(-zb/c))^n, exactly 1 when za == zb.
template <int L2N>
__device__ __forceinline__ float eval_rescale(float za, float zb, float inv_c, int log2n) {
  if (za == zb) return 1.0f;
  return pow2n<L2N>(eval_rho(za * inv_c) * eval_rho(-zb * inv_c), log2n);
}

}  // namespace alg
