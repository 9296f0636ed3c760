// Parameters of the fused-head kernels.
#pragma once

#include "common.h"
#include "ktimer.h"
#include "gemm_core.h"

namespace alg {

constexpr int HT_M = 256, HT_N = 256;  // head GEMM workgroup tile
#ifndef ALG_HEAD_WM
#define ALG_HEAD_WM 2                  // waves along the tile's m dimension
#endif
#ifndef ALG_HEAD_WN
#define ALG_HEAD_WN 4                  // waves along the tile's n dimension
#endif

struct HeadParams {
  const bf16* h;        // (N, d)
  const bf16* E;        // (V, d), already in h's dtype (fused_head.py:168)
  const int* targets;   // (N,)
  int N, d, V, Npad;    // Npad = N rounded up to the GEMM tile
  int Vp;               // row pitch of the token-major U / dZ: V rounded up to 8
  int log2n;
  float inv_c, c, clamp;
  float* partial;       // (ceil(V/HT_M), N) per-vocab-tile row sums
  float* stat;          // (N,)
  float* zt;            // (N,)
  float* pt;            // (N,)
  float* obj_part;      // (nblocks,)
  float* obj;           // (1,)
  const float* g;       // (1,) cotangent of the objective
  bf16* ut;             // residual (Npad, Vp): bf16(w r), target entry (w_t - l) r_t; or nullptr
  float* lsum;          // residual (N,): l = sum_v w; or nullptr
  bf16* dzt;            // recompute path workspace (Npad, Vp): bf16(s (p - y) r)
  bf16* hs;             // residual path workspace (N, d): bf16(s h / l)
  bf16* dh;             // (N, d)
  float* dh_part;       // split-K partials of dh (dh_split, N, d) f32, or nullptr (one split)
  int dh_split;         // k splits of the dh product (1: none)
  int dh_kchunk;        // vocabulary entries per split (a multiple of 128)
  void* dE;             // (V, d) bf16 or f32
  int dE_f32;
  // dE tiles past the last complete round of workgroups, split over the tokens (head_de_plan):
  float* de_part = nullptr;  // (tiles - de_full) * de_split f32 tiles of HT_M x HT_N, or nullptr
  int de_full = 0;      // tiles computed whole (all of them when de_split is 1)
  int de_split = 1;     // token ranges per remaining tile
  int de_kchunk = 0;    // tokens per range (a multiple of 128)
  // Streamed backward (one vocabulary chunk per launch group): E, dE and the logit gradient
  // cover rows [v_off, v_off + V) of the vocabulary, and the dh product accumulates over
  // the chunks in an f32 (N, d) buffer.
  int v_off = 0;        // vocabulary index of E's first row (targets are compared with v + v_off)
  int dh_accum = 0;     // dh product: 0 writes, 1 adds into the f32 accumulator (dh_part, or
                        // dh32 for f32 hidden states), 2 writes bf16(accumulator + product)
  float* pmax;          // eval: (ceil(V/HT_M), N) per-vocab-tile maximum logit
  int* pidx;            // eval: (ceil(V/HT_M), N) its vocabulary index
  float* logprob;       // eval: (N,) log p(target)
  int* argmax;          // eval: (N,) argmax_v z
  // f32 hidden states (the head_f32 kernels; the bf16 pointers above are then unused):
  const float* h32;     // (N, d)
  const float* E32;     // (V, d), already cast to f32
  float* dz32;          // recompute workspace (N, Vp): s (p - y) r, token-major
  float* dh32;          // (N, d)
};

typedef GemmCfg<HT_M, HT_N, ALG_HEAD_WM, ALG_HEAD_WN> HeadGemm;

// Scale of the logit gradient, g n / (c N) (fused_head.py:249-251).
__device__ __forceinline__ float head_grad_scale(const HeadParams& p) {
  return p.g[0] * (((float)(1 << p.log2n) * p.inv_c) / (float)p.N);
}

// ALU-GLU feed-forward products with fused activation epilogues (model.py:185-193).
struct FfnParams {
  const bf16* h2;       // (N, d) block input after its norm
  const bf16* w_gu;     // (d, 2F) = [w_g | w_u]
  bf16* y;              // (N, F) gate * alu(up)
  bf16* gate;           // (N, F) residual for the backward
  bf16* up;             // (N, F) residual for the backward
  const bf16* dout;     // (N, dm) cotangent of the block output
  const bf16* w_d;      // (F, dm)
  bf16* d_gu;           // (N, 2F) = [d_gate | d_up]
  int N, d, F, dm;
  float beta;
};

// Plain bf16 products of the feed-forward block: C (M, N) row-major = A B, f32 accumulation.
struct FfnGemmParams {
  GemmOperand A, B;     // A: M x K, B: K x N, each k- or m/n-contiguous as stored
  bf16* C;              // (M, ldc)
  long ldc;
  int M, N, K;
  float* part;          // f32 tiles of the split tiles (ffn_gemm_plan), or nullptr
  int full;             // tiles computed whole
  int split;            // k ranges per remaining tile
  int kchunk;           // k per range (a multiple of 128)
};

// Row RMS norm with gain (the final norm before the head, model.py:208).
struct RmsNormParams {
  const bf16* x;        // (rows, d)
  const float* gain;    // (d,) or nullptr
  bf16* y;              // forward output (rows, d)
  float* tau;           // (rows,) 1/rms, written by the forward, read by the VJP
  const bf16* dy;       // VJP: cotangent of y
  bf16* dx;             // VJP: (rows, d)
  float* gpart;         // VJP: (nblocks, d) gain-gradient partials and their group sums, or nullptr
  int rows, d;
  float eps;
};

}  // namespace alg
