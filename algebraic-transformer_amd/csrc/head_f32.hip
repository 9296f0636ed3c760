// Fused algebraic likelihood head for f32 hidden states on gfx950.
//
// fused_head.py:168 casts E to h's dtype and the model's compute dtype is a parameter
// (model.py:57), so the head also runs on f32 h (and E). This file is the reference's schedule
// in f32 throughout (fused_head.py:72-156, 194-216; nothing is rounded to bf16):
//  * forward: z^T = E h^T per 128 vocab x 128 token tile; the epilogue keeps, per token and
//    vocabulary tile, the partial sum of w = rho(min(z/c, X))^n and the target logit
//    (fused_head.py:83-103); head.hip's statistics kernels then form stat, pt and the
//    objective;
//  * backward: z = h E^T again, dZ = s (p - y) r written f32 token-major
//    (fused_head.py:120-146), then dh = dZ E (fused_head.py:147) and dE = dZ^T h
//    (fused_head.py:215);
//  * evaluation head: like the bf16 one (weights relative to each group's largest logit, the
//    argmax in jnp.argmax order), finished by head.hip's evaluation statistics kernel.
//
// Products run on v_mfma_f32_32x32x2f32 (f32 operands, f32 accumulation) over 128 x 128
// workgroup tiles: 4 waves (2 x 2), each a 64 x 64 block of 2 x 2 MFMA tiles. Every 16-deep k
// step is loaded into registers one step ahead (16-byte loads along the operand's contiguous
// dimension, zeros outside the matrix or the product's k range) and stored into a
// double-buffered LDS tile laid out [m or n][k] with a padded row pitch. An MFMA takes one k
// value from each lane half, and the MFMA j of a step pairs k = j (lanes 0-31) with k = j + 8
// (lanes 32-63), so the eight operands a lane needs per step and operand are two 16-byte LDS
// reads of its own row.
#include <algorithm>
#include <cmath>

#include "head_eval.h"
#include "head_params.h"
#include "launchers.h"

namespace alg {

constexpr int F_TM = 128, F_TN = 128;  // workgroup tile (m x n)
constexpr int F_TK = 16;               // k step
constexpr int F_WM = 2, F_WN = 2;      // wave grid
constexpr int F_NT = 64 * F_WM * F_WN;
constexpr int F_WT = 64;               // wave tile (m and n)
constexpr int F_PITCH = F_TK + 4;      // LDS row pitch (floats) of a [mn][k] tile
constexpr int F_TILE = 128 * F_PITCH;  // floats per operand tile
static_assert(F_TM == 128 && F_TN == 128 && F_WM * F_WT == F_TM && F_WN * F_WT == F_TN, "tile shape");

struct F32Op {
  const float* ptr;
  long ld;       // leading dimension (elements) of the stored matrix
  int mn_valid;  // extent of the m (A) or n (B) dimension
  int k_valid;   // end of the k range this product may read
};

// One operand tile (128 along m/n, 16 along k) is 512 chunks of 4 consecutive stored elements;
// thread t holds chunks t and t + 256. KM: stored [mn][k] (k contiguous), else [k][mn].
template <bool KM>
__device__ __forceinline__ void f32_load(const F32Op& op, int mn0, int k0, float (&c)[2][4]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int id = threadIdx.x + F_NT * j;
    const int mn = KM ? mn0 + (id >> 2) : mn0 + ((id & 31) << 2);
    const int k = KM ? k0 + ((id & 3) << 2) : k0 + (id >> 5);
    const bool line = KM ? mn < op.mn_valid : k < op.k_valid;  // the stored row exists
    const int c0 = KM ? k : mn;                                // first element along the row
    const int lim = KM ? op.k_valid : op.mn_valid;
    const float* src = op.ptr + (KM ? (long)mn * op.ld + k : (long)k * op.ld + mn);
    if (line && c0 + 4 <= lim) {
      const float4 x = *reinterpret_cast<const float4*>(src);
      c[j][0] = x.x; c[j][1] = x.y; c[j][2] = x.z; c[j][3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) c[j][e] = line && c0 + e < lim ? src[e] : 0.0f;
    }
  }
}

template <bool KM>
__device__ __forceinline__ void f32_store(float* tile, const float (&c)[2][4]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int id = threadIdx.x + F_NT * j;
    if constexpr (KM) {
      *reinterpret_cast<float4*>(tile + (id >> 2) * F_PITCH + ((id & 3) << 2)) =
          make_float4(c[j][0], c[j][1], c[j][2], c[j][3]);
    } else {
      const int kr = id >> 5, m = (id & 31) << 2;
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[(m + e) * F_PITCH + kr] = c[j][e];
    }
  }
}

// acc[mb][nb] = the wave's 32 x 32 block at rows wm*64 + mb*32 and columns wn*64 + nb*32 of
// the tile, summed over k in [kbeg, kend) (the operands' k_valid must not exceed kend).
template <bool AK, bool BK>
__device__ __forceinline__ void f32_mainloop(float (&sA)[2][F_TILE], float (&sB)[2][F_TILE], const F32Op& A,
                                             const F32Op& B, int m0, int n0, int kbeg, int kend,
                                             floatx16 (&acc)[2][2]) {
  const int lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / F_WN, wn = wave % F_WN;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
  const int nk = kend > kbeg ? (kend - kbeg + F_TK - 1) / F_TK : 0;
  if (nk == 0) return;
  float ca[2][4], cb[2][4];
  f32_load<AK>(A, m0, kbeg, ca);
  f32_load<BK>(B, n0, kbeg, cb);
  f32_store<AK>(sA[0], ca);
  f32_store<BK>(sB[0], cb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      f32_load<AK>(A, m0, kbeg + (kt + 1) * F_TK, ca);
      f32_load<BK>(B, n0, kbeg + (kt + 1) * F_TK, cb);
    }
    float a[2][8], b[2][8];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float* src = sA[cur] + (wm * F_WT + mb * 32 + l32) * F_PITCH + 8 * hf;
      const float4 x = *reinterpret_cast<const float4*>(src), y = *reinterpret_cast<const float4*>(src + 4);
      a[mb][0] = x.x; a[mb][1] = x.y; a[mb][2] = x.z; a[mb][3] = x.w;
      a[mb][4] = y.x; a[mb][5] = y.y; a[mb][6] = y.z; a[mb][7] = y.w;
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float* src = sB[cur] + (wn * F_WT + nb * 32 + l32) * F_PITCH + 8 * hf;
      const float4 x = *reinterpret_cast<const float4*>(src), y = *reinterpret_cast<const float4*>(src + 4);
      b[nb][0] = x.x; b[nb][1] = x.y; b[nb][2] = x.z; b[nb][3] = x.w;
      b[nb][4] = y.x; b[nb][5] = y.y; b[nb][6] = y.z; b[nb][7] = y.w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma_f32(a[mb][j], b[nb][j], acc[mb][nb]);
    if (more) {
      f32_store<AK>(sA[cur ^ 1], ca);
      f32_store<BK>(sB[cur ^ 1], cb);
    }
    __syncthreads();
  }
}

// Row of acc element i (of a 32 x 32 block) for lane half hf; the column is the lane (l32).
__device__ __forceinline__ int f32_row(int i, int hf) { return 8 * (i >> 2) + 4 * hf + (i & 3); }

struct F32Wave {
  int lane, hf, l32, wm, wn;
  __device__ F32Wave() {
    lane = threadIdx.x & 63;
    hf = lane >> 5;
    l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave / F_WN;
    wn = wave % F_WN;
  }
};

// Forward: z^T = E h^T (m = vocabulary, n = tokens), per-token partial sums of w over the tile's
// vocabulary rows and the target logit (fused_head.py:83-103).
__global__ __launch_bounds__(F_NT) void head_fwd_f32_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) float sA[2][F_TILE], sB[2][F_TILE];
  __shared__ float red[F_WM][F_TN];
  const int nbm = (p.V + F_TM - 1) / F_TM, nbn = (p.N + F_TN - 1) / F_TN;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * F_TM, n0 = tn * F_TN;
  const F32Op A{p.E32, p.d, p.V, p.d}, B{p.h32, p.d, p.N, p.d};
  floatx16 acc[2][2];
  f32_mainloop<true, true>(sA, sB, A, B, m0, n0, 0, p.d, acc);
  const F32Wave w;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int col = w.wn * F_WT + nb * 32 + w.l32;
    const int tok = n0 + col;
    const int tgt = tok < p.N ? p.targets[tok] : -1;
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = m0 + w.wm * F_WT + mb * 32 + f32_row(i, w.hf);
        if (v >= p.V) continue;
        const float z = acc[mb][nb][i];
        float r;
        part += pow2n<0>(rho_fast(fminf(z * p.inv_c, p.clamp), r), p.log2n);  // fused_head.py:98-100
        if (v == tgt) p.zt[tok] = z;
      }
    part += __shfl_xor(part, 32, 64);  // the other lane half holds the tile's other rows
    if (w.hf == 0) red[w.wm][col] = part;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < F_TN; t += F_NT) {
    const int tok = n0 + t;
    if (tok < p.N) p.partial[(size_t)tm * p.N + tok] = red[0][t] + red[1][t];
  }
}

// Backward, logit gradient: z = h E^T (m = tokens, n = vocabulary, so the f32 stores run along
// the vocabulary), dZ = ((p - y) r) s with p = (rho(x) stat)^n (fused_head.py:133-146).
__global__ __launch_bounds__(F_NT) void head_dz_f32_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) float sA[2][F_TILE], sB[2][F_TILE];
  const int nbm = (p.N + F_TM - 1) / F_TM, nbn = (p.V + F_TN - 1) / F_TN;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * F_TM, n0 = tn * F_TN;
  const F32Op A{p.h32, p.d, p.N, p.d}, B{p.E32, p.d, p.V, p.d};
  floatx16 acc[2][2];
  f32_mainloop<true, true>(sA, sB, A, B, m0, n0, 0, p.d, acc);
  const F32Wave w;
  const float scale = head_grad_scale(p);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = m0 + w.wm * F_WT + mb * 32 + f32_row(i, w.hf);
      if (tok >= p.N) continue;
      const int tgt = p.targets[tok];
      const float st = p.stat[tok];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int v = n0 + w.wn * F_WT + nb * 32 + w.l32;
        if (v >= p.V) continue;
        float r;
        const float t = pow2n<0>(rho_fast(fminf(acc[mb][nb][i] * p.inv_c, p.clamp), r) * st, p.log2n);
        const float y = v + p.v_off == tgt ? 1.0f : 0.0f;
        p.dz32[(size_t)tok * p.Vp + v] = (t - y) * r * scale;
      }
    }
}

// dh = dZ E: A = dZ stored [token][v] (k contiguous), B = E stored [v][d] (n contiguous). With
// several vocabulary splits each workgroup writes its f32 partial for head_dh_f32_reduce_kernel.
__global__ __launch_bounds__(F_NT) void head_dh_f32_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) float sA[2][F_TILE], sB[2][F_TILE];
  const int nbm = (p.N + F_TM - 1) / F_TM, nbn = (p.d + F_TN - 1) / F_TN;
  int tr, tn;
  xcd_tile_rowmajor(blockIdx.x, nbm * p.dh_split, nbn, tr, tn);
  const int tm = tr / p.dh_split, split = tr - tm * p.dh_split;
  const int m0 = tm * F_TM, n0 = tn * F_TN;
  const int kbeg = min(p.V, split * p.dh_kchunk), kend = min(p.V, kbeg + p.dh_kchunk);
  const F32Op A{p.dz32, p.Vp, p.N, kend}, B{p.E32, p.d, p.d, kend};
  floatx16 acc[2][2];
  f32_mainloop<true, false>(sA, sB, A, B, m0, n0, kbeg, kend, acc);
  const F32Wave w;
  float* out = p.dh_split > 1 ? p.dh_part + (size_t)split * p.N * p.d : p.dh32;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = m0 + w.wm * F_WT + mb * 32 + f32_row(i, w.hf);
      if (tok >= p.N) continue;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int col = n0 + w.wn * F_WT + nb * 32 + w.l32;
        if (col >= p.d) continue;
        if (p.dh_accum) out[(size_t)tok * p.d + col] += acc[mb][nb][i];  // a later vocabulary chunk
        else out[(size_t)tok * p.d + col] = acc[mb][nb][i];
      }
    }
}

// dh = sum over the vocabulary splits of the partials, added in split order.
__global__ __launch_bounds__(256) void head_dh_f32_reduce_kernel(HeadParams p) {
  const size_t plane = (size_t)p.N * p.d;
  for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < plane / 4; c += (size_t)gridDim.x * 256) {
    float4 a = reinterpret_cast<const float4*>(p.dh_part)[c];
    for (int s = 1; s < p.dh_split; ++s) {
      const float4 x = reinterpret_cast<const float4*>(p.dh_part + s * plane)[c];
      a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
    }
    reinterpret_cast<float4*>(p.dh32)[c] = a;
  }
}

// dE = dZ^T h: A = dZ stored [token][v] (m contiguous), B = h stored [token][d] (n contiguous).
__global__ __launch_bounds__(F_NT) void head_de_f32_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) float sA[2][F_TILE], sB[2][F_TILE];
  const int nbm = (p.V + F_TM - 1) / F_TM, nbn = (p.d + F_TN - 1) / F_TN;
  int tm, tn;
  xcd_tile_rowmajor(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * F_TM, n0 = tn * F_TN;
  const F32Op A{p.dz32, p.Vp, p.V, p.N}, B{p.h32, p.d, p.d, p.N};
  floatx16 acc[2][2];
  f32_mainloop<false, false>(sA, sB, A, B, m0, n0, 0, p.N, acc);
  const F32Wave w;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int v = m0 + w.wm * F_WT + mb * 32 + f32_row(i, w.hf);
      if (v >= p.V) continue;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int col = n0 + w.wn * F_WT + nb * 32 + w.l32;
        if (col >= p.d) continue;
        const size_t o = (size_t)v * p.d + col;
        if (p.dE_f32) reinterpret_cast<float*>(p.dE)[o] = acc[mb][nb][i];
        else reinterpret_cast<bf16*>(p.dE)[o] = f2bf(acc[mb][nb][i]);
      }
    }
}

// Evaluation head: z^T = E h^T as in the forward; per token and vocabulary tile the largest
// logit with its first index, the sum of weights relative to it and the target logit
// (src/algebraic/evaluation.py:13-23, src/algebraic/benchmarking.py:178-188).
__global__ __launch_bounds__(F_NT) void head_eval_f32_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) float sA[2][F_TILE], sB[2][F_TILE];
  __shared__ float red[F_WM][F_TN];
  __shared__ float redm[F_WM][F_TN];
  __shared__ int redi[F_WM][F_TN];
  const int nbm = (p.V + F_TM - 1) / F_TM, nbn = (p.N + F_TN - 1) / F_TN;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * F_TM, n0 = tn * F_TN;
  const F32Op A{p.E32, p.d, p.V, p.d}, B{p.h32, p.d, p.N, p.d};
  floatx16 acc[2][2];
  f32_mainloop<true, true>(sA, sB, A, B, m0, n0, 0, p.d, acc);
  const F32Wave w;
  const float inv_c = p.inv_c;
  const int vrow0 = m0 + w.wm * F_WT;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int col = w.wn * F_WT + nb * 32 + w.l32;
    const int tok = n0 + col;
    const int tgt = tok < p.N ? p.targets[tok] : -1;
    // The lane's largest logit and its first index (its rows increase with (mb, i)), and the
    // target logit.
    float zm = -INFINITY;
    int im = EVAL_NO_INDEX;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vrow0 + mb * 32 + f32_row(i, w.hf);
        const float z = acc[mb][nb][i];
        if (v < p.V) {
          if (!(z <= zm) && zm == zm) { zm = z; im = v; }
          if (v == tgt) p.zt[tok] = z;
        }
      }
    const float sh = eval_rho(-zm * inv_c);
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vrow0 + mb * 32 + f32_row(i, w.hf);
        if (v < p.V) part += pow2n<0>(eval_rho(acc[mb][nb][i] * inv_c) * sh, p.log2n);
      }
    // Merge with the other lane half (the same token's other rows of this wave's block).
    const float pz = __shfl_xor(zm, 32, 64);
    const float pp = __shfl_xor(part, 32, 64);
    const int pi = __shfl_xor(im, 32, 64);
    const bool take = pi != EVAL_NO_INDEX && eval_better(pz, pi, zm, im);
    const float zn = take ? pz : zm;
    const float mine = part == 0.0f ? 0.0f : part * eval_rescale<0>(zm, zn, inv_c, p.log2n);
    const float other = pp == 0.0f ? 0.0f : pp * eval_rescale<0>(pz, zn, inv_c, p.log2n);
    if (take) { zm = pz; im = pi; }
    if (w.hf == 0) { red[w.wm][col] = mine + other; redm[w.wm][col] = zm; redi[w.wm][col] = im; }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < F_TN; t += F_NT) {
    const int tok = n0 + t;
    float m = -INFINITY;
    int ix = EVAL_NO_INDEX;
#pragma unroll
    for (int wm = 0; wm < F_WM; ++wm)  // the waves cover increasing vocabulary rows
      if (redi[wm][t] != EVAL_NO_INDEX && eval_better(redm[wm][t], redi[wm][t], m, ix)) { m = redm[wm][t]; ix = redi[wm][t]; }
    float s = 0.0f;
#pragma unroll
    for (int wm = 0; wm < F_WM; ++wm)
      if (red[wm][t] != 0.0f) s += red[wm][t] * eval_rescale<0>(redm[wm][t], m, inv_c, p.log2n);
    if (tok < p.N) {
      p.partial[(size_t)tm * p.N + tok] = s;
      p.pmax[(size_t)tm * p.N + tok] = m;
      p.pidx[(size_t)tm * p.N + tok] = ix;
    }
  }
}

int head_f32_vocab_tiles(int V) { return (V + F_TM - 1) / F_TM; }

// Vocabulary splits of the dh product: double them while the product has fewer than about
// 1024 workgroups (4 per CU) and each split keeps at least 256 vocabulary entries.
int head_f32_dh_split(int N, int d, int V) {
  const long tiles = (long)((N + F_TM - 1) / F_TM) * ((d + F_TN - 1) / F_TN);
  int s = 1;
  while (s < 32 && tiles * s < 1024 && V / (2 * s) >= 256) s *= 2;
  return s;
}
// Vocabulary entries per split: a multiple of the k step (so every split starts 16-byte aligned).
int head_f32_dh_kchunk(int V, int split) { return ((V + split - 1) / split + F_TK - 1) / F_TK * F_TK; }

hipError_t launch_head_fwd_f32(const HeadParams& p, hipStream_t st) {
  const int tiles = head_f32_vocab_tiles(p.V) * ((p.N + F_TN - 1) / F_TN);
  {
    KTimer t("head_fwd_f32", st);
    hipLaunchKernelGGL(head_fwd_f32_kernel, dim3(tiles), dim3(F_NT), 0, st, p);
  }
  return launch_head_stats(p, head_f32_vocab_tiles(p.V), st);
}

hipError_t launch_head_bwd_f32(const HeadParams& p, hipStream_t st) {
  const int ntok = (p.N + F_TM - 1) / F_TM, nd = (p.d + F_TN - 1) / F_TN;
  {
    KTimer t("head_dz_f32", st);
    hipLaunchKernelGGL(head_dz_f32_kernel, dim3(ntok * head_f32_vocab_tiles(p.V)), dim3(F_NT), 0, st, p);
  }
  {
    KTimer t("head_dh_f32", st);
    hipLaunchKernelGGL(head_dh_f32_kernel, dim3(ntok * nd * p.dh_split), dim3(F_NT), 0, st, p);
  }
  if (p.dh_split > 1) {
    const size_t chunks = (size_t)p.N * p.d / 4;
    const int blocks = (int)std::min<size_t>((chunks + 255) / 256, 4096);
    KTimer t("head_dh_f32_reduce", st);
    hipLaunchKernelGGL(head_dh_f32_reduce_kernel, dim3(blocks), dim3(256), 0, st, p);
  }
  {
    KTimer t("head_de_f32", st);
    hipLaunchKernelGGL(head_de_f32_kernel, dim3(head_f32_vocab_tiles(p.V) * nd), dim3(F_NT), 0, st, p);
  }
  return hipGetLastError();
}

// Streamed backward in f32: per vocabulary chunk of `chunk` rows the logit gradient (N,
// pitch(chunk)) in p.dz32, then the chunk's dh product added into dh32 (written by the first
// chunk) and its dE rows.
hipError_t launch_head_bwd_f32_streamed(const HeadParams& p, int chunk, hipStream_t st) {
  const int ntok = (p.N + F_TM - 1) / F_TM, nd = (p.d + F_TN - 1) / F_TN;
  const int nchunks = (p.V + chunk - 1) / chunk;
  for (int k = 0; k < nchunks; ++k) {
    HeadParams q = head_vocab_chunk(p, k * chunk, std::min(chunk, p.V - k * chunk));
    q.dh_split = 1;
    q.dh_kchunk = head_f32_dh_kchunk(q.V, 1);
    q.dh_part = nullptr;
    q.dh_accum = k > 0;
    const int vt = head_f32_vocab_tiles(q.V);
    { KTimer t("head_dz_f32", st); hipLaunchKernelGGL(head_dz_f32_kernel, dim3(ntok * vt), dim3(F_NT), 0, st, q); }
    { KTimer t("head_dh_f32", st); hipLaunchKernelGGL(head_dh_f32_kernel, dim3(ntok * nd), dim3(F_NT), 0, st, q); }
    { KTimer t("head_de_f32", st); hipLaunchKernelGGL(head_de_f32_kernel, dim3(vt * nd), dim3(F_NT), 0, st, q); }
  }
  return hipGetLastError();
}

hipError_t launch_head_eval_f32(const HeadParams& p, hipStream_t st) {
  const int tiles = head_f32_vocab_tiles(p.V) * ((p.N + F_TN - 1) / F_TN);
  {
    KTimer t("head_eval_f32", st);
    hipLaunchKernelGGL(head_eval_f32_kernel, dim3(tiles), dim3(F_NT), 0, st, p);
  }
  return launch_head_eval_stats(p, head_f32_vocab_tiles(p.V), st);
}

}  // namespace alg
