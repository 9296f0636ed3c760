// Fused tied-embedding algebraic likelihood head for gfx950.
//
// Replaces src/algebraic/kernels/fused_head.py:72-275 (forward statistics, telemetry,
// backward) including the XLA embedding-gradient matmul of fused_head.py:215.
//
// Forward (logits never stored): z^T = E h^T per 256 vocab x 256 token tile (bf16 MFMA, f32
// accumulate); the epilogue forms x = min(z/c, X), w = rho_fast(x)^n, r = rsqrt(1+x^2),
// per-token partial sums of w for this vocab tile and the target logit zt
// (fused_head.py:83-103). A statistics kernel reduces the partials in a fixed order:
// stat = l^(-1/n) (fused_head.py:116), telemetry pt = (rho(min(zt/c, X)) stat)^n and the
// objective mean(1 - pt) (fused_head.py:219-229).
//
// Backward, three schedules over the same GEMM core:
//  * residual (3 products): with p = w/l the logit gradient is
//        dz = s (p - y) r = (s/l) U',  U' = w r except U'_t = (w_t - l) r_t,
//    so the forward epilogue also stores U = bf16(w r) token-major and the statistics kernel
//    patches the target entries once l is known. Then dh = (s/l) (U' E) and
//    dE = U'^T (s h / l): no logit recompute.
//  * recompute (4 products, the reference's schedule, fused_head.py:120-156, 194-216): the
//    backward recomputes z, writes bf16(s (p - y) r) token-major, then dh = dZ E and
//    dE = dZ^T h.
//  * streamed (the recompute schedule one vocabulary chunk at a time, launch_head_bwd_streamed):
//    per chunk dZ of the chunk only, its dh product accumulated in f32 across the chunks and its
//    rows of dE, so no (N, V) block is held at all.
// Every product reads its operands in their natural layout (k-contiguous fragments via
// ds_read_b128, transposed ones via ds_read_b64_tr_b16).
#include <cmath>
#include <type_traits>

#include "gemm_core.h"
#include "head_eval.h"
#include "head_params.h"
#include "launchers.h"

namespace alg {

typedef HeadGemm HC;
constexpr int NT = HC::THREADS;

__device__ __forceinline__ float head_w(float z, const HeadParams& p, float& r) {
  const float x = fminf(z * p.inv_c, p.clamp);  // fused_head.py:98
  float t = rho_fast(x, r);
  for (int e = 0; e < p.log2n; ++e) t = t * t;
  return t;
}

// Token-major staging of a wave's WTM (v) x WTN (tok) block of a bf16 (tok, v) matrix (the
// forward's residual U, the recompute schedules' logit gradient dZ): the wave writes its block
// into its own share of the idle pipeline buffers as [tok][v] rows, 16-byte chunks
// XOR-swizzled by the token, then stores it with 16-byte stores that cover whole token rows
// (full cache lines) per instruction.
constexpr int UCH = HC::WTM / 8;          // 16-byte chunks per staged token row
constexpr int UWAVE = HC::WTM * HC::WTN;  // staged elements per wave
static_assert(UCH <= 64 && 64 % UCH == 0 && (UCH & (UCH - 1)) == 0, "staged row width");
__device__ __forceinline__ int ustage_at(int tl, int vl) {
  return tl * HC::WTM + (((vl >> 3) ^ (tl & (UCH - 1))) << 3) + (vl & 7);
}

// Stores the staged block: token rows tok0 + (0..WTN-1), vocabulary entries v0 + (0..WTM-1) of
// out (row pitch Vp, Npad rows). AUX is the store's cache policy.
template <int AUX>
__device__ __forceinline__ void store_staged_tokmajor(const bf16* ub, bf16* out, int Npad, int Vp, int tok0, int v0,
                                                      int lane) {
  const size_t ubase = (size_t)tok0 * Vp + v0;
  const size_t rest = ((size_t)Npad * Vp - ubase) * 2;  // bytes of out from the base
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(
      out + ubase, (short)0, (int)std::min<size_t>(rest, 0x7fffffff), BUF_RSRC_WORD3);
  constexpr int RPS = 64 / UCH;  // token rows per store instruction
  const int ch = lane % UCH;
  const int voff = ((lane / UCH) * Vp + ch * 8) * 2;
  // The row offset goes into the per-lane offset and the scalar offset stays the constant
  // 0. A 16-byte store needs one wait state before a VALU instruction may overwrite its
  // data registers; the compiler inserts it only when the scalar offset is not an SGPR.
  // With the row offset in an SGPR (an earlier form of this loop) the next instruction
  // reused the data registers of the store just issued, and on gfx950 the store wrote the
  // new values (measured: about 0.1 % of the U entries replaced by address arithmetic).
#pragma unroll
  for (int j = 0; j < HC::WTN / RPS; ++j) {
    const int tl = RPS * j + lane / UCH;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ub + ustage_at(tl, ch * 8));
    __builtin_amdgcn_raw_buffer_store_b128(v, urs, voff + RPS * j * Vp * 2, 0, AUX);
  }
}

// z^T = E h^T with the forward epilogue (row sums, target logit, optional U residual).
// L2N > 0 fixes n = 2^L2N at compile time (0: taken from the parameters).
// acc[mb][nb][4g + e] for the row offset dt = mb*32 + 8g + e (bit 2 of dt, the lane half,
// already matched).
__device__ __forceinline__ float select_row(const floatx16 (&acc)[HC::MB][HC::NB], int nb, int dt) {
  float z = 0.0f;
#pragma unroll
  for (int mb = 0; mb < HC::MB; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) z = dt == mb * 32 + 8 * (i >> 2) + (i & 3) ? acc[mb][nb][i] : z;
  return z;
}

template <int L2N>
__global__ __launch_bounds__(NT, 1) void head_fwd_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, KMAJOR, HC> s0, s1;
  __shared__ float red[HC::WM][HT_N];
  const int nbm = (p.V + HT_M - 1) / HT_M, nbn = p.Npad / HT_N;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * HT_M;  // vocab
  const int n0 = tn * HT_N;  // tokens
  GemmOperand A{p.E, p.d, p.V, p.d, (long)p.V * p.d}, B{p.h, p.d, p.N, p.d, (long)p.N * p.d};
  floatx16 acc[HC::MB][HC::NB];
  gemm_mainloop<KMAJOR, KMAJOR, HC>(s0, s1, A, B, m0, n0, 0, p.d, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<HC>(wm, wn);
  const float inv_c = p.inv_c, clamp = p.clamp;
  const int vrow0 = m0 + wm * HC::WTM;  // first vocab row of this wave
  // Interior tile (every row and column live); WITH_U also stores the residual. U is
  // token-major (element (tok, v) at tok * Vp + v), staged per wave and written with 16-byte
  // stores marked non-temporal so the 1 GB stream of U does not evict the E / h panels the
  // GEMM is reusing from L2.
  constexpr int NWAVES = HC::THREADS / 64;
  static_assert(NWAVES * UWAVE * 2 <= 2 * (int)sizeof(s0), "staging fits the pipeline buffers");
  static_assert((NWAVES / 2) * UWAVE * 2 <= (int)sizeof(s0) || NWAVES == 1, "half the waves per stage");
  auto interior = [&](auto with_u) {
    constexpr bool WITH_U = decltype(with_u)::value;
    bf16* ub = nullptr;
    if constexpr (WITH_U) {
      __syncthreads();  // every wave is done reading the pipeline buffers
      const int wi = wm * HC::WN + wn;
      ub = reinterpret_cast<bf16*>(wi < NWAVES / 2 ? static_cast<void*>(&s0) : static_cast<void*>(&s1)) +
           (wi % (NWAVES / 2)) * UWAVE;
    }
#pragma unroll
    for (int nb = 0; nb < HC::NB; ++nb) {
      const int col = wn * HC::WTN + nb * 32 + l32;
      const int tok = n0 + col;
      const int dt = p.targets[tok] - vrow0 - 4 * h;  // target row relative to this lane's rows
      float part = 0.0f;
#pragma unroll
      for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float u[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float z = acc[mb][nb][4 * g + e];
            const float x = fminf(z * inv_c, clamp);  // fused_head.py:98
            float r;
            const float w = pow2n<L2N>(rho_fast(x, r), p.log2n);
            part += w;
            u[e] = w * r;
          }
          if constexpr (WITH_U) {
            u32x2 pk;
            pk[0] = pack_bf16x2(u[0], u[1]);
            pk[1] = pack_bf16x2(u[2], u[3]);
            *reinterpret_cast<u32x2*>(ub + ustage_at(nb * 32 + l32, mb * 32 + 8 * g + 4 * h)) = pk;
          }
        }
      }
      // The lane holds rows mb*32 + 8g + e (+4h) of the block: the target's row is one of them
      // when its offset dt has bit 2 clear and lies in [0, WTM). That is rare (WTM of V rows
      // per token), so the select runs behind a wave-uniform branch, skipped by every wave
      // where no lane hits.
      const bool mine = (unsigned)dt < (unsigned)HC::WTM && !(dt & 4);
      if (__builtin_amdgcn_ballot_w64(mine)) {
        int dsel = dt;
        asm volatile("" : "+v"(dsel));  // keeps the select inside the branch (not speculated)
        const float z = select_row(acc, nb, dsel);
        if (mine) p.zt[tok] = z;
      }
      part += xor32(part);
      if (h == 0) red[wm][col] = part;
    }
    // Rows of this wave's block: tokens n0 + wn*64 + (0..63), vocabulary vrow0 + (0..127).
    if constexpr (WITH_U) store_staged_tokmajor<BUF_NT>(ub, p.ut, p.Npad, p.Vp, n0 + wn * HC::WTN, vrow0, lane);
  };
  if (m0 + HT_M <= p.V && n0 + HT_N <= p.N) {
    if (p.ut) interior(std::true_type{});
    else interior(std::false_type{});
  } else {
#pragma unroll
    for (int nb = 0; nb < HC::NB; ++nb) {
      const int col = wn * HC::WTN + nb * 32 + l32;
      const int tok = n0 + col;
      const bool live = tok < p.N;
      const int tgt = live ? p.targets[tok] : -1;
      float part = 0.0f;
#pragma unroll
      for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int v = vrow0 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          const float z = acc[mb][nb][i];
          const float x = fminf(z * inv_c, clamp);
          float r;
          const float w = pow2n<L2N>(rho_fast(x, r), p.log2n);
          if (v < p.V) {
            part += w;
            if (p.ut && live) p.ut[(size_t)tok * p.Vp + v] = f2bf(w * r);
          }
          if (v == tgt) p.zt[tok] = z;
        }
      }
      part += xor32(part);
      if (h == 0) red[wm][col] = part;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < HT_N; t += NT) {
    const int tok = n0 + t;
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < HC::WM; ++w) s += red[w][t];
    if (tok < p.N) p.partial[(size_t)tm * p.N + tok] = s;
  }
}

// Evaluation head (src/algebraic/evaluation.py:13-23 with the argmax of
// src/algebraic/benchmarking.py:178-188): z^T = E h^T as in the forward. The scorer's
// log_softmax(n asinh(z/c)) has no clamp, so the weights are evaluated relative to the largest
// logit z_m of a group of logits: w' = (rho(z/c) rho(-z_m/c))^n = exp(n (asinh(z/c) - asinh(z_m/c)))
// <= 1, which neither overflows however large the logits grow nor loses the group's leading
// terms. The epilogue keeps, per token and vocabulary tile, the tile's largest logit with its
// first index (the argmax), the sum of w' relative to that logit, and the target logit.
// Nothing per (token, vocab) pair is stored; head_eval_stats_kernel combines the tiles.

template <int L2N>
__global__ __launch_bounds__(NT, 1) void head_eval_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, KMAJOR, HC> s0, s1;
  __shared__ float red[HC::WM][HT_N];
  __shared__ float redm[HC::WM][HT_N];
  __shared__ int redi[HC::WM][HT_N];
  const int nbm = (p.V + HT_M - 1) / HT_M, nbn = p.Npad / HT_N;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * HT_M;  // vocab
  const int n0 = tn * HT_N;  // tokens
  GemmOperand A{p.E, p.d, p.V, p.d, (long)p.V * p.d}, B{p.h, p.d, p.N, p.d, (long)p.N * p.d};
  floatx16 acc[HC::MB][HC::NB];
  gemm_mainloop<KMAJOR, KMAJOR, HC>(s0, s1, A, B, m0, n0, 0, p.d, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<HC>(wm, wn);
  const float inv_c = p.inv_c;
  const int vrow0 = m0 + wm * HC::WTM;
#pragma unroll
  for (int nb = 0; nb < HC::NB; ++nb) {
    const int col = wn * HC::WTN + nb * 32 + l32;
    const int tok = n0 + col;
    const int tgt = tok < p.N ? p.targets[tok] : -1;
    // Pass 1: this lane's largest logit and its first index (the lane's vocabulary rows
    // increase with (mb, i)), and the target logit.
    float zm = -INFINITY;
    int im = EVAL_NO_INDEX;
#pragma unroll
    for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vrow0 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        const float z = acc[mb][nb][i];
        if (v < p.V) {
          // Rows increase along the lane: take z if it is larger, or the first NaN.
          if (!(z <= zm) && zm == zm) { zm = z; im = v; }
          if (v == tgt) p.zt[tok] = z;
        }
      }
    }
    // Pass 2: the sum of weights relative to that logit.
    const float sh = eval_rho(-zm * inv_c);
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vrow0 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (v < p.V) part += pow2n<L2N>(eval_rho(acc[mb][nb][i] * inv_c) * sh, p.log2n);
      }
    }
    // The other lane half holds the same token's remaining rows of this wave's block.
    const float pz = __shfl_xor(zm, 32, 64);
    const float pp = __shfl_xor(part, 32, 64);
    const int pi = __shfl_xor(im, 32, 64);
    const bool take = pi != EVAL_NO_INDEX && eval_better(pz, pi, zm, im);
    const float zn = take ? pz : zm;
    const float mine = part == 0.0f ? 0.0f : part * eval_rescale<L2N>(zm, zn, inv_c, p.log2n);
    const float other = pp == 0.0f ? 0.0f : pp * eval_rescale<L2N>(pz, zn, inv_c, p.log2n);
    if (take) { zm = pz; im = pi; }
    if (h == 0) { red[wm][col] = mine + other; redm[wm][col] = zm; redi[wm][col] = im; }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < HT_N; t += NT) {
    const int tok = n0 + t;
    float m = -INFINITY;
    int ix = EVAL_NO_INDEX;
#pragma unroll
    for (int w = 0; w < HC::WM; ++w)  // waves cover increasing vocabulary rows
      if (redi[w][t] != EVAL_NO_INDEX && eval_better(redm[w][t], redi[w][t], m, ix)) { m = redm[w][t]; ix = redi[w][t]; }
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < HC::WM; ++w)
      if (red[w][t] != 0.0f) s += red[w][t] * eval_rescale<L2N>(redm[w][t], m, inv_c, p.log2n);
    if (tok < p.N) {
      p.partial[(size_t)tm * p.N + tok] = s;
      p.pmax[(size_t)tm * p.N + tok] = m;
      p.pidx[(size_t)tm * p.N + tok] = ix;
    }
  }
}

// The per-token reductions over vocabulary tiles below read one value per tile (stride N) and
// combine them in tile order within each wave's range of tiles; the loads are issued TB at a
// time so their latencies overlap, while the order of the combining steps stays that of a
// plain loop.
constexpr int TB = 16;

// log p(target) = log_softmax(n asinh(z/c))[t] (src/algebraic/evaluation.py:13-23) from the
// tiles' (largest logit, shifted sum) pairs: with z_m the largest logit of the row and
// L = sum over tiles of S_tile (rho(z_tile/c) rho(-z_m/c))^n = sum_v (rho(z_v/c) rho(-z_m/c))^n,
//   log p = n (log rho(z_t/c) + log rho(-z_m/c)) - log L,
// all in the log domain so that neither large logits nor improbable targets overflow or
// underflow. argmax: the first index of the largest logit over the tiles in vocabulary order
// (the first NaN if there is one, as jnp.argmax).
// 64 tokens per workgroup (lane = token, so each tile row is read as 256 contiguous bytes);
// the EVQ waves take consecutive ranges of the tiles, and their argmax candidates and partial
// sums are combined in range order through LDS. One token per thread over all the tiles left
// three quarters of the SIMDs idle at N = 16384: 48 us against 20.5 us with eight ranges in a
// kernel trace (HIP events: 27 us with four ranges, 24 us with eight).
constexpr int EVQ = 8;  // tile ranges (waves) per token
__global__ __launch_bounds__(64 * EVQ) void head_eval_stats_kernel(HeadParams p, int nvt) {
  __shared__ float sm[EVQ][64];
  __shared__ int si[EVQ][64];
  __shared__ float sl[EVQ][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int tok = blockIdx.x * 64 + lane;
  const bool live = tok < p.N;
  const int per = (nvt + EVQ - 1) / EVQ;
  const int t0 = min(nvt, q * per), t1 = min(nvt, t0 + per);
  float m = -INFINITY;
  int ix = EVAL_NO_INDEX;
  auto take = [&](float pm, int pi) {
    if (pi != EVAL_NO_INDEX && eval_better(pm, pi, m, ix)) { m = pm; ix = pi; }
  };
  if (live) {
    int t = t0;
    for (; t + TB <= t1; t += TB) {
      float vm[TB];
      int vi[TB];
#pragma unroll
      for (int u = 0; u < TB; ++u) {
        const size_t o = (size_t)(t + u) * p.N + tok;
        vm[u] = p.pmax[o];
        vi[u] = p.pidx[o];
      }
#pragma unroll
      for (int u = 0; u < TB; ++u) take(vm[u], vi[u]);
    }
    for (; t < t1; ++t) take(p.pmax[(size_t)t * p.N + tok], p.pidx[(size_t)t * p.N + tok]);
  }
  sm[q][lane] = m;
  si[q][lane] = ix;
  __syncthreads();
  m = -INFINITY;
  ix = EVAL_NO_INDEX;
#pragma unroll
  for (int r = 0; r < EVQ; ++r) take(sm[r][lane], si[r][lane]);
  // Sum of this range's tile sums, each moved onto m, in tile order.
  float l = 0.0f;
  auto add = [&](float s, float pm) {
    if (s != 0.0f) l += s * eval_rescale<0>(pm, m, p.inv_c, p.log2n);
  };
  if (live) {
    int t = t0;
    for (; t + TB <= t1; t += TB) {
      float vs[TB], vm[TB];
#pragma unroll
      for (int u = 0; u < TB; ++u) {
        const size_t o = (size_t)(t + u) * p.N + tok;
        vs[u] = p.partial[o];
        vm[u] = p.pmax[o];
      }
#pragma unroll
      for (int u = 0; u < TB; ++u) add(vs[u], vm[u]);
    }
    for (; t < t1; ++t) add(p.partial[(size_t)t * p.N + tok], p.pmax[(size_t)t * p.N + tok]);
  }
  sl[q][lane] = l;
  __syncthreads();
  if (q != 0 || !live) return;
  l = sl[0][lane];
#pragma unroll
  for (int r = 1; r < EVQ; ++r) l += sl[r][lane];
  // The target logit is written by the tile holding the target; out-of-range targets read 0.
  const int tgt = p.targets[tok];
  const float zt = tgt >= 0 && tgt < p.V ? p.zt[tok] : 0.0f;
  const float rel = zt == m ? 0.0f : logf(rho_exact(zt * p.inv_c)) + logf(rho_exact(-m * p.inv_c));
  p.logprob[tok] = (float)(1 << p.log2n) * rel - logf(l);
  if (p.argmax) p.argmax[tok] = ix == EVAL_NO_INDEX ? 0 : ix;  // every logit -inf: index 0
}

// Per-token statistics and telemetry (fused_head.py:116-117, 219-229); with the residual
// schedule also l and the target entries of U.
// 64 tokens per workgroup, the vocabulary tiles split over EVQ waves as in the eval statistics:
// each wave sums its range in tile order, the ranges are added in range order.
__global__ __launch_bounds__(64 * EVQ) void head_stats_kernel(HeadParams p, int nvt) {
  __shared__ float sl[EVQ][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int tok = blockIdx.x * 64 + lane;
  const int per = (nvt + EVQ - 1) / EVQ;
  const int t0 = min(nvt, q * per), t1 = min(nvt, t0 + per);
  float part = 0.0f;
  if (tok < p.N) {
    int t = t0;
    for (; t + TB <= t1; t += TB) {
      float v[TB];
#pragma unroll
      for (int u = 0; u < TB; ++u) v[u] = p.partial[(size_t)(t + u) * p.N + tok];
#pragma unroll
      for (int u = 0; u < TB; ++u) part += v[u];
    }
    for (; t < t1; ++t) part += p.partial[(size_t)t * p.N + tok];
  }
  sl[q][lane] = part;
  __syncthreads();
  if (q != 0) return;
  float miss = 0.0f;
  if (tok < p.N) {
    float l = sl[0][lane];
#pragma unroll
    for (int r = 1; r < EVQ; ++r) l += sl[r][lane];
    const int n = 1 << p.log2n;
    const float st = inv_root(l, n);
    p.stat[tok] = st;
    // The forward wrote zt only where the target lies in [0, V); elsewhere it is 0
    // (fused_head.py:87 sums no column).
    const int tgt = p.targets[tok];
    const bool valid = tgt >= 0 && tgt < p.V;
    const float zt = valid ? p.zt[tok] : 0.0f;
    if (!valid) p.zt[tok] = 0.0f;
    const float x = fminf(zt / p.c, p.clamp);
    const float pt = ipow_rt(rho_exact(x) * st, n);
    p.pt[tok] = pt;
    miss = 1.0f - pt;
    if (p.lsum) p.lsum[tok] = l;
    if (p.ut) {
      if (valid) {
        float r;
        const float w = head_w(zt, p, r);
        p.ut[(size_t)tok * p.Vp + tgt] = f2bf((w - l) * r);
      }
    }
  }
  // This workgroup's sum of 1 - pt, by a fixed butterfly over the wave.
  for (int m = 32; m >= 1; m >>= 1) miss += __shfl_xor(miss, m, 64);
  if (lane == 0) p.obj_part[blockIdx.x] = miss;
}

__global__ __launch_bounds__(256) void head_obj_kernel(HeadParams p, int nblocks) {
  __shared__ float red[256];
  float s = 0.0f;
  for (int i = threadIdx.x; i < nblocks; i += 256) s += p.obj_part[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int k = 128; k > 0; k >>= 1) {
    if (threadIdx.x < k) red[threadIdx.x] += red[threadIdx.x + k];
    __syncthreads();
  }
  if (threadIdx.x == 0) p.obj[0] = red[0] / (float)p.N;
}

// This wave's share of the pipeline buffers (idle after the main loop; the caller has passed
// a barrier after which no wave reads them): half the waves stage in s0, half in s1.
template <class Stage>
__device__ __forceinline__ bf16* wave_stage(Stage& s0, Stage& s1, int wm, int wn) {
  constexpr int NWAVES = HC::THREADS / 64, UWAVE = HC::WTM * HC::WTN;
  static_assert((NWAVES / 2) * UWAVE * 2 <= (int)sizeof(Stage), "half the waves per stage");
  const int wi = wm * HC::WN + wn;
  return reinterpret_cast<bf16*>(wi < NWAVES / 2 ? static_cast<void*>(&s0) : static_cast<void*>(&s1)) +
         (wi % (NWAVES / 2)) * UWAVE;
}

// Recompute schedules: z^T again, dZ^T = bf16(s (p - y) r), token-major. L2N > 0 fixes
// n = 2^L2N at compile time (0: taken from the parameters). Interior tiles stage each wave's
// block and write whole token rows with 16-byte stores (default cache policy: the dh and dE
// products read dZ right after); edge tiles store element by element.
template <int L2N>
__global__ __launch_bounds__(NT, 1) void head_dz_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, KMAJOR, HC> s0, s1;
  const int nbm = (p.V + HT_M - 1) / HT_M, nbn = p.Npad / HT_N;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * HT_M, n0 = tn * HT_N;
  GemmOperand A{p.E, p.d, p.V, p.d, (long)p.V * p.d}, B{p.h, p.d, p.N, p.d, (long)p.N * p.d};
  floatx16 acc[HC::MB][HC::NB];
  gemm_mainloop<KMAJOR, KMAJOR, HC>(s0, s1, A, B, m0, n0, 0, p.d, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<HC>(wm, wn);
  const float scale = head_grad_scale(p);
  const float inv_c = p.inv_c, clamp = p.clamp;
  const int vrow0 = m0 + wm * HC::WTM;  // first vocab row of this wave
  if (m0 + HT_M <= p.V && n0 + HT_N <= p.N) {
    __syncthreads();  // every wave is done reading the pipeline buffers
    bf16* ub = wave_stage(s0, s1, wm, wn);
#pragma unroll
    for (int nb = 0; nb < HC::NB; ++nb) {
      const int tok = n0 + wn * HC::WTN + nb * 32 + l32;
      const int dt = p.targets[tok] - p.v_off - vrow0 - 4 * h;  // target row relative to this lane's rows
      const float st = p.stat[tok];
#pragma unroll
      for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float u[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = fminf(acc[mb][nb][4 * g + e] * inv_c, clamp);
            float r;
            const float t = pow2n<L2N>(rho_fast(x, r) * st, p.log2n);
            u[e] = t * r * scale;  // (t - y) r s with y = 0; the target entry is patched below
          }
          u32x2 pk;
          pk[0] = pack_bf16x2(u[0], u[1]);
          pk[1] = pack_bf16x2(u[2], u[3]);
          *reinterpret_cast<u32x2*>(ub + ustage_at(nb * 32 + l32, mb * 32 + 8 * g + 4 * h)) = pk;
        }
      }
      // The target entry, (t - 1) r s (y = 1): rare (WTM of V rows per token), so it is formed
      // again behind a wave-uniform branch, as the forward selects the target logit, and
      // overwrites its staged slot (the same lane wrote it above; LDS keeps a wave's order).
      const bool mine = (unsigned)dt < (unsigned)HC::WTM && !(dt & 4);
      if (__builtin_amdgcn_ballot_w64(mine)) {
        int dsel = dt;
        asm volatile("" : "+v"(dsel));  // keeps the select inside the branch (not speculated)
        const float x = fminf(select_row(acc, nb, dsel) * inv_c, clamp);
        float r;
        const float t = pow2n<L2N>(rho_fast(x, r) * st, p.log2n);
        if (mine) ub[ustage_at(nb * 32 + l32, dsel + 4 * h)] = f2bf((t - 1.0f) * r * scale);
      }
    }
    store_staged_tokmajor<0>(ub, p.dzt, p.Npad, p.Vp, n0 + wn * HC::WTN, vrow0, lane);
    return;
  }
#pragma unroll
  for (int nb = 0; nb < HC::NB; ++nb) {
    const int tok = n0 + wn * HC::WTN + nb * 32 + l32;
    const bool live = tok < p.N;
    const int tgt = live ? p.targets[tok] : -1;
    const float st = live ? p.stat[tok] : 0.0f;
#pragma unroll
    for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vrow0 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (v >= p.V) continue;
        const float x = fminf(acc[mb][nb][i] * inv_c, clamp);
        float r;
        const float t = pow2n<L2N>(rho_fast(x, r) * st, p.log2n);
        const float y = (v + p.v_off == tgt) ? 1.0f : 0.0f;
        if (live) p.dzt[(size_t)tok * p.Vp + v] = f2bf((t - y) * r * scale);  // token-major
      }
    }
  }
}

// Residual schedule: hs = bf16(s h / l) (the row scale of dE = U'^T (s h / l)).
__global__ __launch_bounds__(256) void head_hscale_kernel(HeadParams p) {
  const float s = head_grad_scale(p);
  const size_t total8 = (size_t)p.N * p.d / 8;
  for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < total8; c += (size_t)gridDim.x * 256) {
    const int row = (int)((c * 8) / p.d);
    const float f = s / p.lsum[row];
    bf16x8 x = *reinterpret_cast<const bf16x8*>(p.h + c * 8);
    bf16x8 y;
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = f2bf((float)x[j] * f);
    *reinterpret_cast<bf16x8*>(p.hs + c * 8) = y;
  }
}

// Store of a wave's WTM x WTN accumulator block, scaled per row and rounded to bf16, into a
// row-major matrix (interior tiles). Stored straight from the accumulators, each store
// instruction would cover 64 bytes of two rows at 2 bytes a lane; instead the block is staged
// in `stage` (this wave's share of the idle pipeline buffers) as [row][col] rows of WTN
// elements, 16-byte chunks XOR-swizzled by the row, and written back with 16-byte stores
// that cover whole 128-byte row segments. f(r) is the scale of block row r.
template <class RowScale>
__device__ __forceinline__ void store_block_bf16(const floatx16 (&acc)[HC::MB][HC::NB], bf16* stage, bf16* out,
                                                 long ld, RowScale f) {
  constexpr int CH = HC::WTN / 8;  // 16-byte chunks per staged row
  static_assert(CH <= 64 && 64 % CH == 0 && (CH & (CH - 1)) == 0, "staged row width");
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  auto at = [](int r, int c) { return r * HC::WTN + (((c >> 3) ^ (r & (CH - 1))) << 3) + (c & 7); };
#pragma unroll
  for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      const float fr = f(r);
#pragma unroll
      for (int nb = 0; nb < HC::NB; ++nb) stage[at(r, nb * 32 + l32)] = f2bf(acc[mb][nb][i] * fr);
    }
  }
  constexpr int RPS = 64 / CH;  // rows per store instruction
  const int c = lane % CH;
#pragma unroll
  for (int j = 0; j < HC::WTM / RPS; ++j) {
    const int r = RPS * j + lane / CH;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + at(r, c * 8));
    *reinterpret_cast<u32x4*>(out + (long)r * ld + c * 8) = v;
  }
}


// dh = (U' or dZ) E: A stored token-major [n][v] (k-contiguous), B = E stored [v][d]
// (n-contiguous). The residual schedule scales token rows by s/l. When the product has too
// few output tiles to fill the chip (small N*d, long V) the vocabulary is split into
// dh_split ranges: each workgroup writes its f32 partial and head_dh_reduce_kernel sums them
// in a fixed order before the scale and the rounding. ACC (the streamed schedule's later
// vocabulary chunks, p.dh_accum 1 or 2): the tile of the f32 accumulator p.dh_part is read
// whole after the main loop (all loads issued before the first add) and added to the product,
// which then goes back to the accumulator (dh_accum 1) or, rounded, to dh (dh_accum 2).
template <bool ACC>
__global__ __launch_bounds__(NT, 1) void head_dh_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, MNMAJOR, HC> s0, s1;
  const int nbm = p.Npad / HT_M, nbn = (p.d + HT_N - 1) / HT_N;
  int tr, tn;
  xcd_tile_rowmajor(blockIdx.x, nbm * p.dh_split, nbn, tr, tn);  // U panels streamed once
  // Split-major: the workgroups an XCD runs together share one vocabulary range, so its E
  // rows are read by every token tile there from L2 (C2: dh 0.658 -> 0.639 ms).
  const int split = tr / nbm, tm = tr - split * nbm;
  const int m0 = tm * HT_M;  // tokens
  const int n0 = tn * HT_N;  // d
  const int kbeg = min(p.V, split * p.dh_kchunk), kend = min(p.V, kbeg + p.dh_kchunk);
  const bf16* a = p.ut ? p.ut : p.dzt;
  GemmOperand A{a, p.Vp, p.N, p.V, (long)p.Npad * p.Vp}, B{p.E, p.d, p.V, p.d, (long)p.V * p.d};
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<HC>(wm, wn);
  float* part = p.dh_part ? p.dh_part + (size_t)split * p.N * p.d : nullptr;
  floatx16 acc[HC::MB][HC::NB];
  gemm_mainloop<KMAJOR, MNMAJOR, HC>(s0, s1, A, B, m0, n0, kbeg, kend, acc);
  if constexpr (ACC) {
    // One 32 x 32 block at a time: its 16 loads are issued together, then added, and (dh_accum
    // 1) stored back to the accumulator.
    const bool back = p.dh_accum == 1;
#pragma unroll
    for (int mb = 0; mb < HC::MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < HC::NB; ++nb) {
        const int r0 = m0 + wm * HC::WTM + mb * 32 + 4 * h, col = n0 + wn * HC::WTN + nb * 32 + l32;
        float* blk = part + (size_t)r0 * p.d + col;
        float pv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int dr = 8 * (i >> 2) + (i & 3);
          pv[i] = r0 + dr < p.N && col < p.d ? blk[dr * p.d] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int dr = 8 * (i >> 2) + (i & 3);
          acc[mb][nb][i] += pv[i];
          if (back && r0 + dr < p.N && col < p.d) blk[dr * p.d] = acc[mb][nb][i];
        }
      }
    if (back) return;
  }
  const float s = p.ut ? head_grad_scale(p) : 1.0f;
  const bool to_dh = !part || ACC;  // bf16 output (ACC here: the last chunk)
  if (to_dh && m0 + HT_M <= p.N && n0 + HT_N <= p.d) {
    // Interior tile, bf16 output: the row scales s/l once per row (the expression of
    // head_hscale_kernel), then the staged 16-byte stores.
    __shared__ float fsc[HT_M];
    for (int t = threadIdx.x; t < HT_M; t += NT) fsc[t] = p.ut ? s / p.lsum[m0 + t] : 1.0f;
    __syncthreads();  // fsc is written and every wave is done with the pipeline buffers
    const int r0 = wm * HC::WTM;
    store_block_bf16(acc, wave_stage(s0, s1, wm, wn), p.dh + (size_t)(m0 + r0) * p.d + n0 + wn * HC::WTN, p.d,
                     [&](int r) { return fsc[r0 + r]; });
    return;
  }
#pragma unroll
  for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = m0 + wm * HC::WTM + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (tok >= p.N) continue;
      const float f = p.ut ? s / p.lsum[tok] : 1.0f;
#pragma unroll
      for (int nb = 0; nb < HC::NB; ++nb) {
        const int col = n0 + wn * HC::WTN + nb * 32 + l32;
        if (col >= p.d) continue;
        const size_t o = (size_t)tok * p.d + col;
        if (to_dh) p.dh[o] = f2bf(acc[mb][nb][i] * f);
        else part[o] = acc[mb][nb][i];
      }
    }
  }
}

// dh = bf16(f * sum_s partial_s) over the vocabulary splits, summed in split order.
__global__ __launch_bounds__(256) void head_dh_reduce_kernel(HeadParams p) {
  const float s = p.ut ? head_grad_scale(p) : 1.0f;
  const size_t plane = (size_t)p.N * p.d;
  const size_t total8 = plane / 8;
  for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < total8; c += (size_t)gridDim.x * 256) {
    const int row = (int)((c * 8) / p.d);
    const float4* src = reinterpret_cast<const float4*>(p.dh_part + c * 8);
    float4 a = src[0], b = src[1];
    for (int k = 1; k < p.dh_split; ++k) {
      const float4* q = reinterpret_cast<const float4*>(p.dh_part + k * plane + c * 8);
      const float4 x = q[0], y = q[1];
      a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
      b.x += y.x; b.y += y.y; b.z += y.z; b.w += y.w;
    }
    const float f = p.ut ? s / p.lsum[row] : 1.0f;
    bf16x8 out;
    out[0] = f2bf(a.x * f); out[1] = f2bf(a.y * f); out[2] = f2bf(a.z * f); out[3] = f2bf(a.w * f);
    out[4] = f2bf(b.x * f); out[5] = f2bf(b.y * f); out[6] = f2bf(b.z * f); out[7] = f2bf(b.w * f);
    *reinterpret_cast<bf16x8*>(p.dh + c * 8) = out;
  }
}

// dE = (U' or dZ)^T (hs or h): A = U' stored token-major [n][v] (m-contiguous), B stored
// [n][d] (n-contiguous). Workgroups below de_full compute whole tiles, row-major inside each
// XCD's share (U panels streamed once); the rest compute token range (id - de_full) % de_split
// of tile de_full + (id - de_full) / de_split into an f32 tile of de_part, which
// head_de_tail_kernel sums.
__global__ __launch_bounds__(NT, 1) void head_de_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<MNMAJOR, MNMAJOR, HC> s0, s1;
  const int nbn = (p.d + HT_N - 1) / HT_N;
  const int bid = blockIdx.x;
  int lin, kbeg = 0, kend = p.N, unit = -1;
  if (bid < p.de_full) {
    lin = p.de_full % 8 == 0 ? (bid % 8) * (p.de_full / 8) + bid / 8 : bid;
  } else {
    unit = bid - p.de_full;
    lin = p.de_full + unit / p.de_split;
    kbeg = (unit % p.de_split) * p.de_kchunk;
    kend = min(p.N, kbeg + p.de_kchunk);
  }
  const int tm = lin / nbn, tn = lin - tm * nbn;
  const int m0 = tm * HT_M;  // vocab
  const int n0 = tn * HT_N;  // d
  const bf16* a = p.ut ? p.ut : p.dzt;
  const bf16* b = p.ut ? p.hs : p.h;
  GemmOperand A{a, p.Vp, p.N, p.V, (long)p.Npad * p.Vp}, B{b, p.d, p.N, p.d, (long)p.N * p.d};
  floatx16 acc[HC::MB][HC::NB];
  gemm_mainloop<MNMAJOR, MNMAJOR, HC>(s0, s1, A, B, m0, n0, kbeg, kend, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<HC>(wm, wn);
  if (unit >= 0) {  // one token range of a split tile: the whole f32 tile, row-major
    float* part = p.de_part + (size_t)unit * HT_M * HT_N;
#pragma unroll
    for (int mb = 0; mb < HC::MB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = wm * HC::WTM + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
#pragma unroll
        for (int nb = 0; nb < HC::NB; ++nb) part[r * HT_N + wn * HC::WTN + nb * 32 + l32] = acc[mb][nb][i];
      }
    return;
  }
  if (!p.dE_f32 && m0 + HT_M <= p.V && n0 + HT_N <= p.d) {  // interior tile, bf16 output
    __syncthreads();  // every wave is done with the pipeline buffers
    store_block_bf16(acc, wave_stage(s0, s1, wm, wn),
                     reinterpret_cast<bf16*>(p.dE) + (size_t)(m0 + wm * HC::WTM) * p.d + n0 + wn * HC::WTN, p.d,
                     [](int) { return 1.0f; });
    return;
  }
#pragma unroll
  for (int mb = 0; mb < HC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int v = m0 + wm * HC::WTM + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (v >= p.V) continue;
#pragma unroll
      for (int nb = 0; nb < HC::NB; ++nb) {
        const int col = n0 + wn * HC::WTN + nb * 32 + l32;
        if (col >= p.d) continue;
        const size_t o = (size_t)v * p.d + col;
        if (p.dE_f32) reinterpret_cast<float*>(p.dE)[o] = acc[mb][nb][i];
        else reinterpret_cast<bf16*>(p.dE)[o] = f2bf(acc[mb][nb][i]);
      }
    }
  }
}

// dE of a split tile: the de_split token-range tiles summed in range order, 32 rows of the
// tile per workgroup (grid: split tiles x HT_M / 32).
__global__ __launch_bounds__(256) void head_de_tail_kernel(HeadParams p) {
  const int nbn = (p.d + HT_N - 1) / HT_N;
  const int lin = p.de_full + blockIdx.x;
  const int tm = lin / nbn, tn = lin - tm * nbn;
  const float* part = p.de_part + (size_t)blockIdx.x * p.de_split * HT_M * HT_N;
#pragma unroll
  for (int c = 0; c < 32 * HT_N / 8 / 256; ++c) {
    const int e = (threadIdx.x + 256 * c) * 8;
    const int r = blockIdx.y * 32 + e / HT_N, col = e % HT_N;
    const int v = tm * HT_M + r, j0 = tn * HT_N + col;
    if (v >= p.V || j0 >= p.d) continue;
    const size_t o = (size_t)r * HT_N + col;
    float4 a = *reinterpret_cast<const float4*>(part + o), b = *reinterpret_cast<const float4*>(part + o + 4);
    for (int k = 1; k < p.de_split; ++k) {
      const float* q = part + (size_t)k * HT_M * HT_N + o;
      const float4 x = *reinterpret_cast<const float4*>(q), y = *reinterpret_cast<const float4*>(q + 4);
      a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
      b.x += y.x; b.y += y.y; b.z += y.z; b.w += y.w;
    }
    const float vals[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const size_t out = (size_t)v * p.d + j0;  // d % 8 == 0: the 8 columns are in the row
    if (p.dE_f32) {
      float* dst = reinterpret_cast<float*>(p.dE) + out;
      *reinterpret_cast<float4*>(dst) = a;
      *reinterpret_cast<float4*>(dst + 4) = b;
    } else {
      bf16x8 o8;
#pragma unroll
      for (int t = 0; t < 8; ++t) o8[t] = f2bf(vals[t]);
      *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.dE) + out) = o8;
    }
  }
}

int head_vocab_tiles(int V) { return (V + HT_M - 1) / HT_M; }
int head_token_pad(int N) { return ((N + HT_N - 1) / HT_N) * HT_N; }
int head_vocab_pitch(int V) { return (V + 7) / 8 * 8; }
int head_stat_blocks(int N) { return (N + 63) / 64; }

// Vocabulary splits of the dh product: minimise the rounds of 256 workgroups per unit of
// k work (ceil(tiles*S/256)/S) for products with fewer than two rounds of tiles, keeping at
// least 512 vocabulary entries per split; ties keep the smaller split count.
int head_dh_split(int N, int d, int V) {
  const int tiles = (head_token_pad(N) / HT_M) * ((d + HT_N - 1) / HT_N);
  if (tiles >= 512) return 1;
  int best = 1;
  double best_cost = std::ceil(tiles / 256.0);
  for (int s = 2; s <= 16 && V / s >= 512; ++s) {
    const double cost = std::ceil(tiles * (double)s / 256.0) / s;
    if (cost < best_cost - 1e-9) { best = s; best_cost = cost; }
  }
  return best;
}
int head_dh_kchunk(int V, int split) { return ((V + split - 1) / split + 127) / 128 * 128; }

// dE tiles past the last complete round of 256 workgroups are split over the tokens when that
// shortens the last round: S ranges per tile finish it in ceil(tail*S/256)/S of a tile's time
// instead of one (C2's 591 tiles: two full rounds, then 79 tiles x 3 ranges in a third of a
// tile's time). A range keeps at least 1024 tokens, and a split must save a quarter of a round
// (its f32 tiles are written and summed by head_de_tail_kernel); ties keep the smaller split.
HeadDePlan head_de_plan(int N, int d, int V) {
  HeadDePlan pl;
  pl.tiles = head_vocab_tiles(V) * ((d + HT_N - 1) / HT_N);
  pl.full = pl.tiles;
  pl.split = 1;
  pl.kchunk = 0;
  const int full = pl.tiles / 256 * 256, tail = pl.tiles - full;
  if (tail == 0) return pl;
  int best = 1;
  double best_cost = 1.0;
  for (int s = 2; s <= 8 && N / s >= 1024; ++s) {
    const double cost = std::ceil(tail * (double)s / 256.0) / s;
    if (cost < best_cost - 1e-9) { best = s; best_cost = cost; }
  }
  if (best == 1 || best_cost > 0.75) return pl;
  pl.full = full;
  pl.split = best;
  pl.kchunk = ((N + best - 1) / best + 127) / 128 * 128;
  return pl;
}

hipError_t launch_head_fwd(const HeadParams& p, hipStream_t st) {
  const int tiles = head_vocab_tiles(p.V) * (p.Npad / HT_N);
  {
    KTimer t("head_fwd", st);
    if (p.log2n == 3) hipLaunchKernelGGL(head_fwd_kernel<3>, dim3(tiles), dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(head_fwd_kernel<0>, dim3(tiles), dim3(NT), 0, st, p);
  }
  return launch_head_stats(p, head_vocab_tiles(p.V), st);
}

// Statistics, telemetry and objective from the forward's per-tile partial sums (any tiling:
// vocab_tiles partial rows of N).
hipError_t launch_head_stats(const HeadParams& p, int vocab_tiles, hipStream_t st) {
  const int nb = head_stat_blocks(p.N);
  { KTimer t("head_stats", st); hipLaunchKernelGGL(head_stats_kernel, dim3(nb), dim3(64 * EVQ), 0, st, p, vocab_tiles); }
  { KTimer t("head_obj", st); hipLaunchKernelGGL(head_obj_kernel, dim3(1), dim3(256), 0, st, p, nb); }
  return hipGetLastError();
}

hipError_t launch_head_eval_stats(const HeadParams& p, int vocab_tiles, hipStream_t st) {
  KTimer t("head_eval_stats", st);
  hipLaunchKernelGGL(head_eval_stats_kernel, dim3(head_stat_blocks(p.N)), dim3(64 * EVQ), 0, st, p, vocab_tiles);
  return hipGetLastError();
}

hipError_t launch_head_eval(const HeadParams& p, hipStream_t st) {
  const int tiles = head_vocab_tiles(p.V) * (p.Npad / HT_N);
  {
    KTimer t("head_eval", st);
    if (p.log2n == 3) hipLaunchKernelGGL(head_eval_kernel<3>, dim3(tiles), dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(head_eval_kernel<0>, dim3(tiles), dim3(NT), 0, st, p);
  }
  return launch_head_eval_stats(p, head_vocab_tiles(p.V), st);
}

// dh = (U' or dZ) E, and the sum over vocabulary splits when the product is split.
static void launch_head_dh(const HeadParams& p, hipStream_t st) {
  const int dtiles = (p.d + HT_N - 1) / HT_N;
  {
    KTimer t("head_dh", st);
    const dim3 grid((p.Npad / HT_M) * dtiles * p.dh_split);
    if (p.dh_accum) hipLaunchKernelGGL(head_dh_kernel<true>, grid, dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(head_dh_kernel<false>, grid, dim3(NT), 0, st, p);
  }
  if (p.dh_split > 1) {
    const size_t chunks = (size_t)p.N * p.d / 8;
    const int blocks = (int)std::min<size_t>((chunks + 255) / 256, 4096);
    KTimer t("head_dh_reduce", st);
    hipLaunchKernelGGL(head_dh_reduce_kernel, dim3(blocks), dim3(256), 0, st, p);
  }
}

// dE = (U' or dZ)^T (hs or h), with the token split of head_de_plan when p carries one.
static void launch_head_de(const HeadParams& p, hipStream_t st) {
  const int de_tiles = head_vocab_tiles(p.V) * ((p.d + HT_N - 1) / HT_N);
  if (p.de_split > 1 && p.de_part) {
    const int tail = de_tiles - p.de_full;
    { KTimer t("head_de", st); hipLaunchKernelGGL(head_de_kernel, dim3(p.de_full + tail * p.de_split), dim3(NT), 0, st, p); }
    { KTimer t("head_de_tail", st); hipLaunchKernelGGL(head_de_tail_kernel, dim3(tail, HT_M / 32), dim3(256), 0, st, p); }
  } else {
    HeadParams q = p;
    q.de_full = de_tiles;
    q.de_split = 1;
    { KTimer t("head_de", st); hipLaunchKernelGGL(head_de_kernel, dim3(de_tiles), dim3(NT), 0, st, q); }
  }
}

static void launch_head_dz(const HeadParams& p, hipStream_t st) {
  const int tiles = head_vocab_tiles(p.V) * (p.Npad / HT_N);
  KTimer t("head_dz", st);
  if (p.log2n == 3) hipLaunchKernelGGL(head_dz_kernel<3>, dim3(tiles), dim3(NT), 0, st, p);
  else hipLaunchKernelGGL(head_dz_kernel<0>, dim3(tiles), dim3(NT), 0, st, p);
}

hipError_t launch_head_bwd(const HeadParams& p, hipStream_t st) {
  if (p.ut) {
    const size_t chunks = (size_t)p.N * p.d / 8;
    const int blocks = (int)std::min<size_t>((chunks + 255) / 256, 8192);
    { KTimer t("head_hscale", st); hipLaunchKernelGGL(head_hscale_kernel, dim3(blocks), dim3(256), 0, st, p); }
  } else {
    launch_head_dz(p, st);
  }
  launch_head_dh(p, st);
  launch_head_de(p, st);
  return hipGetLastError();
}

HeadParams head_vocab_chunk(const HeadParams& p, int v0, int vc) {
  HeadParams q = p;
  q.V = vc;
  q.Vp = head_vocab_pitch(vc);
  q.v_off = v0;
  const size_t rows = (size_t)v0 * p.d;
  if (p.E) q.E = p.E + rows;
  if (p.E32) q.E32 = p.E32 + rows;
  q.dE = p.dE_f32 ? static_cast<void*>(static_cast<float*>(p.dE) + rows) : static_cast<void*>(static_cast<bf16*>(p.dE) + rows);
  return q;
}

hipError_t launch_head_bwd_streamed(const HeadParams& p, int chunk, hipStream_t st) {
  const int nchunks = (p.V + chunk - 1) / chunk;
  for (int k = 0; k < nchunks; ++k) {
    HeadParams q = head_vocab_chunk(p, k * chunk, std::min(chunk, p.V - k * chunk));
    q.dh_split = 1;
    q.dh_kchunk = head_dh_kchunk(q.V, 1);
    q.dh_part = nchunks > 1 ? p.dh_part : nullptr;
    q.dh_accum = k == 0 ? 0 : (k == nchunks - 1 ? 2 : 1);
    const HeadDePlan de = head_de_plan(p.N, p.d, q.V);
    q.de_full = de.full;
    q.de_split = de.split;
    q.de_kchunk = de.kchunk;
    launch_head_dz(q, st);
    launch_head_dh(q, st);
    launch_head_de(q, st);
  }
  return hipGetLastError();
}

}  // namespace alg
