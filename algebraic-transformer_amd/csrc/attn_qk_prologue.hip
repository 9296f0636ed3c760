// Fused attention prologue for gfx950: QK RMS normalisation with a learned gain, the Cayley
// rotation, the query pre-scale and the range guard's maxima in one pass over q, k and v,
// and its VJP in one pass back.
//
// Replaces the model's path into the attention kernel, src/algebraic/model.py:170-174
// (qk_norm: algebraic.py:76-83; apply_rotary: algebraic.py:172-179), plus
// flash.py:823-849 (q_s = round(q alpha), guard maxima), and the Cayley tables of
// algebraic.py:124-169.
//
// The raw projections and every (B, ., ., D) output (q_s, k_r; dq, dk and the cotangents in the
// VJP) are stored (B, H, T, D) or (B, T, H, D) (the projection layout before the head
// transpose, model.py:167-169); the per-row 1/rms vectors are (B, H, T). A row of D elements
// is split between D/(2 CH) lanes; lane li holds the
// 16-byte chunk li of both halves, so the rotate-half pairs (x_j, x_{j+D/2}) sit in one lane
// and only the row's sum of squares crosses lanes.
//
// Rounding follows the reference: tau = 1/sqrt(mean(x^2) + eps) in f32; y = round((x tau) g);
// the tables are rounded to the input dtype and every rotated product and sum is rounded
// (XLA's bf16 elementwise semantics); q_s = round(y alpha). Floating-point contraction is
// off in this file: a product of two bf16 values rounded to bf16 and then added is otherwise
// rewritten as a bf16 multiply fused into the add, which drops the product's rounding.
#include "launchers.h"

#pragma clang fp contract(off)

#ifndef PRO_U
#define PRO_U 1
#endif

namespace alg {

namespace {

__device__ __forceinline__ float nanmax_p(float a, float b) { return (a > b || a != a) ? a : b; }

template <typename T>
__device__ __forceinline__ float rnd(float x) { return (float)(T)x; }

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }

// Grid: one workgroup per (b*H + h, block of 4*RPW*PRO_ITER consecutive positions t); wave w
// handles positions t0 + RPW*(w + 4 j) + sub, j < PRO_ITER. Row addresses are a per-head base
// plus t times the row stride of the layout (D for (B, H, T, D), H*D for (B, T, H, D)).
#ifndef PRO_ITER_N
#define PRO_ITER_N 8
#endif
constexpr int PRO_ITER = PRO_ITER_N;

struct RowAddr {
  size_t base;    // element offset of position 0 of this head
  size_t stride;  // elements between consecutive positions
};

__device__ __forceinline__ RowAddr head_rows(int H, int T, int D, int layout) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  RowAddr a;
  if (layout == 0) {
    a.base = (size_t)bh * T * D;
    a.stride = D;
  } else {
    a.base = ((size_t)b * T * H + h) * D;
    a.stride = (size_t)H * D;
  }
  return a;
}

template <typename T>
__device__ __forceinline__ uint4 ld16(const void* base, size_t off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(base) + off);
}

template <typename T, int CH>
__device__ __forceinline__ void cvt_chunk(const uint4& raw, float (&x)[CH]) {
  T v[CH];
  *reinterpret_cast<uint4*>(v) = raw;
#pragma unroll
  for (int e = 0; e < CH; ++e) x[e] = (float)v[e];
}

template <typename T, int CH>
__device__ __forceinline__ void store_chunk(void* base, size_t off, const float (&x)[CH]) {
  T v[CH];
#pragma unroll
  for (int e = 0; e < CH; ++e) v[e] = (T)x[e];
  *reinterpret_cast<uint4*>(reinterpret_cast<T*>(base) + off) = *reinterpret_cast<uint4*>(v);
}

template <int CH>
__device__ __forceinline__ void load_f32(const float* p, float (&x)[CH]) {
#pragma unroll
  for (int e = 0; e < CH; e += 4) *reinterpret_cast<float4*>(&x[e]) = *reinterpret_cast<const float4*>(p + e);
}

// Gain entries c0 .. c0 + CH - 1 of both halves (1 without a gain): one uniform branch around
// the vector loads, so they issue together.
template <int CH>
__device__ __forceinline__ void load_gain_halves(const float* g, int c0, int half, float (&ga)[CH], float (&gb)[CH]) {
  if (g) {
    load_f32<CH>(g + c0, ga);
    load_f32<CH>(g + half + c0, gb);
  } else {
#pragma unroll
    for (int e = 0; e < CH; ++e) ga[e] = gb[e] = 1.0f;
  }
}

template <int LPR>
__device__ __forceinline__ float row_sum(float s) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) s += __shfl_xor(s, m, 64);
  return s;
}

// One tensor's row: y = rot(round((x tau) g)) in the I/O dtype (as f32 values), tau out.
template <typename T, int CH, int LPR>
__device__ __forceinline__ float norm_rotate(float (&a)[CH], float (&b)[CH], const float (&ga)[CH],
                                             const float (&gb)[CH], const float (&ca)[CH],
                                             const float (&sa)[CH], bool rotate, float inv_d, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < CH; ++e) ss += a[e] * a[e] + b[e] * b[e];
  ss = row_sum<LPR>(ss);
  const float tau = 1.0f / sqrtf(ss * inv_d + eps);
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    float ya = mul_rn(a[e], tau), yb = mul_rn(b[e], tau);
    ya = mul_rn(ya, ga[e]);  // gain 1 when there is none: the product is exact
    yb = mul_rn(yb, gb[e]);
    ya = rnd<T>(ya);
    yb = rnd<T>(yb);
    if (rotate) {
      const float c = rnd<T>(ca[e]), s = rnd<T>(sa[e]);
      a[e] = rnd<T>(rnd<T>(mul_rn(ya, c)) - rnd<T>(mul_rn(yb, s)));
      b[e] = rnd<T>(rnd<T>(mul_rn(ya, s)) + rnd<T>(mul_rn(yb, c)));
    } else {
      a[e] = ya;
      b[e] = yb;
    }
  }
  return tau;
}

}  // namespace

__global__ __launch_bounds__(256) void cayley_tables_kernel(const float* w, int half, int T, float* cos_out,
                                                            float* sin_out) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)T * half) return;
  const int m = (int)(idx / half), kk = (int)(idx - (long)m * half);
  const float wk = w[kk];
  const float w2 = mul_rn(wk, wk);
  float c = (1.0f - w2) / (1.0f + w2);
  float s = mul_rn(2.0f, wk) / (1.0f + w2);
  float oc = 1.0f, os = 0.0f;
  for (int bit = 0; (1 << bit) < T; ++bit) {
    if ((m >> bit) & 1) {
      const float nc = __fsub_rn(mul_rn(oc, c), mul_rn(os, s));
      const float ns = __fadd_rn(mul_rn(oc, s), mul_rn(os, c));
      oc = nc;
      os = ns;
    }
    const float c2 = __fsub_rn(mul_rn(c, c), mul_rn(s, s));
    const float s2 = mul_rn(mul_rn(2.0f, c), s);
    const float inv = 1.0f / sqrtf(__fadd_rn(mul_rn(c2, c2), mul_rn(s2, s2)));
    c = mul_rn(c2, inv);
    s = mul_rn(s2, inv);
  }
  const float inv = 1.0f / sqrtf(__fadd_rn(mul_rn(oc, oc), mul_rn(os, os)));
  cos_out[idx] = mul_rn(oc, inv);
  sin_out[idx] = mul_rn(os, inv);
}

// ROT: the Cayley rotation (cos/sin tables given); GUARD: the guard's |v| maxima (v read). Both
// are template parameters so that every load of a row sits in one block and issues together.
template <typename T, int D, bool ROT, bool GUARD>
__global__ __launch_bounds__(256) void attn_qk_prologue_kernel(QkPrologueParams p) {
  constexpr int CH = 16 / sizeof(T), HALF = D / 2, LPR = HALF / CH, RPW = 64 / LPR;
  static_assert(HALF % CH == 0 && 64 % LPR == 0, "row split");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, li = lane - sub * LPR;
  const int c0 = li * CH;
  float gqa[CH], gqb[CH], gka[CH], gkb[CH];
  load_gain_halves<CH>(p.q_gain, c0, HALF, gqa, gqb);
  load_gain_halves<CH>(p.k_gain, c0, HALF, gka, gkb);
  constexpr bool rotate = ROT;
  const float inv_d = 1.0f / (float)D;
  float mq = 0.0f, mk = 0.0f, mv = 0.0f;
  const RowAddr ra = head_rows(p.H, p.T, D, p.layout);
  const int t0 = blockIdx.y * (4 * RPW * PRO_ITER) + wave * RPW + sub;
  // U rows per lane and iteration: every load of the U rows is issued before any compute.
  constexpr int U = PRO_U;
#pragma unroll 1
  for (int j = 0; j < PRO_ITER; j += U) {
    uint4 rq[U][2], rk[U][2], rv[U][2];
    float ca[U][CH], sa[U][CH];
    int tt[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + 4 * RPW * (j + u);
      ok[u] = t < p.T;
      tt[u] = ok[u] ? t : p.T - 1;
      const size_t in = ra.base + (size_t)tt[u] * ra.stride + c0;
      rq[u][0] = ld16<T>(p.q, in);
      rq[u][1] = ld16<T>(p.q, in + HALF);
      rk[u][0] = ld16<T>(p.k, in);
      rk[u][1] = ld16<T>(p.k, in + HALF);
      if constexpr (GUARD) {
        rv[u][0] = ld16<T>(p.v, in);
        rv[u][1] = ld16<T>(p.v, in + HALF);
      }
      if constexpr (ROT) {
        load_f32<CH>(p.cos + (size_t)tt[u] * HALF + c0, ca[u]);
        load_f32<CH>(p.sin + (size_t)tt[u] * HALF + c0, sa[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float qa[CH], qb[CH], ka[CH], kb[CH];
      cvt_chunk<T, CH>(rq[u][0], qa);
      cvt_chunk<T, CH>(rq[u][1], qb);
      cvt_chunk<T, CH>(rk[u][0], ka);
      cvt_chunk<T, CH>(rk[u][1], kb);
      // max |v| with NaN propagation at two VALU ops per element: a NaN-ignoring maximum plus
      // a sum of v*0, which is NaN exactly when some v is NaN or infinite (either fails the
      // guard's |v| bound, as the reference's comparison with a NaN maximum does).
      float av = 0.0f;
      if constexpr (GUARD) {
        float va[CH], vb[CH], nan_acc = 0.0f;
        cvt_chunk<T, CH>(rv[u][0], va);
        cvt_chunk<T, CH>(rv[u][1], vb);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
          av = fmaxf(av, fmaxf(__builtin_fabsf(va[e]), __builtin_fabsf(vb[e])));
          nan_acc = __builtin_fmaf(va[e], 0.0f, __builtin_fmaf(vb[e], 0.0f, nan_acc));
        }
        if (nan_acc != nan_acc) av = nan_acc;
      }
      const float tq = norm_rotate<T, CH, LPR>(qa, qb, gqa, gqb, ca[u], sa[u], rotate, inv_d, p.eps);
      const float tk = norm_rotate<T, CH, LPR>(ka, kb, gka, gkb, ca[u], sa[u], rotate, inv_d, p.eps);
      float sq = 0.0f, sk = 0.0f;
#pragma unroll
      for (int e = 0; e < CH; ++e) {
        qa[e] = rnd<T>(mul_rn(qa[e], p.alpha));
        qb[e] = rnd<T>(mul_rn(qb[e], p.alpha));
        sq += qa[e] * qa[e] + qb[e] * qb[e];
        sk += ka[e] * ka[e] + kb[e] * kb[e];
      }
      sq = row_sum<LPR>(sq);
      sk = row_sum<LPR>(sk);
      if (ok[u]) {
        const size_t out = ra.base + (size_t)tt[u] * ra.stride + c0;
        store_chunk<T, CH>(p.q_s, out, qa);
        store_chunk<T, CH>(p.q_s, out + HALF, qb);
        store_chunk<T, CH>(p.k_r, out, ka);
        store_chunk<T, CH>(p.k_r, out + HALF, kb);
        if (li == 0) {
          const size_t row = (size_t)blockIdx.x * p.T + tt[u];
          p.tau_q[row] = tq;
          p.tau_k[row] = tk;
        }
        mq = nanmax_p(mq, sq);
        mk = nanmax_p(mk, sk);
        mv = nanmax_p(mv, av);
      }
    }
  }
  for (int m = 32; m >= 1; m >>= 1) {
    mq = nanmax_p(mq, __shfl_xor(mq, m, 64));
    mk = nanmax_p(mk, __shfl_xor(mk, m, 64));
    mv = nanmax_p(mv, __shfl_xor(mv, m, 64));
  }
  __shared__ float red[4][3];
  if (lane == 0) { red[wave][0] = mq; red[wave][1] = mk; red[wave][2] = mv; }
  __syncthreads();
  if (threadIdx.x < 3) {
    float m = red[0][threadIdx.x];
    for (int w = 1; w < 4; ++w) m = nanmax_p(m, red[w][threadIdx.x]);
    p.part[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 3 + threadIdx.x] = m;
  }
}

// VJP of one row of one tensor. dy (the rotated output's cotangent) arrives in a/b; on exit
// a/b hold dx. Accumulates the gain-gradient terms dy_n * (x tau) into ga_acc/gb_acc.
template <typename T, int CH, int LPR>
__device__ __forceinline__ void norm_rotate_vjp(float (&a)[CH], float (&b)[CH], const float (&xa)[CH],
                                                const float (&xb)[CH], const float (&ga)[CH], const float (&gb)[CH],
                                                const float (&ca)[CH], const float (&sa)[CH], bool rotate, float tau,
                                                float inv_d, float (&ga_acc)[CH], float (&gb_acc)[CH]) {
  if (rotate) {
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      const float c = rnd<T>(ca[e]), s = rnd<T>(sa[e]);
      const float d1 = a[e], d2 = b[e];
      a[e] = rnd<T>(rnd<T>(mul_rn(d1, c)) + rnd<T>(mul_rn(d2, s)));
      b[e] = rnd<T>(rnd<T>(mul_rn(d2, c)) - rnd<T>(mul_rn(d1, s)));
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    ga_acc[e] += mul_rn(a[e], mul_rn(xa[e], tau));
    gb_acc[e] += mul_rn(b[e], mul_rn(xb[e], tau));
    a[e] = mul_rn(ga[e], a[e]);
    b[e] = mul_rn(gb[e], b[e]);
    s += mul_rn(a[e], xa[e]) + mul_rn(b[e], xb[e]);
  }
  s = row_sum<LPR>(s);
  const float coef = mul_rn(mul_rn(mul_rn(tau, tau), tau), s) * inv_d;
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    a[e] = rnd<T>(__fsub_rn(mul_rn(a[e], tau), mul_rn(xa[e], coef)));
    b[e] = rnd<T>(__fsub_rn(mul_rn(b[e], tau), mul_rn(xb[e], coef)));
  }
}

template <typename T, int D, bool ROT>
__global__ __launch_bounds__(256) void attn_qk_prologue_bwd_kernel(QkPrologueBwdParams p) {
  constexpr int CH = 16 / sizeof(T), HALF = D / 2, LPR = HALF / CH, RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, li = lane - sub * LPR;
  const int c0 = li * CH;
  float gqa[CH], gqb[CH], gka[CH], gkb[CH];
  float aq_a[CH], aq_b[CH], ak_a[CH], ak_b[CH];  // gain-gradient accumulators
  load_gain_halves<CH>(p.q_gain, c0, HALF, gqa, gqb);
  load_gain_halves<CH>(p.k_gain, c0, HALF, gka, gkb);
#pragma unroll
  for (int e = 0; e < CH; ++e) aq_a[e] = aq_b[e] = ak_a[e] = ak_b[e] = 0.0f;
  constexpr bool rotate = ROT;
  const float inv_d = 1.0f / (float)D;
  const RowAddr ra = head_rows(p.H, p.T, D, p.layout);
  const int t0 = blockIdx.y * (4 * RPW * PRO_ITER) + wave * RPW + sub;
  constexpr int U = PRO_U;
#pragma unroll 1
  for (int j = 0; j < PRO_ITER; j += U) {
    uint4 rxq[U][2], rxk[U][2], rdq[U][2], rdk[U][2];
    float ca[U][CH], sa[U][CH], tq[U], tk[U];
    size_t in[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + 4 * RPW * (j + u);
      ok[u] = t < p.T;
      const int tc = ok[u] ? t : p.T - 1;
      in[u] = ra.base + (size_t)tc * ra.stride + c0;
      const size_t gr = in[u];
      rxq[u][0] = ld16<T>(p.q, in[u]);
      rxq[u][1] = ld16<T>(p.q, in[u] + HALF);
      rxk[u][0] = ld16<T>(p.k, in[u]);
      rxk[u][1] = ld16<T>(p.k, in[u] + HALF);
      rdq[u][0] = ld16<T>(p.dq_r, gr);
      rdq[u][1] = ld16<T>(p.dq_r, gr + HALF);
      rdk[u][0] = ld16<T>(p.dk_r, gr);
      rdk[u][1] = ld16<T>(p.dk_r, gr + HALF);
      const size_t row = (size_t)blockIdx.x * p.T + tc;
      tq[u] = p.tau_q[row];
      tk[u] = p.tau_k[row];
      if constexpr (ROT) {
        load_f32<CH>(p.cos + (size_t)tc * HALF + c0, ca[u]);
        load_f32<CH>(p.sin + (size_t)tc * HALF + c0, sa[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float xqa[CH], xqb[CH], xka[CH], xkb[CH], dqa[CH], dqb[CH], dka[CH], dkb[CH];
      cvt_chunk<T, CH>(rxq[u][0], xqa);
      cvt_chunk<T, CH>(rxq[u][1], xqb);
      cvt_chunk<T, CH>(rxk[u][0], xka);
      cvt_chunk<T, CH>(rxk[u][1], xkb);
      cvt_chunk<T, CH>(rdq[u][0], dqa);
      cvt_chunk<T, CH>(rdq[u][1], dqb);
      cvt_chunk<T, CH>(rdk[u][0], dka);
      cvt_chunk<T, CH>(rdk[u][1], dkb);
      float zq_a[CH], zq_b[CH], zk_a[CH], zk_b[CH];
#pragma unroll
      for (int e = 0; e < CH; ++e) zq_a[e] = zq_b[e] = zk_a[e] = zk_b[e] = 0.0f;
      norm_rotate_vjp<T, CH, LPR>(dqa, dqb, xqa, xqb, gqa, gqb, ca[u], sa[u], rotate, tq[u], inv_d, zq_a, zq_b);
      norm_rotate_vjp<T, CH, LPR>(dka, dkb, xka, xkb, gka, gkb, ca[u], sa[u], rotate, tk[u], inv_d, zk_a, zk_b);
      if (ok[u]) {
        store_chunk<T, CH>(p.dq, in[u], dqa);
        store_chunk<T, CH>(p.dq, in[u] + HALF, dqb);
        store_chunk<T, CH>(p.dk, in[u], dka);
        store_chunk<T, CH>(p.dk, in[u] + HALF, dkb);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
          aq_a[e] += zq_a[e]; aq_b[e] += zq_b[e];
          ak_a[e] += zk_a[e]; ak_b[e] += zk_b[e];
        }
      }
    }
  }
  // Gain-gradient partials: lanes with the same li (same columns) are LPR apart.
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    for (int m = LPR; m < 64; m <<= 1) {
      aq_a[e] += __shfl_xor(aq_a[e], m, 64);
      aq_b[e] += __shfl_xor(aq_b[e], m, 64);
      ak_a[e] += __shfl_xor(ak_a[e], m, 64);
      ak_b[e] += __shfl_xor(ak_b[e], m, 64);
    }
  }
  __shared__ float red[4][2][D];
  if (sub == 0) {
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      red[wave][0][c0 + e] = aq_a[e];
      red[wave][0][HALF + c0 + e] = aq_b[e];
      red[wave][1][c0 + e] = ak_a[e];
      red[wave][1][HALF + c0 + e] = ak_b[e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * D; i += 256) {
    const int x = i / D, d = i - x * D;
    const size_t nb = (size_t)gridDim.x * gridDim.y, blk = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    p.gpart[(size_t)i * nb + blk] = red[0][x][d] + red[1][x][d] + red[2][x][d] + red[3][x][d];
  }
}

// Gain gradients: one workgroup per column sums that column's per-block partials (stored
// column by column) with a fixed-order tree.
__global__ __launch_bounds__(256) void attn_qk_gain_reduce_kernel(const float* gpart, int nblocks, int D,
                                                                  float* dq_gain, float* dk_gain) {
  __shared__ float red[256];
  const int i = blockIdx.x;
  float s = 0.0f;
  for (int b = threadIdx.x; b < nblocks; b += 256) s += gpart[(size_t)i * nblocks + b];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float* dst = i < D ? dq_gain : dk_gain;
    if (dst) dst[i < D ? i : i - D] = red[0];
  }
}

// Positions per workgroup: 4 waves x rows per wave x PRO_ITER.
int attn_qk_rows_per_wg(int D, bool bf16_io) {
  const int ch = bf16_io ? 8 : 4;
  const int lpr = D / 2 / ch;
  return 4 * (64 / lpr) * PRO_ITER;
}
// Workgroups of the prologue grids; sizes the guard and gain partials (an upper bound over
// both dtypes when bf16_io is unknown: the f32 rows per workgroup are the fewer).
int attn_qk_prologue_blocks(int B, int H, int T, int D, bool bf16_io) {
  const int rpw = attn_qk_rows_per_wg(D, bf16_io);
  return B * H * ((T + rpw - 1) / rpw);
}

hipError_t launch_cayley_tables(const float* w, int half, int T, float* cos_out, float* sin_out, hipStream_t st) {
  const long n = (long)T * half;
  hipLaunchKernelGGL(cayley_tables_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, half, T, cos_out,
                     sin_out);
  return hipGetLastError();
}

hipError_t launch_attn_qk_prologue(const QkPrologueParams& p, bool bf16_io, GuardParams g, hipStream_t st) {
  const int nb = attn_qk_prologue_blocks(p.B, p.H, p.T, p.D, bf16_io);
  const dim3 grid(p.B * p.H, (p.T + attn_qk_rows_per_wg(p.D, bf16_io) - 1) / attn_qk_rows_per_wg(p.D, bf16_io));
  {
    KTimer t("attn_qk_prologue", st);
    auto go = [&](auto tc, auto dc) {
      typedef decltype(tc) T;
      constexpr int D = decltype(dc)::value;
      const bool rot = p.cos != nullptr, guard = p.want_guard != 0;
      if (rot && guard) hipLaunchKernelGGL((attn_qk_prologue_kernel<T, D, true, true>), grid, dim3(256), 0, st, p);
      else if (rot) hipLaunchKernelGGL((attn_qk_prologue_kernel<T, D, true, false>), grid, dim3(256), 0, st, p);
      else if (guard) hipLaunchKernelGGL((attn_qk_prologue_kernel<T, D, false, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((attn_qk_prologue_kernel<T, D, false, false>), grid, dim3(256), 0, st, p);
    };
    if (bf16_io) {
      if (p.D == 128) go(bf16{}, std::integral_constant<int, 128>{});
      else go(bf16{}, std::integral_constant<int, 64>{});
    } else {
      if (p.D == 128) go(float{}, std::integral_constant<int, 128>{});
      else go(float{}, std::integral_constant<int, 64>{});
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  g.part = p.part;
  g.nblocks = nb;
  return launch_attn_guard(g, st);
}

hipError_t launch_attn_qk_prologue_bwd(const QkPrologueBwdParams& p, bool bf16_io, float* dq_gain, float* dk_gain,
                                       hipStream_t st) {
  const int nb = attn_qk_prologue_blocks(p.B, p.H, p.T, p.D, bf16_io);
  const dim3 grid(p.B * p.H, (p.T + attn_qk_rows_per_wg(p.D, bf16_io) - 1) / attn_qk_rows_per_wg(p.D, bf16_io));
  {
    KTimer t("attn_qk_prologue_bwd", st);
    auto go = [&](auto tc, auto dc) {
      typedef decltype(tc) T;
      constexpr int D = decltype(dc)::value;
      if (p.cos) hipLaunchKernelGGL((attn_qk_prologue_bwd_kernel<T, D, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((attn_qk_prologue_bwd_kernel<T, D, false>), grid, dim3(256), 0, st, p);
    };
    if (bf16_io) {
      if (p.D == 128) go(bf16{}, std::integral_constant<int, 128>{});
      else go(bf16{}, std::integral_constant<int, 64>{});
    } else {
      if (p.D == 128) go(float{}, std::integral_constant<int, 128>{});
      else go(float{}, std::integral_constant<int, 64>{});
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (dq_gain || dk_gain) {
    KTimer t("attn_qk_gain_reduce", st);
    hipLaunchKernelGGL(attn_qk_gain_reduce_kernel, dim3(2 * p.D), dim3(256), 0, st, p.gpart, nb, p.D, dq_gain,
                       dk_gain);
  }
  return hipGetLastError();
}

}  // namespace alg
