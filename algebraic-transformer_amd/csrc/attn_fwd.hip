// Causal algebraic attention forward for gfx950.
//
// Replaces the Pallas forward kernels src/algebraic/kernels/flash.py:189-326 and
// src/algebraic/kernels/head_resident.py:25-89 (same maths, MI355X tiling).
//
// Work decomposition: one workgroup = 4 waves = 128 query rows of one (b, h); each wave owns
// 32 consecutive queries and streams K/V through LDS in 64-key tiles. Scores are formed
// transposed, S^T = K Q^T (32x32x16 bf16 MFMA, or 32x32x2 f32 MFMA for f32 inputs), so
// every lane owns one query column: the per-row weight sum is a per-lane running sum,
// reduced across the two lane halves once at the end, and the running maximum of the
// shifted variant is per lane as well. The weight tile P^T feeds the PV product directly
// as the B operand of O^T = V^T P^T; V^T fragments come from the row-major LDS tile with
// ds_read_b64_tr_b16. Causal tiles above the diagonal are skipped per wave; only tiles
// crossing it evaluate the mask.
#include <type_traits>

#include "attn_common.h"

namespace alg {

constexpr int FWD_BK = 64;   // keys per LDS tile

template <typename T>
__device__ __forceinline__ void load_rows(T* dst, int pitch, const T* src, int r0, int nrows, int T_, int D) {
  constexpr int CH = 16 / sizeof(T);
  const int cpr = D / CH;
  for (int c = threadIdx.x; c < nrows * cpr; c += blockDim.x) {
    const int row = c / cpr, col = (c - row * cpr) * CH;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (r0 + row < T_) val = *reinterpret_cast<const uint4*>(src + (size_t)(r0 + row) * D + col);
    *reinterpret_cast<uint4*>(dst + row * pitch + col) = val;
  }
}

// Registers <-> LDS staging of one 64-row K or V tile (16-byte chunks, rows >= T are zero).
template <typename T, int D>
struct KVTile {
  static constexpr int CH = 16 / sizeof(T);
  static constexpr int CPR = D / CH;
  static constexpr int PER = FWD_BK * CPR / 256;  // chunks per thread
  static __device__ __forceinline__ void load(uint4 (&r)[PER], const T* src, int r0, int T_, int ld) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx / CPR, col = (idx - row * CPR) * CH;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r0 + row < T_) v = *reinterpret_cast<const uint4*>(src + (size_t)(r0 + row) * ld + col);
      r[c] = v;
    }
  }
  // bf16 tiles are unpadded and swizzled (swz_at); f32 tiles are row-major with `pitch`.
  static __device__ __forceinline__ void store(T* dst, int pitch, const uint4 (&r)[PER]) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx / CPR, col = (idx - row * CPR) * CH;
      if constexpr (sizeof(T) == 2) *reinterpret_cast<uint4*>(dst + swz_at<CPR>(row, col)) = r[c];
      else *reinterpret_cast<uint4*>(dst + row * pitch + col) = r[c];
    }
  }
};

template <typename T, int D, int MODE, int L2N>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnFwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr bool BF = sizeof(T) == 2;
  constexpr int PITCH = D + F32_PAD;  // f32 tiles
  constexpr int CPR = D / 8;          // bf16 tiles: 16-byte chunks per row
  constexpr int TILE = BF ? FWD_BK * D : FWD_BK * PITCH;
  constexpr int NDB = D / 32;  // 32-wide d blocks of the O^T accumulator
  typedef KVTile<T, D> KV;
  __shared__ __attribute__((aligned(16))) T Ks[2][TILE];
  __shared__ __attribute__((aligned(16))) T Vs[2][TILE];

  if (p.flag) {  // device-side guard dispatch (lax.cond at flash.py:853-856)
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int T_ = p.T;
  const int nqb = ceil_div(T_, FWD_BQ);
  // One 128-query block of one head. The in-range kernel takes one per workgroup from its 2-D
  // grid; the fallbacks loop over them (grid-stride), heaviest causal rows first.
  auto run = [&](int bh, int qb) __attribute__((always_inline)) {
  const int head = bh % p.H;
  const size_t base = (size_t)bh * T_ * D;  // internal (B, H, T, D) buffers (o_precise)
  const size_t hb = head_base(bh, p.H, T_, D, p.layout);
  const int ld = row_stride(p.H, D, p.layout);
  const T* Q = reinterpret_cast<const T*>(p.q) + hb;
  const T* K = reinterpret_cast<const T*>(p.k) + hb;
  const T* V = reinterpret_cast<const T*>(p.v) + hb;
  const int q0 = qb * FWD_BQ + wave * 32;
  const int myq = q0 + l32;
  const bool wave_live = q0 < T_;

  // Query fragments (B operand of S^T = K Q^T), held for the whole kernel.
  constexpr int NQF = BF ? D / 16 : D / 8;
  typedef typename std::conditional<BF, bf16x8, floatx4>::type QFrag;
  QFrag qf[NQF];
#pragma unroll
  for (int s = 0; s < NQF; ++s) {
    if constexpr (BF) {
      bf16x8 z = {};
      qf[s] = myq < T_ ? ld8(reinterpret_cast<const bf16*>(Q) + (size_t)myq * ld + 16 * s + 8 * h) : z;
    } else {
      floatx4 z = {};
      qf[s] = myq < T_ ? *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(Q) + (size_t)myq * ld + 8 * s + 4 * h) : z;
    }
  }

  const int log2n = p.log2n;
  const bool has_sink = p.sink != nullptr;
  const float beta = has_sink ? p.sink[head] : 0.0f;
  floatx16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = floatx16{};
  float lsum = 0.0f;
  // Shifted state (flash.py:209-214): m = sink or NEG, l = 1 (sink) or 0; the sink's unit
  // mass sits in lane half 0 so the half-sum reduction counts it once.
  float m_run = has_sink ? beta : -1e4f;
  if (MODE == MODE_SHIFTED && has_sink && h == 0) lsum = 1.0f;
  bool first = true;

  // One 32-key block of the tile in buffer `buf`: S^T, weights, O^T += V^T P^T.
  auto block = [&](int buf, int sub, int kb, bool diag) {
    const T* krow = Ks[buf] + (sub * 32 + l32) * PITCH;
    floatx16 s = {};
#pragma unroll
    for (int st = 0; st < NQF; ++st) {
      if constexpr (BF) {
        bf16x8 kf = *reinterpret_cast<const bf16x8*>(Ks[buf] + swz_at<CPR>(sub * 32 + l32, 16 * st + 8 * h));
        s = mfma_bf16(kf, qf[st], s);
      } else {
        floatx4 kf = *reinterpret_cast<const floatx4*>(krow + 8 * st + 4 * h);
#pragma unroll
        for (int u = 0; u < 4; ++u) s = mfma_f32(kf[u], qf[st][u], s);
      }
    }
    float w[16];
    if constexpr (MODE != MODE_SHIFTED) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = s[i];
        if constexpr (MODE == MODE_CLIPPED) x = fminf(x, p.clamp);
        w[i] = pow2n<L2N>(rho_fast(x), log2n);
      }
      if (diag) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key > myq) w[i] = 0.0f;
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) lsum += w[i];
    } else {
      // Running maximum over this 32-key block (flash.py:235-259).
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
        if (!diag || key <= myq) tmax = fmaxf(tmax, s[i]);
      }
      tmax = fmaxf(tmax, xor32(tmax));
      float m_new = fmaxf(m_run, tmax);
      float m_prev = m_run;
      if (!has_sink && first) { m_new = tmax; m_prev = tmax; }
      const float shift = rho_exact(-m_new);
      const float alpha = ipow_rt(rho_exact(m_prev) * shift, 1 << log2n);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
        const bool valid = !diag || key <= myq;
        const float x = valid ? s[i] : 0.0f;
        const float r0 = p.fast_rho ? rho_fast(x) : rho_exact(x);
        const float t = pow2n<L2N>(r0 * shift, log2n);
        w[i] = valid ? t : 0.0f;
      }
      float ts = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) ts += w[i];
      lsum = alpha * lsum + ts;
#pragma unroll
      for (int db = 0; db < NDB; ++db) oacc[db] = oacc[db] * alpha;
      m_run = m_new;
    }
    first = false;
    if constexpr (BF) {
      bf16x8 pf0, pf1;
#pragma unroll
      for (int j = 0; j < 8; ++j) { pf0[j] = f2bf(w[j]); pf1[j] = f2bf(w[8 + j]); }
      const bf16* vt = reinterpret_cast<const bf16*>(Vs[buf]);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        bf16x8 v0 = swz_tr_frag<CPR>(vt, sub * 32 + 4 * h, sub * 32 + 8 + 4 * h, db * 32, lane);
        oacc[db] = mfma_bf16(v0, pf0, oacc[db]);
        bf16x8 v1 = swz_tr_frag<CPR>(vt, sub * 32 + 16 + 4 * h, sub * 32 + 24 + 4 * h, db * 32, lane);
        oacc[db] = mfma_bf16(v1, pf1, oacc[db]);
      }
    } else {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int krow_i = sub * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          const float a = reinterpret_cast<const float*>(Vs[buf])[krow_i * PITCH + db * 32 + l32];
          oacc[db] = mfma_f32(a, w[i], oacc[db]);
        }
      }
    }
  };

  const int q_last = min(qb * FWD_BQ + FWD_BQ, T_) - 1;
  const int ntiles = q_last / FWD_BK + 1;
  // K/V tiles are double-buffered: the next tile's global loads are in flight while the
  // current tile is consumed; one barrier per tile.
  uint4 kr[KV::PER], vr[KV::PER];
  KV::load(kr, K, 0, T_, ld);
  KV::load(vr, V, 0, T_, ld);
  KV::store(Ks[0], PITCH, kr);
  KV::store(Vs[0], PITCH, vr);
  __syncthreads();
  for (int kt = 0; kt < ntiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ntiles;
    if (more) {
      KV::load(kr, K, (kt + 1) * FWD_BK, T_, ld);
      KV::load(vr, V, (kt + 1) * FWD_BK, T_, ld);
    }
    if (wave_live) {
      const int kb0 = kt * FWD_BK;
      if (kb0 + FWD_BK - 1 <= q0) {  // every key precedes every query of this wave: no mask
        block(cur, 0, kb0, false);
        block(cur, 1, kb0 + 32, false);
      } else {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const int kb = kb0 + sub * 32;
          if (kb <= q0 + 31 && kb < T_) block(cur, sub, kb, kb + 31 > q0);
        }
      }
    }
    if (more) {
      KV::store(Ks[cur ^ 1], PITCH, kr);
      KV::store(Vs[cur ^ 1], PITCH, vr);
    }
    __syncthreads();
  }
  if (!wave_live) return;

  // Finalize (flash.py:271-284).
  float Z = lsum + xor32(lsum);
  float stat;
  if constexpr (MODE != MODE_SHIFTED) {
    if (has_sink) {
      float b = beta;
      if constexpr (MODE == MODE_CLIPPED) b = fminf(b, p.clamp);
      Z += pow2n<L2N>(rho_fast(b), log2n);
    }
    const float inv = 1.0f / Z;
    stat = (MODE == MODE_CLIPPED && !p.inv_stat) ? inv_root(Z, 1 << log2n) : inv;
    Z = inv;  // reuse as the output scale
  } else {
    stat = rho_exact(-m_run) * inv_root(Z, 1 << log2n);
    Z = 1.0f / Z;
  }
  const float scale = Z;
  if (myq < T_) {
    T* O = reinterpret_cast<T*>(p.o) + hb + (size_t)myq * ld;
    // o_precise carries the shifted branch's unrounded output only (flash.py:322).
    float* OP = (MODE == MODE_SHIFTED && p.o_precise) ? p.o_precise + base + (size_t)myq * D : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * h;
        floatx4 val;
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = oacc[db][4 * g + e] * scale;
        if constexpr (BF) {
          bf16x4 ob;
#pragma unroll
          for (int e = 0; e < 4; ++e) ob[e] = f2bf(val[e]);
          *reinterpret_cast<bf16x4*>(O + d0) = ob;
        } else {
          *reinterpret_cast<floatx4*>(O + d0) = val;
        }
        if (OP) *reinterpret_cast<floatx4*>(OP + d0) = val;
      }
    }
    if (h == 0) p.stat[(size_t)bh * T_ + myq] = stat;
  }
  };
  if constexpr (MODE == MODE_INRANGE) {
    run(blockIdx.x, nqb - 1 - blockIdx.y);
  } else {
    const int nbh = p.B * p.H;
    for (int L = blockIdx.x; L < nbh * nqb; L += gridDim.x) {
      run(L % nbh, nqb - 1 - L / nbh);
      __syncthreads();  // the next block's first K/V tile overwrites LDS
    }
  }
}

// In-range forward for f32 inputs at D = 64 with each row's keys split over several waves:
// one workgroup = QG groups of 32 queries of one (b, h) (lane = query), and each group's
// causal key range (its 32-key tiles) is split over KS = 4 / QG waves, wave part j taking the
// j-th run of ceil(tiles / KS) tiles. Every part streams its own K/V tiles (all 256 threads
// stage the parts' next tiles in registers while the current ones are consumed). At the end
// parts 1.. add their O^T partials and row sums to part 0's through LDS, in part order, and
// part 0 finalizes. An fp32 MFMA (v_mfma_f32_32x32x2f32) takes 64 cycles and a row's work
// grows along the causal range, so at small batch (24 heads of 1024 positions) the longest
// rows set the time: the split divides that path by KS and multiplies the workgroups by
// 4 / QG. The row sum is accumulated in KS parts and added at the end, an order of f32
// additions of its own (the mathematics is that of attn_fwd_kernel's in-range branch).
constexpr int F32S_BK = 32;  // keys per tile
__device__ __forceinline__ float guard_max(float a, float b);
// FROM_Q: the guarded forward's first launch (as attn_fwd_bf16_kernel's): q holds the raw
// queries; the kernel forms q_s = q * alpha in its query fragments, writes it, and leaves its
// workgroup's guard maxima (its queries' ||q_s||^2, and ||k||^2 and |v| of the key rows at its
// own query positions) with the row sums in the prep kernel's order, so the guard decides
// exactly as after alg_attn_prepare.
template <int QG, int L2N, bool FROM_Q>
__global__ __launch_bounds__(256, 2) void attn_fwd_f32_split_kernel(AttnFwdParams p) {
  static_assert(QG == 1 || QG == 2, "query groups per workgroup");
  constexpr int KS = 4 / QG, BQ = 32 * QG;
  constexpr int D = 64, PITCH = D + F32_PAD, TILE = F32S_BK * PITCH, NDB = D / 32, NQF = D / 8;
  constexpr int CPR = D / 4;                 // 16-byte chunks per row
  constexpr int PER = F32S_BK * CPR / 256;   // chunks per thread and tile
  __shared__ __attribute__((aligned(16))) float Ks[KS][TILE];  // [part]
  __shared__ __attribute__((aligned(16))) float Vs[KS][TILE];

  if (p.flag && *p.flag == 0) return;  // device-side guard dispatch (flash.py:853-856)
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int qg = wave % QG, part = wave / QG;
  const int T_ = p.T;
  const int nqb = ceil_div(T_, BQ);
  const int bh = blockIdx.x;
  const int qb = nqb - 1 - blockIdx.y;  // heaviest causal rows first
  const int head = bh % p.H;
  const size_t hb = head_base(bh, p.H, T_, D, p.layout);
  const int ld = row_stride(p.H, D, p.layout);
  const float* Q = reinterpret_cast<const float*>(p.q) + hb;
  const float* K = reinterpret_cast<const float*>(p.k) + hb;
  const float* V = reinterpret_cast<const float*>(p.v) + hb;
  const int q0 = qb * BQ + qg * 32;
  const int myq = q0 + l32;
  const bool wave_live = q0 < T_;

  floatx4 qf[NQF];  // query fragments (B operand of S^T = K Q^T)
#pragma unroll
  for (int s = 0; s < NQF; ++s) {
    const floatx4 z = {};
    qf[s] = myq < T_ ? *reinterpret_cast<const floatx4*>(Q + (size_t)myq * ld + 8 * s + 4 * h) : z;
  }
  if constexpr (FROM_Q) {  // q_s = q * alpha (flash.py:833; an f32 product for f32 inputs)
    const float alpha = p.alpha;
#pragma unroll
    for (int s = 0; s < NQF; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) qf[s][u] = qf[s][u] * alpha;
    if (part == 0 && myq < T_) {
      float* Qs = reinterpret_cast<float*>(p.q_s_out) + hb + (size_t)myq * ld;
#pragma unroll
      for (int s = 0; s < NQF; ++s) *reinterpret_cast<floatx4*>(Qs + 8 * s + 4 * h) = qf[s];
    }
  }
  const int log2n = p.log2n;
  floatx16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = floatx16{};
  float lsum = 0.0f;

  // One 32-key tile: S^T, weights, O^T += V^T P^T (the in-range branch of attn_fwd_kernel,
  // flash.py:215-233).
  auto block = [&](const float* Kt, const float* Vt, int kb, bool diag) {
    const float* krow = Kt + l32 * PITCH;
    floatx16 s = {};
#pragma unroll
    for (int st = 0; st < NQF; ++st) {
      const floatx4 kf = *reinterpret_cast<const floatx4*>(krow + 8 * st + 4 * h);
#pragma unroll
      for (int u = 0; u < 4; ++u) s = mfma_f32(kf[u], qf[st][u], s);
    }
    float w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = pow2n<L2N>(rho_fast(s[i]), log2n);
    if (diag) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
        if (key > myq) w[i] = 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) lsum += w[i];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int krow_i = 8 * (i >> 2) + 4 * h + (i & 3);
        oacc[db] = mfma_f32(Vt[krow_i * PITCH + db * 32 + l32], w[i], oacc[db]);
      }
    }
  };

  // Registers <-> LDS staging of one 32-row tile; rows at or past T read as zeros.
  auto load_tile = [&](uint4 (&r)[PER], const float* src, int r0) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx / CPR, col = (idx - row * CPR) * 4;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r0 + row < T_) v = *reinterpret_cast<const uint4*>(src + (size_t)(r0 + row) * ld + col);
      r[c] = v;
    }
  };
  auto store_tile = [&](float* dst, const uint4 (&r)[PER]) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx / CPR, col = (idx - row * CPR) * 4;
      *reinterpret_cast<uint4*>(dst + row * PITCH + col) = r[c];
    }
  };

  const int q_last = min(qb * BQ + BQ, T_) - 1;
  const int ntiles = q_last / F32S_BK + 1;
  const int nper = ceil_div(ntiles, KS);  // tiles per part (the last parts may have fewer)
  uint4 kr[KS][PER], vr[KS][PER];
  // Step j's tile of every part into registers; a part's rows past its range start at T
  // (read as zeros, never consumed).
  auto load_step = [&](int j) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      const int t = q * nper + j;
      const int r0 = t < ntiles ? t * F32S_BK : T_;
      load_tile(kr[q], K, r0);
      load_tile(vr[q], V, r0);
    }
  };
  load_step(0);
  for (int j = 0; j < nper; ++j) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      store_tile(Ks[q], kr[q]);
      store_tile(Vs[q], vr[q]);
    }
    __syncthreads();
    if (j + 1 < nper) load_step(j + 1);  // in flight while this step's tiles are consumed
    const int t = part * nper + j;
    const int kb = t * F32S_BK;
    // Tiles past the range, or keys past this wave's last query (or past T), are skipped.
    if (wave_live && t < ntiles && kb <= q0 + 31) block(Ks[part], Vs[part], kb, kb + 31 > q0);
    __syncthreads();  // every wave is done with the tiles before the next step stores
  }

  if constexpr (FROM_Q) {
    __shared__ float gred[4][3];
    // ||q_s||^2: chunk 2s + h (4 columns) of row myq is qf[s] on lane half h; each chunk is
    // summed in column order, chunks 2s and 2s + 1 meet across the halves, and the pair sums
    // combine in the prep kernel's butterfly order. Only part 0's waves hold distinct rows.
    float ps[NQF];
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      floatx4 qv = qf[s];
      asm volatile("" : "+v"(qv));  // formed here, not carried through the main loop
      float c = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) c += qv[u] * qv[u];
      ps[s] = c + __shfl_xor(c, 32, 64);
    }
#pragma unroll
    for (int w = 1; w < NQF; w <<= 1)
#pragma unroll
      for (int s = 0; s < NQF; s += 2 * w) ps[s] = ps[s] + ps[s + w];
    float mq = part == 0 && myq < T_ ? ps[0] : 0.0f;
    // ||k||^2 and |v| of the key rows at this workgroup's query positions (every row of the
    // head once over the launch): 16 lanes per row, lane li holding columns 4 li .. 4 li + 3.
    float mk = 0.0f, mv = 0.0f;
    {
      const int li = threadIdx.x & 15, rsub = threadIdx.x >> 4;
#pragma unroll
      for (int r = 0; r < BQ; r += 16) {
        const int key = qb * BQ + r + rsub;
        float sk = 0.0f;
        if (key < T_) {
          const floatx4 kv = *reinterpret_cast<const floatx4*>(K + (size_t)key * ld + 4 * li);
          const floatx4 vv = *reinterpret_cast<const floatx4*>(V + (size_t)key * ld + 4 * li);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            sk += kv[u] * kv[u];
            mv = guard_max(mv, __builtin_fabsf(vv[u]));
          }
        }
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) sk += __shfl_xor(sk, m, 64);
        mk = guard_max(mk, sk);
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      mq = guard_max(mq, __shfl_xor(mq, m, 64));
      mk = guard_max(mk, __shfl_xor(mk, m, 64));
      mv = guard_max(mv, __shfl_xor(mv, m, 64));
    }
    if (lane == 0) {
      gred[wave][0] = mq;
      gred[wave][1] = mk;
      gred[wave][2] = mv;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
      float m = gred[0][threadIdx.x];
#pragma unroll
      for (int w = 1; w < 4; ++w) m = guard_max(m, gred[w][threadIdx.x]);
      p.guard_part[3 * ((size_t)bh * gridDim.y + blockIdx.y) + threadIdx.x] = m;
    }
  }

  // Parts 1.. hand their O^T partials and row sums to part 0 through LDS (the tiles are free
  // after the loop's last barrier): RS floats per lane, an odd stride (no bank conflicts).
  constexpr int RS = 16 * NDB + 1;
  static_assert((KS - 1) * QG * 64 * RS <= KS * TILE, "partials fit the K tiles");
  float* red = &Ks[0][0];
  if (part > 0) {
    float* dst = red + (((part - 1) * QG + qg) * 64 + lane) * RS;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[db * 16 + i] = oacc[db][i];
    dst[16 * NDB] = lsum;
  }
  __syncthreads();
  if (part > 0 || !wave_live) return;
#pragma unroll
  for (int q = 1; q < KS; ++q) {
    const float* src = red + (((q - 1) * QG + qg) * 64 + lane) * RS;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[db][i] += src[db * 16 + i];
    lsum += src[16 * NDB];
  }

  // Finalize (flash.py:271-284): Z over both lane halves (+ the sink's weight), stat = 1/Z.
  float Z = lsum + xor32(lsum);
  if constexpr (FROM_Q) {
    if (p.sink_logit) Z += pow2n<L2N>(rho_fast(p.sink_logit[p.sink_count == 1 ? 0 : head] / p.sink_c), log2n);
  } else {
    if (p.sink) Z += pow2n<L2N>(rho_fast(p.sink[head]), log2n);
  }
  const float inv = 1.0f / Z;
  if (myq < T_) {
    float* O = reinterpret_cast<float*>(p.o) + hb + (size_t)myq * ld;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 val;
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = oacc[db][4 * g + e] * inv;
        *reinterpret_cast<floatx4*>(O + db * 32 + 8 * g + 4 * h) = val;
      }
    }
    if (h == 0) p.stat[(size_t)bh * T_ + myq] = inv;
  }
}

// NaN-propagating maximum of the guard (a NaN anywhere fails it, as the reference's
// comparisons do).
__device__ __forceinline__ float guard_max(float a, float b) { return (a > b || a != a) ? a : b; }

// Guard maxima of one forward workgroup (flash.py:841-849) over the queries it owns and the
// keys at the same positions q0 .. q0 + FWD_BQ - 1, so the workgroups of a launch cover every
// row once. Row sums follow the chunk order of the prep kernel (8 elements per 16-byte chunk,
// then a butterfly over the row's chunks), so the guard sees the same sums either way.
//
// Keys and values: the workgroup's own key rows are its two diagonal tiles, which pass
// through LDS anyway; guard_kv_tile folds one such tile (rows past T are zero-filled there and
// add nothing) into the thread's running maxima mk (||k||^2) and mvb (|v|). |v| is tracked on
// the bf16 bit patterns: with the sign cleared they order as the magnitudes do, every NaN
// above infinity, so a packed 16-bit integer maximum over (bits & 0x7fff) pairs is the
// NaN-propagating maximum of |v| (guard_v_max turns it back into a float) at one instruction
// per two values.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
template <int D>
__device__ __forceinline__ void guard_kv_tile(const bf16* Ks, const bf16* Vs, float& mk, u16x2& mvb) {
  constexpr int CPR = D / 8, RPS = 256 / CPR, NR = FWD_BK / RPS;
  const int c = threadIdx.x % CPR, r0 = threadIdx.x / CPR;
  uint4 kr[NR], vr[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    kr[i] = *reinterpret_cast<const uint4*>(Ks + swz_at<CPR>(r0 + RPS * i, 8 * c));
    vr[i] = *reinterpret_cast<const uint4*>(Vs + swz_at<CPR>(r0 + RPS * i, 8 * c));
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    bf16 kv[8];
    *reinterpret_cast<uint4*>(kv) = kr[i];
    float sk = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float kf = (float)kv[j];
      sk += kf * kf;
    }
    const unsigned vw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      mvb = __builtin_elementwise_max(mvb, __builtin_bit_cast(u16x2, vw[j] & 0x7fff7fffu));
#pragma unroll
    for (int m = 1; m < CPR; m <<= 1) sk += __shfl_xor(sk, m, 64);
    mk = guard_max(mk, sk);
  }
}

// |v| maximum from guard_kv_tile's bit patterns: the larger half; NaN above 0x7f80 (infinity).
__device__ __forceinline__ float guard_v_max(u16x2 mvb) {
  const unsigned m = mvb.x > mvb.y ? mvb.x : mvb.y;
  return m > 0x7f80u ? __builtin_nanf("") : __uint_as_float(m << 16);
}

// Queries, from the fragments the kernel holds, and the workgroup's maxima: called by every
// thread once the main loop is done; writes part[0..2].
template <int D>
__device__ __forceinline__ void fwd_guard_partials(const bf16x8 (&qf)[D / 16], bool live, float mk, float mv,
                                                   float* part, float (&red)[4][3]) {
  constexpr int NF = D / 16;
  // The thread index and the query fragments pass through empty asm statements so the compiler
  // forms the row sums here, after the main loop, instead of computing them early and carrying
  // them through it (that cost the kernel 10-19 more VGPRs, and at D = 64 one wave per SIMD of
  // occupancy).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6;
  // Chunk 2s + h of row myq is qf[s] on lane half h; chunks 2s and 2s + 1 meet across the
  // halves, then the pair sums combine in the butterfly's order.
  float ps[NF];
#pragma unroll
  for (int s = 0; s < NF; ++s) {
    float c = 0.0f;
    bf16x8 qv = qf[s];
    asm volatile("" : "+v"(qv));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = (float)qv[j];
      c += f * f;
    }
    ps[s] = c + __shfl_xor(c, 32, 64);
  }
#pragma unroll
  for (int w = 1; w < NF; w <<= 1)
#pragma unroll
    for (int s = 0; s < NF; s += 2 * w) ps[s] = ps[s] + ps[s + w];
  float mq = live ? ps[0] : 0.0f;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    mq = guard_max(mq, __shfl_xor(mq, m, 64));
    mk = guard_max(mk, __shfl_xor(mk, m, 64));
    mv = guard_max(mv, __shfl_xor(mv, m, 64));
  }
  if (lane == 0) {
    red[wave][0] = mq;
    red[wave][1] = mk;
    red[wave][2] = mv;
  }
  __syncthreads();
  if (tid < 3) {
    float m = red[0][tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = guard_max(m, red[w][tid]);
    part[tid] = m;
  }
}

// In-range forward for bf16 inputs (the guarded "low" variant): same decomposition as
// attn_fwd_kernel (4 waves x 32 queries, lane = query, S^T = K Q^T, O^T += V^T P^T), with K/V
// tiles in two ping-pong LDS buffer sets, each filled by range-checked buffer copies issued
// during the previous tile's first steps, and each 64-key tile software-pipelined over its two
// 32-key blocks:
//   R1  S^T of keys 0..31 | copy of the next tile (MFMA | VMEM)
//   R2  S^T of keys 32..63 | weights of 0..31   (MFMA | VALU)
//   R3  O^T over keys 0..31 | weights of 32..63 (MFMA | VALU)
//   R4  O^T over keys 32..63                    (MFMA)
// The two tiles that cross this workgroup's diagonal evaluate the causal mask per element.
// FROM_Q: the guarded forward's first launch, before the guard has run (no flag to read): q
// holds the raw queries; the kernel rounds q * alpha into its query fragments, writes them out
// as q_s, and leaves its guard maxima for the guard kernel (fwd_guard_partials).
template <int D, int L2N, int LAYOUT, bool FROM_Q>
__global__ __launch_bounds__(256, 2) void attn_fwd_bf16_kernel(AttnFwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr int BK = FWD_BK, CPR = D / 8, NDB = D / 32, NF = D / 16;
  __shared__ __attribute__((aligned(16))) bf16 Ks0[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Ks1[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Vs0[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Vs1[BK * D];
  __shared__ float gred[FROM_Q ? 4 : 1][3];

  if (p.flag && *p.flag == 0) return;  // device-side guard dispatch (flash.py:853-856)
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  const int nqb = ceil_div(T_, FWD_BQ);
  const int bh = blockIdx.x;
  const int qb = nqb - 1 - blockIdx.y;  // heaviest causal rows first
  const int head = bh % p.H;
  const size_t base = head_base(bh, p.H, T_, D, LAYOUT);
  const int ld = LAYOUT ? p.H * D : D;  // elements between positions
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + base;
  const bf16* K = reinterpret_cast<const bf16*>(p.k) + base;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + base;
  const int nbytes = head_bytes(T_, ld, D, 2);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)K, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)V, (short)0, nbytes, BUF_RSRC_WORD3);
  const int myq = qb * FWD_BQ + wave * 32 + l32;
  const int wave_qmax = qb * FWD_BQ + wave * 32 + 31;  // this wave's last query (wave-uniform)
  const int log2n = p.log2n;
  const int ntiles = min(qb * FWD_BQ + FWD_BQ - 1, T_ - 1) / BK + 1;  // key tiles up to the last query

  constexpr int PW = 64 * CPR / 64 / 4;  // copy instruction pairs per wave and tile
  tile_dma2<D>(Ks0, Vs0, rk, rv, 0, wave, lane, ld);
  // Query fragments (B operand of S^T = K Q^T), held for the whole kernel.
  bf16x8 qf[NF];
  const bool live = myq < T_;
#pragma unroll
  for (int s = 0; s < NF; ++s) {
    const bf16x8 z = {};
    qf[s] = live ? ld8(Q + (size_t)myq * ld + 16 * s + 8 * h) : z;
  }
  if constexpr (FROM_Q) {  // q_s = round(q * alpha) (flash.py:833)
    const float alpha = p.alpha;
    bf16* Qs = reinterpret_cast<bf16*>(p.q_s_out) + base + (size_t)myq * ld;
#pragma unroll
    for (int s = 0; s < NF; ++s) {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[s][j] = f2bf((float)qf[s][j] * alpha);
      if (live) *reinterpret_cast<bf16x8*>(Qs + 16 * s + 8 * h) = qf[s];
    }
  }
  floatx16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = floatx16{};
  float lsum = 0.0f;

  const int trow = (lane & 15) >> 2;
  int row_off[NF];  // row fragments of K: row l32, k chunk 2 st + h
#pragma unroll
  for (int st = 0; st < NF; ++st) row_off[st] = swz_at<CPR>(l32, 16 * st + 8 * h);
  int tv_lo[NDB], tv_hi[NDB];  // transposed V fragments: rows 4h + (0..3), 4h + 8 + (0..3)
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tv_lo[db] = swz_at<CPR>(4 * h + trow, tr_col(db * 32, lane));
    tv_hi[db] = swz_at<CPR>(4 * h + 8 + trow, tr_col(db * 32, lane));
  }

  bf16x8 rk3[3];  // row fragments of K, two steps ahead
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
  rk3[0] = ld8(Ks0 + row_off[0]);
  rk3[1] = ld8(Ks0 + row_off[1]);
  constexpr int VE = 10;  // VALU instructions per weight (scheduling hint)

  float gmk = 0.0f;  // FROM_Q: guard maxima of the diagonal tiles' keys and values
  u16x2 gmv = {0, 0};
  auto tile = [&](auto bufc, auto maskc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool MASKED = decltype(maskc)::value;
    const bf16* Ks = BUF ? Ks1 : Ks0;
    const bf16* Vs = BUF ? Vs1 : Vs0;
    const int kb0 = kt * BK;
    if constexpr (FROM_Q && MASKED) guard_kv_tile<D>(Ks, Vs, gmk, gmv);  // this workgroup's own keys
    if constexpr (MASKED) {
      if (kb0 > wave_qmax) {
        // Every key of the tile lies after this wave's queries: all its weights are zero, so
        // the wave only takes part in the copies (none are left after the last tile) and the
        // barrier.
        const int rn = kt + 1 < ntiles ? kb0 + BK : T_ + BK;
#pragma unroll
        for (int g = 0; g < PW; ++g) {
          if constexpr (BUF) tile_dma2_part<D>(Ks0, Vs0, rk, rv, rn, wave, lane, g, ld);
          else tile_dma2_part<D>(Ks1, Vs1, rk, rv, rn, wave, lane, g, ld);
        }
        __builtin_amdgcn_s_waitcnt(VMCNT0);
        __syncthreads();
        const bf16* Kn = BUF ? Ks0 : Ks1;
        rk3[0] = ld8(Kn + row_off[0]);
        rk3[1] = ld8(Kn + row_off[1]);
        return;
      }
    }
    floatx16 s[2];
    bf16x8 pf[2][2];
    float w[16];
    auto s_step = [&](int g) {
      const int blk = g / NF, st = g % NF;
      const int gn = g + 2;
      if (gn < 2 * NF) rk3[gn % 3] = ld8(Ks + (gn / NF) * 32 * D + row_off[gn % NF]);
      s[blk] = mfma_bf16(rk3[g % 3], qf[st], s[blk]);
    };
    // Weight of key element i of block blk for this lane's query (flash.py:215-233).
    auto elem = [&](int blk, int i) {
      float x = s[blk][i];
      float wi = pow2n<L2N>(rho_fast(x), log2n);
      if (MASKED && kb0 + blk * 32 + 8 * (i >> 2) + 4 * h + (i & 3) > myq) wi = 0.0f;
      lsum += wi;
      w[i] = wi;
      if (i & 1) {
        pf[blk][i >> 3][(i & 7) - 1] = f2bf(w[i - 1]);
        pf[blk][i >> 3][i & 7] = f2bf(w[i]);
      }
    };
    bf16x8 ft[2][2];
    auto pv_load = [&](int blk, int db, bf16x8 (&f)[2]) {
      const bf16* vb = Vs + blk * 32 * D;
      f[0] = tr_frag_at(vb, tv_lo[db], tv_hi[db]);
      f[1] = tr_frag_at(vb + 16 * D, tv_lo[db], tv_hi[db]);
    };

    // R1: S^T of keys 0..31, with the copy of the next tile into the other buffer set (free
    // since the barrier that ended the previous tile) spread over its steps, one instruction
    // pair per step: issued in one burst, the copies of the CU's eight waves queue on the
    // vector memory path and stall the waves. Past the last tile the rows lie beyond the
    // descriptors' ranges (no memory is read; zeros land in the unused buffer set).
    s[0] = floatx16{};
    s[1] = floatx16{};
    const int r_next = kt + 1 < ntiles ? kb0 + BK : T_ + BK;
#pragma unroll
    for (int g = 0; g < NF; ++g) {
      s_step(g);
      if (g < PW) {
        if constexpr (BUF) tile_dma2_part<D>(Ks0, Vs0, rk, rv, r_next, wave, lane, g, ld);
        else tile_dma2_part<D>(Ks1, Vs1, rk, rv, r_next, wave, lane, g, ld);
      }
      step_order<1, 0, 2, 0>();
    }
    // R2: S^T of keys 32..63 under the weights of keys 0..31.
    constexpr int E2 = 16 / NF;
#pragma unroll
    for (int g = NF; g < 2 * NF; ++g) {
      s_step(g);
#pragma unroll
      for (int k = 0; k < E2; ++k) elem(0, E2 * (g - NF) + k);
      if (g == 2 * NF - 1) pv_load(0, 0, ft[0]);
      step_order<1, VE * E2, 2, 0>();
    }
    // R3: O^T over keys 0..31 under the weights of keys 32..63.
    constexpr int E3 = 16 / NDB;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int c = db & 1;
      if (db + 1 < NDB) pv_load(0, db + 1, ft[c ^ 1]);
      else pv_load(1, 0, ft[c ^ 1]);
      oacc[db] = mfma_bf16(ft[c][0], pf[0][0], oacc[db]);
      oacc[db] = mfma_bf16(ft[c][1], pf[0][1], oacc[db]);
#pragma unroll
      for (int k = 0; k < E3; ++k) elem(1, E3 * db + k);
      step_order<2, VE * E3, 4, 0>();
    }
    // R4: O^T over keys 32..63.
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int c = (db + NDB) & 1;
      if (db + 1 < NDB) pv_load(1, db + 1, ft[c ^ 1]);
      oacc[db] = mfma_bf16(ft[c][0], pf[1][0], oacc[db]);
      oacc[db] = mfma_bf16(ft[c][1], pf[1][1], oacc[db]);
      step_order<2, 0, 4, 0>();
    }

    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this wave's copies of the next tile have landed
    __syncthreads();                     // the next tile is complete; this buffer set is free
    {
      const bf16* Kn = BUF ? Ks0 : Ks1;
      rk3[0] = ld8(Kn + row_off[0]);
      rk3[1] = ld8(Kn + row_off[1]);
    }
  };

  // Key tiles 0 .. 2 qb - 1 lie wholly before this workgroup's queries; tiles 2 qb and
  // 2 qb + 1 cross the diagonal (keys past T, zero-filled, are masked there too).
  const int nfull = min(2 * qb, ntiles);
  int kt = 0;
  for (; kt < nfull; kt += 2) {
    tile(std::integral_constant<int, 0>{}, std::false_type{}, kt);
    tile(std::integral_constant<int, 1>{}, std::false_type{}, kt + 1);
  }
  if (kt < ntiles) {
    tile(std::integral_constant<int, 0>{}, std::true_type{}, kt);
    if (kt + 1 < ntiles) tile(std::integral_constant<int, 1>{}, std::true_type{}, kt + 1);
  }
  // Finalize (flash.py:271-284): Z over both lane halves (+ the sink's weight), stat = 1/Z.
  auto finalize = [&]() __attribute__((always_inline)) {
    float Z = lsum + xor32(lsum);
    if constexpr (FROM_Q) {
      if (p.sink_logit) Z += pow2n<L2N>(rho_fast(p.sink_logit[p.sink_count == 1 ? 0 : head] / p.sink_c), log2n);
    } else {
      if (p.sink) Z += pow2n<L2N>(rho_fast(p.sink[head]), log2n);
    }
    const float inv = 1.0f / Z;
    bf16* O = reinterpret_cast<bf16*>(p.o) + base + (size_t)myq * ld;  // (o_precise: shifted only)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * h;
        bf16x4 ob;
#pragma unroll
        for (int e = 0; e < 4; ++e) ob[e] = f2bf(oacc[db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4*>(O + d0) = ob;
      }
    }
    if (h == 0) p.stat[(size_t)bh * T_ + myq] = inv;
  };
  if constexpr (FROM_Q) {
    // After the output (its accumulators are dead), with every lane of the workgroup.
    if (live) finalize();
    fwd_guard_partials<D>(qf, live, gmk, guard_v_max(gmv), p.guard_part + 3 * ((size_t)bh * nqb + blockIdx.y), gred);
  } else {
    if (!live) return;
    finalize();
  }
}

int attn_fwd_f32_query_block(int B, int H, int T);

template <typename T, int D>
static hipError_t launch_fwd_mode(const AttnFwdParams& p, int mode, hipStream_t st) {
  dim3 grid(p.B * p.H, ceil_div(p.T, FWD_BQ)), block(256);
  // The fallbacks loop over (head, query block) items: one workgroup each when the host chose
  // the variant, a small grid (a multiple of 8) when it is the branch the device guard
  // usually skips.
  const int items = p.B * p.H * ceil_div(p.T, FWD_BQ);
  const int fallback_items = p.flag ? std::min(items, FALLBACK_GRID) : items;
  switch (mode) {
    case MODE_INRANGE: {
      KTimer t("attn_fwd_inrange", st);
      if constexpr (sizeof(T) == 2) {
        if (p.q_s_out) {
          if (p.layout) {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 4, 1, true>), grid, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 0, 1, true>), grid, block, 0, st, p);
          } else {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 4, 0, true>), grid, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 0, 0, true>), grid, block, 0, st, p);
          }
        } else if (p.layout) {
          if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 4, 1, false>), grid, block, 0, st, p);
          else hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 0, 1, false>), grid, block, 0, st, p);
        } else {
          if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 4, 0, false>), grid, block, 0, st, p);
          else hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 0, 0, false>), grid, block, 0, st, p);
        }
      } else if constexpr (D == 64) {
        // Four-way key split (32 queries per workgroup) while two-way workgroups would not
        // fill two rounds of the CUs; two-way (64 queries) above that.
        const int bq = attn_fwd_f32_query_block(p.B, p.H, p.T);
        const dim3 gq(p.B * p.H, ceil_div(p.T, bq));
        if (bq == 32) {
          if (p.q_s_out) {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_f32_split_kernel<1, 4, true>), gq, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_f32_split_kernel<1, 0, true>), gq, block, 0, st, p);
          } else {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_f32_split_kernel<1, 4, false>), gq, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_f32_split_kernel<1, 0, false>), gq, block, 0, st, p);
          }
        } else {
          if (p.q_s_out) {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_f32_split_kernel<2, 4, true>), gq, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_f32_split_kernel<2, 0, true>), gq, block, 0, st, p);
          } else {
            if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_f32_split_kernel<2, 4, false>), gq, block, 0, st, p);
            else hipLaunchKernelGGL((attn_fwd_f32_split_kernel<2, 0, false>), gq, block, 0, st, p);
          }
        }
      } else {
        if (p.log2n == 4) hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE_INRANGE, 4>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE_INRANGE, 0>), grid, block, 0, st, p);
      }
    } break;
    case MODE_CLIPPED: {
      KTimer t("attn_fwd_clipped", st);
      hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE_CLIPPED, 0>), dim3(fallback_items), block, 0, st, p);
    } break;
    case MODE_SHIFTED: {
      KTimer t("attn_fwd_shifted", st);
      hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE_SHIFTED, 0>), dim3(fallback_items), block, 0, st, p);
    } break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Queries per workgroup of the f32 D = 64 forward: 32 (four-way key split) while 64-query
// workgroups would not fill two rounds of the CUs, 64 (two-way) above that.
int attn_fwd_f32_query_block(int B, int H, int T) { return B * H * ceil_div(T, 64) < 512 ? 32 : 64; }

hipError_t launch_attn_fwd(const AttnFwdParams& p, int D, bool bf16_io, int mode, hipStream_t st) {
  if (bf16_io) {
    if (D == 64) return launch_fwd_mode<bf16, 64>(p, mode, st);
    if (D == 128) return launch_fwd_mode<bf16, 128>(p, mode, st);
  } else {
    if (D == 64) return launch_fwd_mode<float, 64>(p, mode, st);
    if (D == 128) return launch_fwd_mode<float, 128>(p, mode, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace alg
