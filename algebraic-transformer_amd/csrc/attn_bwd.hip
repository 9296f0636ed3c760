// Causal algebraic attention backward for gfx950.
//
// Replaces src/algebraic/kernels/flash.py:333-361 (tile gradients), 515-627 (fused and
// resident backward schedules), 630-645 (di), 694-726 (sink VJP) and
// src/algebraic/kernels/head_resident.py:91-119.
//
// bf16 launches, in order:
//   dq    query-stationary: one workgroup = 128 queries of one (b,h). It first forms
//         di = sum_d dO*o for its queries (from the rounded output, flash.py:633; on the
//         shifted fallback from a first pass over the keys, see attn_bwd_dq_kernel) and the
//         per-(b,h,query block) partial sums of mass*di for the sink gradient
//         (flash.py:694-705, 721-723), writes di, then forms S^T and dP^T again and
//         accumulates dQ^T += K^T dS^T in registers, written once. No atomics and no
//         per-key-block dQ partials (unlike flash.py:537-544): f32 atomics run at about a
//         sixth of the store bandwidth on this GPU, so recomputing two products is cheaper.
//   dkdv  key-stationary: dK/dV accumulate in registers while the kernel streams 64-query
//         tiles of Q, dO, stat and di through LDS. Scores are formed as S = Q K^T so a lane
//         owns one key column; P^T and dS^T feed dV += P^T dO and dK += dS^T Q directly as
//         MFMA A operands, with dO/Q fragments transposed by ds_read_b64_tr_b16. In range:
//         attn_bwd_dkdv16_kernel, 16 keys per wave on 16x16x32 MFMAs (4 waves = 64 keys per
//         workgroup, two or three waves per SIMD); clipped and shifted: attn_bwd_bf16_kernel,
//         32 keys per wave on 32x32x16 MFMAs (4 waves = 128 keys). The last workgroup also
//         reduces the dQ kernel's partials into the per-head sink gradient (no separate launch).
// f32 launches: pre (di from the f32 output, sink partials, zeroed dQ accumulator), one
// key-stationary kernel adding dQ to an f32 accumulator with atomics, post (dq from the
// accumulator: round(round(n * acc) * dq_scale), and the sink gradient).
// The fallback variants (shifted, clipped) loop over their work items (grid-stride), so the
// guarded path's launch of the branch the device flag did not select is a small grid that
// exits at once.
#include <type_traits>

#include "attn_common.h"

namespace alg {

constexpr int BWD_BK = 128;  // keys per workgroup
// Queries per streamed tile: 64, or 32 where 64 would not fit in LDS (f32 with D=128).
template <typename T, int D>
constexpr int bwd_bq() { return (sizeof(T) == 4 && D == 128) ? 32 : 64; }
// Rows per pre-kernel workgroup, and per block of the sink-gradient partials: the bf16 dQ
// kernel writes one partial per 128-query workgroup, the f32 pre kernel one per 128 rows.
constexpr int SINK_ROWS = 128;

// ---------------------------------------------------------------------------
// pre (f32): di, dq_acc = 0, sink partials
// ---------------------------------------------------------------------------
// The branch taken (the guard flag or the host's mode) is uniform over the grid; the body is
// straight-line, with every row's loads issued before any is waited for.
template <typename T, int D>
__device__ __forceinline__ void attn_bwd_pre_body(const AttnBwdParams& p, bool shifted) {
  const int bh = blockIdx.x;
  const int head = bh % p.H;
  const int T_ = p.T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.y * SINK_ROWS;
  const size_t hb = head_base(bh, p.H, T_, D, p.layout);
  const int ld = row_stride(p.H, D, p.layout);
  const int n = 1 << p.log2n;
  float b = p.sink ? p.sink[head] : 0.0f;
  if (p.mode == MODE_CLIPPED && !p.flag) b = fminf(b, p.clamp);
  const float rb = rho_exact(b);
  const bool inv_stat = !shifted && (p.mode != MODE_CLIPPED || p.inv_stat);
  const float rbn = ipow_rt(rb, n);
  float part = 0.0f;
  // 8 elements per lane, D/8 lanes per row (vector loads of dO, o; vector zero-fill of dq_acc);
  // each lane loads PRE_U rows before reducing any, to keep more bytes in flight.
  constexpr int PRE_U = 2;
  constexpr int lpr = D / 8, rpw = 64 / lpr;
  const int sub = lane / lpr, li = lane - sub * lpr;
  const int rend = min(row0 + SINK_ROWS, T_);
  for (int r0 = row0 + wave * rpw; r0 < rend; r0 += 4 * rpw * PRE_U) {
    float dov[PRE_U][8], ov[PRE_U][8], stv[PRE_U];
#pragma unroll
    for (int u = 0; u < PRE_U; ++u) {
      const int r = r0 + u * 4 * rpw + sub;
      const int rc = min(r, rend - 1);
      stv[u] = p.stat[(size_t)bh * T_ + rc];
      const size_t xoff = hb + (size_t)rc * ld + li * 8;  // dO and o in the call's layout
      const T* dsrc = reinterpret_cast<const T*>(p.dO) + xoff;
      const T* osrc = reinterpret_cast<const T*>(p.o) + xoff;
      if constexpr (sizeof(T) == 2) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(dsrc);
        const bf16x8 c = *reinterpret_cast<const bf16x8*>(osrc);
#pragma unroll
        for (int j = 0; j < 8; ++j) { dov[u][j] = (float)a[j]; ov[u][j] = (float)c[j]; }
      } else {
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(dsrc), a1 = *reinterpret_cast<const floatx4*>(dsrc + 4);
        const floatx4 c0 = *reinterpret_cast<const floatx4*>(osrc), c1 = *reinterpret_cast<const floatx4*>(osrc + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dov[u][j] = a0[j]; dov[u][4 + j] = a1[j];
          ov[u][j] = c0[j]; ov[u][4 + j] = c1[j];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < PRE_U; ++u) {
      const int r = r0 + u * 4 * rpw + sub;
      const bool ok = r < rend;
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s += dov[u][j] * ov[u][j];
      if (ok) {
        const size_t off = ((size_t)bh * T_ + r) * D + li * 8;  // dq_acc is (B, H, T, D)
        const floatx4 z = {};
        *reinterpret_cast<floatx4*>(p.dq_acc + off) = z;
        *reinterpret_cast<floatx4*>(p.dq_acc + off + 4) = z;
      }
#pragma unroll
      for (int m = 1; m < lpr; m <<= 1) s += __shfl_xor(s, m, 64);
      if (ok && li == 0) {
        p.di[(size_t)bh * T_ + r] = s;
        const float st = stv[u];
        const float mass = inv_stat ? rbn * st : ipow_rt(rb * st, n);
        part += mass * s;
      }
    }
  }
  for (int m = 1; m < 64; m <<= 1) part += __shfl_xor(part, m, 64);
  __shared__ float red[4];
  if (lane == 0) red[wave] = part;
  __syncthreads();
  if (threadIdx.x == 0) p.sink_part[(size_t)bh * gridDim.y + blockIdx.y] = red[0] + red[1] + red[2] + red[3];
}

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_pre_kernel(AttnBwdParams p, int D) {
  bool shifted = p.mode == MODE_SHIFTED;
  if (p.flag) shifted = *p.flag == 0;
  if (D == 128) attn_bwd_pre_body<T, 128>(p, shifted);
  else attn_bwd_pre_body<T, 64>(p, shifted);
}

// ---------------------------------------------------------------------------
// main
// ---------------------------------------------------------------------------
// Registers <-> LDS staging of an R-row tile of a (T, D) matrix (16-byte chunks; rows >= T
// read as zero).
template <typename T, int D, int R>
struct RowTile {
  static constexpr int CH = 16 / sizeof(T);
  static constexpr int CPR = D / CH;
  static constexpr int PER = (R * CPR + 255) / 256;  // chunks per thread
  // Rows past T load the last row instead (clamped, unconditional loads that nothing waits
  // for until the tile is stored). The query tiles' rows past T carry stat = 0, so their
  // weights and score gradients are exactly zero and the finite stand-in values add nothing.
  static __device__ __forceinline__ void load(uint4 (&r)[PER], const T* src, int r0, int T_, int ld) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = min(idx / CPR, R - 1), col = (idx - (idx / CPR) * CPR) * CH;
      r[c] = *reinterpret_cast<const uint4*>(src + (size_t)min(r0 + row, T_ - 1) * ld + col);
    }
  }
  // bf16 tiles are unpadded and swizzled (swz_at); f32 tiles are row-major with `pitch`.
  static __device__ __forceinline__ void store(T* dst, int pitch, const uint4 (&r)[PER]) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx / CPR, col = (idx - row * CPR) * CH;
      if (row < R) {
        if constexpr (sizeof(T) == 2) *reinterpret_cast<uint4*>(dst + swz_at<CPR>(row, col)) = r[c];
        else *reinterpret_cast<uint4*>(dst + row * pitch + col) = r[c];
      }
    }
  }
};

template <typename T, int D, int MODE, int L2N>
__global__ __launch_bounds__(256, 1) void attn_bwd_kernel(AttnBwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr bool BF = sizeof(T) == 2;
  constexpr int BWD_BQ = bwd_bq<T, D>();
  // f32 tiles: padded row-major; bf16 tiles: unpadded, swizzled (CPR / SCPR chunks per row).
  constexpr int PITCH = D + F32_PAD;
  constexpr int SPITCH = BWD_BQ + F32_PAD;
  constexpr int CPR = D / 8, SCPR = BWD_BQ / 8;
  constexpr int NDB = D / 32;
  __shared__ __attribute__((aligned(16))) T Ks[BF ? BWD_BK * D : BWD_BK * PITCH];
  __shared__ __attribute__((aligned(16))) T Qs[BF ? BWD_BQ * D : BWD_BQ * PITCH];
  __shared__ __attribute__((aligned(16))) T dOs[BF ? BWD_BQ * D : BWD_BQ * PITCH];
  __shared__ __attribute__((aligned(16))) T dSs[BF ? BWD_BK * BWD_BQ : BWD_BK * SPITCH];
  __shared__ __attribute__((aligned(16))) float st_s[BWD_BQ];
  __shared__ __attribute__((aligned(16))) float di_s[BWD_BQ];

  if (p.flag) {
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  // One 128-key block of one head. The in-range kernel takes one per workgroup from its 2-D
  // grid; the fallbacks loop over them (grid-stride), key block 0 (the most causal work) first.
  auto run = [&](int bh, int kblk) __attribute__((always_inline)) {
  const int k0 = kblk * BWD_BK;
  const size_t base = (size_t)bh * T_ * D;  // internal (B, H, T, D) buffers (dq_acc)
  const size_t hb = head_base(bh, p.H, T_, D, p.layout);
  const int ld = row_stride(p.H, D, p.layout);
  const T* Q = reinterpret_cast<const T*>(p.q) + hb;
  const T* K = reinterpret_cast<const T*>(p.k) + hb;
  const T* V = reinterpret_cast<const T*>(p.v) + hb;
  const T* dO = reinterpret_cast<const T*>(p.dO) + hb;
  const float* stat = p.stat + (size_t)bh * T_;
  const float* di = p.di + (size_t)bh * T_;
  float* dq_acc = p.dq_acc + base;
  const int wk0 = k0 + wave * 32;    // this wave's first key
  const int mykey = wk0 + l32;
  const int log2n = p.log2n;

  {
    typedef RowTile<T, D, BWD_BK> KT;
    uint4 kr[KT::PER];
    KT::load(kr, K, k0, T_, ld);
    KT::store(Ks, PITCH, kr);
  }

  // K and V fragments as B operands of S = Q K^T and dP = dO V^T.
  constexpr int NF = BF ? D / 16 : D / 8;
  typedef typename std::conditional<BF, bf16x8, floatx4>::type Frag;
  Frag kf[NF], vf[NF];
#pragma unroll
  for (int s = 0; s < NF; ++s) {
    if constexpr (BF) {
      bf16x8 z = {};
      const size_t o = (size_t)mykey * ld + 16 * s + 8 * h;
      kf[s] = mykey < T_ ? ld8(reinterpret_cast<const bf16*>(K) + o) : z;
      vf[s] = mykey < T_ ? ld8(reinterpret_cast<const bf16*>(V) + o) : z;
    } else {
      floatx4 z = {};
      const size_t o = (size_t)mykey * ld + 8 * s + 4 * h;
      kf[s] = mykey < T_ ? *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(K) + o) : z;
      vf[s] = mykey < T_ ? *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(V) + o) : z;
    }
  }
  floatx16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) { dk[db] = floatx16{}; dv[db] = floatx16{}; }

  const int nq = ceil_div(T_, BWD_BQ);
  const int qstart = k0 / BWD_BQ;
  // Q/dO/stat/di tiles are prefetched into registers one iteration ahead and written to
  // LDS between the dS barrier and the dQ phase (which reads only dS and K).
  typedef RowTile<T, D, BWD_BQ> QT;
  uint4 qr[QT::PER], dr[QT::PER];
  float str = 0.0f, dir = 0.0f;
  auto prefetch = [&](int qbase) {
    QT::load(qr, Q, qbase, T_, ld);
    QT::load(dr, dO, qbase, T_, ld);
    if (threadIdx.x < BWD_BQ) {  // raw loads; rows past T are zeroed when committed
      const int q = min(qbase + (int)threadIdx.x, T_ - 1);
      str = stat[q];
      dir = di[q];
    }
  };
  auto commit = [&](int qbase) {
    QT::store(Qs, PITCH, qr);
    QT::store(dOs, PITCH, dr);
    if (threadIdx.x < BWD_BQ) {
      const bool live = qbase + (int)threadIdx.x < T_;  // stat = 0 removes rows past T
      st_s[threadIdx.x] = live ? str : 0.0f;
      di_s[threadIdx.x] = live ? dir : 0.0f;
    }
  };
  prefetch(qstart * BWD_BQ);
  commit(qstart * BWD_BQ);
  __syncthreads();
  for (int qt = qstart; qt < nq; ++qt) {
    const int qbase = qt * BWD_BQ;
    const bool more = qt + 1 < nq;
    if (more) prefetch(qbase + BWD_BQ);
    // One 32-query block against this wave's 32 keys: S, dP, P, dS, dV += P^T dO,
    // dK += dS^T Q, dS staged in LDS for the dQ phase.
    auto sub_block = [&](int sub, bool diag) {
      const int sq0 = qbase + sub * 32;
      T* dsrow = dSs + (wave * 32 + l32) * SPITCH + sub * 32;
        const T* qrow = Qs + (sub * 32 + l32) * PITCH;
        const T* dorow = dOs + (sub * 32 + l32) * PITCH;
        floatx16 s = {}, dp = {};
  #pragma unroll
        for (int st = 0; st < NF; ++st) {
          if constexpr (BF) {
            const int at = swz_at<CPR>(sub * 32 + l32, 16 * st + 8 * h);
            bf16x8 qa = *reinterpret_cast<const bf16x8*>(Qs + at);
            s = mfma_bf16(qa, kf[st], s);
            bf16x8 da = *reinterpret_cast<const bf16x8*>(dOs + at);
            dp = mfma_bf16(da, vf[st], dp);
          } else {
            floatx4 qa = *reinterpret_cast<const floatx4*>(qrow + 8 * st + 4 * h);
            floatx4 da = *reinterpret_cast<const floatx4*>(dorow + 8 * st + 4 * h);
  #pragma unroll
            for (int u = 0; u < 4; ++u) {
              s = mfma_f32(qa[u], kf[st][u], s);
              dp = mfma_f32(da[u], vf[st][u], dp);
            }
          }
        }
        float pv[16], dsv[16];
  #pragma unroll
        for (int g = 0; g < 4; ++g) {
          const floatx4 stq = *reinterpret_cast<const floatx4*>(st_s + sub * 32 + 8 * g + 4 * h);
          const floatx4 diq = *reinterpret_cast<const floatx4*>(di_s + sub * 32 + 8 * g + 4 * h);
  #pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * g + e;
            float x = s[i];
            float r, pw;
            if constexpr (MODE == MODE_INRANGE) {
              pw = pow2n<L2N>(rho_fast(x, r), log2n) * stq[e];
            } else if constexpr (MODE == MODE_CLIPPED) {
              x = fminf(x, p.clamp);
              float t = rho_fast(x, r);
              if (p.inv_stat) {
                for (int k2 = 0; k2 < log2n; ++k2) t = t * t;
                pw = t * stq[e];
              } else {
                t = t * stq[e];
                for (int k2 = 0; k2 < log2n; ++k2) t = t * t;
                pw = t;
              }
            } else {
              const int q = sq0 + 8 * g + 4 * h + e;
              if (diag && mykey > q) x = 0.0f;
              const float t = p.fast_rho ? rho_fast(x, r) : rho_exact(x, r);
              pw = pow2n<L2N>(t * stq[e], log2n);
            }
            float dsx = pw * (dp[i] - diq[e]) * r;
            if constexpr (MODE == MODE_CLIPPED) dsx = s[i] < p.clamp ? dsx : 0.0f;
            if (diag) {
              const int q = sq0 + 8 * g + 4 * h + e;
              if (mykey > q) { pw = 0.0f; dsx = 0.0f; }
            }
            pv[i] = pw;
            dsv[i] = dsx;
          }
        }
        if constexpr (BF) {
          bf16x8 pa0, pa1, da0, da1;
  #pragma unroll
          for (int j = 0; j < 8; ++j) {
            pa0[j] = f2bf(pv[j]); pa1[j] = f2bf(pv[8 + j]);
            da0[j] = f2bf(dsv[j]); da1[j] = f2bf(dsv[8 + j]);
          }
          const bf16* qt_ = reinterpret_cast<const bf16*>(Qs);
          const bf16* dot_ = reinterpret_cast<const bf16*>(dOs);
  #pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const int r0 = sub * 32 + 4 * h;
            bf16x8 ob0 = swz_tr_frag<CPR>(dot_, r0, r0 + 8, db * 32, lane);
            bf16x8 ob1 = swz_tr_frag<CPR>(dot_, r0 + 16, r0 + 24, db * 32, lane);
            dv[db] = mfma_bf16(pa0, ob0, dv[db]);
            dv[db] = mfma_bf16(pa1, ob1, dv[db]);
            bf16x8 qb0 = swz_tr_frag<CPR>(qt_, r0, r0 + 8, db * 32, lane);
            bf16x8 qb1 = swz_tr_frag<CPR>(qt_, r0 + 16, r0 + 24, db * 32, lane);
            dk[db] = mfma_bf16(da0, qb0, dk[db]);
            dk[db] = mfma_bf16(da1, qb1, dk[db]);
          }
          // Stage dS (rounded, as the dq/dk operands are) in LDS as [key][query].
  #pragma unroll
          for (int g = 0; g < 4; ++g) {
            bf16x4 v4;
  #pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = f2bf(dsv[4 * g + e]);
            *reinterpret_cast<bf16x4*>(dSs + swz_at<SCPR>(wave * 32 + l32, sub * 32 + 8 * g + 4 * h)) = v4;
          }
        } else {
          const float* qt_ = reinterpret_cast<const float*>(Qs);
          const float* dot_ = reinterpret_cast<const float*>(dOs);
  #pragma unroll
          for (int db = 0; db < NDB; ++db) {
  #pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int qr = sub * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
              dv[db] = mfma_f32(pv[i], dot_[qr * PITCH + db * 32 + l32], dv[db]);
              dk[db] = mfma_f32(dsv[i], qt_[qr * PITCH + db * 32 + l32], dk[db]);
            }
          }
  #pragma unroll
          for (int g = 0; g < 4; ++g) {
            floatx4 v4;
  #pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = dsv[4 * g + e];
            *reinterpret_cast<floatx4*>(dsrow + 8 * g + 4 * h) = v4;
          }
        }
    };
    if (wk0 < T_ && qbase >= wk0 + 31) {  // every query follows every key: no masking
#pragma unroll
      for (int sub = 0; sub < BWD_BQ / 32; ++sub) sub_block(sub, false);
    } else {
#pragma unroll
      for (int sub = 0; sub < BWD_BQ / 32; ++sub) {
        const int sq0 = qbase + sub * 32;
        if (sq0 + 31 < wk0 || wk0 >= T_) {  // all queries precede all keys of this wave
          T* dsrow = dSs + (wave * 32 + l32) * SPITCH + sub * 32;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            if constexpr (BF) {
              bf16x4 z = {};
              *reinterpret_cast<bf16x4*>(dSs + swz_at<SCPR>(wave * 32 + l32, sub * 32 + 8 * g + 4 * h)) = z;
            }
            else { floatx4 z = {}; *reinterpret_cast<floatx4*>(dsrow + 8 * g + 4 * h) = z; }
          }
        } else {
          sub_block(sub, wk0 + 31 > sq0);
        }
      }
    }
    __syncthreads();
    if (more) commit(qbase + BWD_BQ);
    // dQ tile = dS K over this workgroup's keys; each wave takes 32 queries x DBW blocks.
    {
      constexpr int NQH = BWD_BQ / 32;         // 32-query slices of the tile
      constexpr int WPH = 4 / NQH;             // waves per slice
      constexpr int DBW = NDB / WPH;           // 32-wide d blocks per wave
      static_assert(DBW >= 1, "tile shape");
      const int qs = wave / WPH;
      const int db0 = (wave % WPH) * DBW;
      floatx16 dqa[DBW];
#pragma unroll
      for (int j = 0; j < DBW; ++j) dqa[j] = floatx16{};
      if constexpr (BF) {
        const bf16* ds_ = reinterpret_cast<const bf16*>(dSs);
        const bf16* k_ = reinterpret_cast<const bf16*>(Ks);
        // DBW >= 2 independent accumulator chains keep the MFMA pipe busy.
#pragma unroll
        for (int ks = 0; ks < BWD_BK / 16; ++ks) {
          const int klo = ks * 16 + 8 * h;
          bf16x8 a0 = swz_tr_frag<SCPR>(ds_, klo, klo + 4, qs * 32, lane);
#pragma unroll
          for (int j = 0; j < DBW; ++j) {
            bf16x8 b0 = swz_tr_frag<CPR>(k_, klo, klo + 4, (db0 + j) * 32, lane);
            dqa[j] = mfma_bf16(a0, b0, dqa[j]);
          }
        }
      } else {
        const float* ds_ = reinterpret_cast<const float*>(dSs);
        const float* k_ = reinterpret_cast<const float*>(Ks);
#pragma unroll 8
        for (int ks = 0; ks < BWD_BK / 2; ++ks) {
          const int key = 2 * ks + h;
          const float a = ds_[key * SPITCH + qs * 32 + l32];
#pragma unroll
          for (int j = 0; j < DBW; ++j) dqa[j] = mfma_f32(a, k_[key * PITCH + (db0 + j) * 32 + l32], dqa[j]);
        }
      }
      {
        // Buffer atomics over this slice's rows: the row offset is part of the range-checked
        // VGPR offset, so rows at or past T (beyond num_records) are dropped by the hardware;
        // the d-block offset is the scalar offset.
        const int rowbase = qbase + qs * 32;
        const int live_rows = max(0, T_ - rowbase);
        const __amdgpu_buffer_rsrc_t dqr = __builtin_amdgcn_make_buffer_rsrc(
            dq_acc + (size_t)rowbase * D, (short)0, live_rows * D * 4, BUF_RSRC_WORD3);
        const int lane_off = (4 * h * D + l32) * 4;
#pragma unroll
        for (int j = 0; j < DBW; ++j) {
#pragma unroll
          for (int i = 0; i < 16; ++i)
            __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(dqa[j][i], dqr,
                                                            lane_off + (8 * (i >> 2) + (i & 3)) * D * 4,
                                                            (db0 + j) * 128, 0);
        }
      }
    }
    __syncthreads();
  }

  // dK = n * acc, dV = acc (flash.py:591-597), rounded to the input dtype.
  const float slope = (float)(1 << log2n);
  T* DK = reinterpret_cast<T*>(p.dk) + hb;
  T* DV = reinterpret_cast<T*>(p.dv) + hb;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = wk0 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (key < T_) {
        const size_t o = (size_t)key * ld + db * 32 + l32;
        DK[o] = (T)(dk[db][i] * slope);
        DV[o] = (T)(dv[db][i]);
      }
    }
  }
  };
  if constexpr (MODE == MODE_INRANGE) {
    run(blockIdx.x, blockIdx.y);
  } else {
    const int nbh = p.B * p.H, total = nbh * ceil_div(T_, BWD_BK);
    for (int L = blockIdx.x; L < total; L += gridDim.x) {
      run(L % nbh, L / nbh);
      __syncthreads();  // the next block's K tile overwrites LDS
    }
  }
}

// ---------------------------------------------------------------------------
// main, bf16: query tiles staged by direct global -> LDS copies
// ---------------------------------------------------------------------------
// Weight p and score gradient dS for one score (flash.py:333-361); `masked` zeroes both
// (keys after the query, or query rows at or past T).
template <int MODE, int L2N>
__device__ __forceinline__ void bwd_elem(float x, float dp, float stq, float diq, bool masked,
                                         const AttnBwdParams& p, int log2n, float& pw, float& dsx) {
  const float s0 = x;
  float r;
  if constexpr (MODE == MODE_INRANGE) {
    pw = pow2n<L2N>(rho_fast(x, r), log2n) * stq;
  } else if constexpr (MODE == MODE_CLIPPED) {
    x = fminf(x, p.clamp);
    float t = rho_fast(x, r);
    if (p.inv_stat) {
      pw = pow2n<0>(t, log2n) * stq;
    } else {
      pw = pow2n<0>(t * stq, log2n);
    }
  } else {
    if (masked) x = 0.0f;
    const float t = p.fast_rho ? rho_fast(x, r) : rho_exact(x, r);
    pw = pow2n<L2N>(t * stq, log2n);
  }
  dsx = pw * (dp - diq) * r;
  if constexpr (MODE == MODE_CLIPPED) dsx = s0 < p.clamp ? dsx : 0.0f;
  if (masked) {
    pw = 0.0f;
    dsx = 0.0f;
  }
}

// Per-head sink gradient (flash.py:694-705, 721-723) from the partial sums of mass * di that
// the dQ kernel (bf16) or the pre kernel (f32) wrote, in one workgroup: one wave per head,
// lane l adds partials l, l + 64, ... of the head's B * nblk, then a butterfly over the wave
// (a fixed order for a given shape). Run by the bf16 dK/dV kernel's last workgroup (after the
// dQ kernel that wrote the partials) and by the f32 post kernel.
__device__ __forceinline__ void attn_sink_grad(const AttnBwdParams& p, int nblk) {
  if (!p.dbeta) return;
  bool shifted = p.mode == MODE_SHIFTED;
  if (p.flag) shifted = *p.flag == 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
  const int cnt = p.B * nblk;
  for (int hh = wave; hh < p.H; hh += nwave) {
    float s = 0.0f;
    if (p.sink)
      for (int i = lane; i < cnt; i += 64) {
        const int b = i / nblk, k = i - b * nblk;
        s += p.sink_part[(size_t)(b * p.H + hh) * nblk + k];
      }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    if (lane != 0) continue;
    if (!p.sink) { p.dbeta[hh] = 0.0f; continue; }
    float beta = p.sink[hh];
    const bool clipped = !shifted && p.mode == MODE_CLIPPED && !p.flag;
    float bb = clipped ? fminf(beta, p.clamp) : beta;
    float r;
    rho_exact(bb, r);
    float sl = (float)(1 << p.log2n) * r;
    if (clipped && !(beta < p.clamp)) sl = 0.0f;  // flash.py:703-704
    p.dbeta[hh] = -s * sl;
  }
}

constexpr int BF_BQ = 64;  // queries per streamed tile (bf16 kernel)
constexpr int BWD_XCDS = 8;    // workgroup i runs on XCD i % 8
constexpr int BWD_GROUP = 4;   // heads whose key blocks one XCD interleaves

// Work item L -> (head, key block) of the bf16 dK/dV kernel (1-D grid; L is the workgroup id,
// or for the grid-stride fallbacks the workgroup id plus multiples of a grid size that is a
// multiple of 8, so L % 8 is still the XCD). Each XCD works through its own share of the heads
// in groups of BWD_GROUP, key block by key block within a group (heaviest causal blocks
// first), so the query tiles of only a few heads are live in that XCD's L2 at a time. Head
// counts that do not split evenly over the XCDs use the plain key-block-major order.
__device__ __forceinline__ void bwd_block_coords(int L, int nbh, int nkb, int& bh, int& kblk) {
  if (nbh % (BWD_XCDS * BWD_GROUP) == 0) {
    const int xcd = L % BWD_XCDS, idx = L / BWD_XCDS;
    const int g = idx / (BWD_GROUP * nkb), r = idx - g * BWD_GROUP * nkb;
    kblk = r / BWD_GROUP;
    bh = xcd * (nbh / BWD_XCDS) + g * BWD_GROUP + (r - kblk * BWD_GROUP);
  } else {
    bh = L % nbh;
    kblk = L / nbh;
  }
}

// Per-row statistics of a 64-query tile (stat by wave 0, di by wave 1); rows at or past T
// land as zeros.
__device__ __forceinline__ void bwd_stat_dma(float* lst, float* ldi, __amdgpu_buffer_rsrc_t rst,
                                             __amdgpu_buffer_rsrc_t rdi, int qbase, int wave, int lane) {
  if (wave == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(rst, LDS_PTR(void, lst), 4, (qbase + lane) * 4, 0, 0, 0);
  if (wave == 1) __builtin_amdgcn_raw_ptr_buffer_load_lds(rdi, LDS_PTR(void, ldi), 4, (qbase + lane) * 4, 0, 0, 0);
}

// VALU instructions per score element (scheduling hint).
template <int MODE>
constexpr int bwd_valu_per_elem() { return MODE == MODE_INRANGE ? 14 : 20; }
// Waves per SIMD the dK/dV kernel is built for: at D = 64 its dK/dV accumulators, K/V
// fragments and one tile's S/dP fit in 256 registers, so two waves share a SIMD (VGPR-held
// accumulators); at D = 128 they take about 420 and the kernel runs one wave per SIMD.
template <int D>
constexpr int bwd_bf16_waves_per_simd() { return D == 64 ? 2 : 1; }

// dK/dV kernel for bf16 inputs (the clipped and shifted variants; the in-range path runs
// attn_bwd_dkdv16_kernel below): 128 keys per workgroup, 32 per wave (lane = key), dK/dV
// accumulated in registers over the 64-query tiles of the causal range. dQ is formed by
// attn_bwd_dq_kernel, so this kernel stages nothing for it. Arranged for one wave per SIMD
// as a software pipeline of fixed steps; each step's MFMAs use LDS fragments read two steps
// earlier, so no MFMA waits on a just-issued read:
//   R1  S, dP of query block 0 (MFMA), the copy of the next tile spread over its steps
//   R2  S, dP of block 1 (MFMA) | P, dS of block 0, elements 0..7 (VALU)
//   C   16 steps of dV += P^T dO, dK += dS^T Q, one 16-query quarter and one d block each:
//       quarter 0 under elements 8..15 of block 0, quarter 1 under 0..7 of block 1, quarter
//       2 under 8..15 of block 1, quarter 3 alone (every quarter's weights are ready by then)
//   barrier (the next tile's copy has landed)
// Query tiles ping-pong between two LDS buffer sets (distinct __shared__ objects). The causal
// mask is evaluated only on the two tiles that cross the diagonal; every LDS access is a
// per-lane swizzled offset computed once plus an immediate.
template <int D, int MODE, int L2N, int LAYOUT>
__global__ __launch_bounds__(256, bwd_bf16_waves_per_simd<D>()) void attn_bwd_bf16_kernel(AttnBwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr int BQ = BF_BQ, CPR = D / 8, NDB = D / 32, NF = D / 16;
  constexpr int PW = 64 * CPR / 64 / 4;  // copy instruction pairs per wave and tile
  __shared__ __attribute__((aligned(16))) bf16 Qs0[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 Qs1[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dOs0[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dOs1[BQ * D];
  __shared__ __attribute__((aligned(16))) float st0[BQ];
  __shared__ __attribute__((aligned(16))) float st1[BQ];
  __shared__ __attribute__((aligned(16))) float di0[BQ];
  __shared__ __attribute__((aligned(16))) float di1[BQ];

  if (p.flag) {
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  const int nbh = p.B * p.H, nkb = ceil_div(T_, BWD_BK);
  auto run = [&](int L) __attribute__((always_inline)) {
  int bh, kblk;
  bwd_block_coords(L, nbh, nkb, bh, kblk);
  const int k0 = kblk * BWD_BK;
  const size_t base = head_base(bh, p.H, T_, D, LAYOUT);
  const int ld = LAYOUT ? p.H * D : D;  // elements between positions
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + base;
  const bf16* K = reinterpret_cast<const bf16*>(p.k) + base;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + base;
  const bf16* dO = reinterpret_cast<const bf16*>(p.dO) + base;
  const int nbytes = head_bytes(T_, ld, D, 2);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)Q, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rdo = __builtin_amdgcn_make_buffer_rsrc((void*)dO, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rst =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.stat + (size_t)bh * T_), (short)0, T_ * 4, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rdi =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.di + (size_t)bh * T_), (short)0, T_ * 4, BUF_RSRC_WORD3);
  const int wk0 = k0 + wave * 32;  // this wave's first key
  const int mykey = wk0 + l32;
  const int log2n = p.log2n;
  const int nq = ceil_div(T_, BQ);
  const int qstart = k0 / BQ;

  tile_dma2<D>(Qs0, dOs0, rq, rdo, qstart * BQ, wave, lane, ld);
  bwd_stat_dma(st0, di0, rst, rdi, qstart * BQ, wave, lane);
  // K and V fragments of this wave's keys: B operands of S = Q K^T and dP = dO V^T. Keys
  // past T are zero and always masked.
  bf16x8 kf[NF], vf[NF];
#pragma unroll
  for (int s = 0; s < NF; ++s) {
    const bf16x8 z = {};
    const size_t o = (size_t)mykey * ld + 16 * s + 8 * h;
    kf[s] = mykey < T_ ? ld8(K + o) : z;
    vf[s] = mykey < T_ ? ld8(V + o) : z;
  }
  floatx16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = floatx16{};
    dv[db] = floatx16{};
  }

  // Per-lane swizzled offsets: the swizzle repeats every 16 rows, so every access below is
  // one of these plus a multiple of 16 rows (an immediate offset).
  const int trow = (lane & 15) >> 2;  // row within a transposed read's 4-row group
  int row_off[NF];                    // row fragments of Q / dO: row l32, k chunk 2 st + h
#pragma unroll
  for (int st = 0; st < NF; ++st) row_off[st] = swz_at<CPR>(l32, 16 * st + 8 * h);
  int tq_lo[NDB], tq_hi[NDB];  // transposed Q / dO fragments: rows 4h + (0..3), 4h + 8 + (0..3)
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tq_lo[db] = swz_at<CPR>(4 * h + trow, tr_col(db * 32, lane));
    tq_hi[db] = swz_at<CPR>(4 * h + 8 + trow, tr_col(db * 32, lane));
  }

  bf16x8 rq4[4], ro4[4];  // row fragments of Q / dO, three steps ahead (R1, R2)
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    rq4[g] = ld8(Qs0 + row_off[g]);
    ro4[g] = ld8(dOs0 + row_off[g]);
  }
  constexpr int VE = bwd_valu_per_elem<MODE>();

  // One query tile. BUF selects the LDS buffer set, MASKED the tiles that cross the diagonal.
  auto tile = [&](auto bufc, auto maskc, int qt) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool MASKED = decltype(maskc)::value;
    const bf16* Qs = BUF ? Qs1 : Qs0;
    const bf16* dOs = BUF ? dOs1 : dOs0;
    const float* sts = BUF ? st1 : st0;
    const float* dis = BUF ? di1 : di0;
    const int qbase = qt * BQ;

    floatx16 s[2], dp[2];
    bf16x8 pa[2][2], da[2][2];
    floatx4 sq[2][2], dq4[2][2];  // stat and di of a quarter's queries (slot = quarter & 1)
    float pv[16], dsv[16];

    // R1/R2 step g = NF * sub + st: MFMAs on the fragments of step g, reads for step g + 3.
    auto sdp_step = [&](int g) {
      const int sub = g / NF, st = g % NF;
      const int gn = g + 3;
      if (gn < 2 * NF) {
        rq4[gn % 4] = ld8(Qs + (gn / NF) * 32 * D + row_off[gn % NF]);
        ro4[gn % 4] = ld8(dOs + (gn / NF) * 32 * D + row_off[gn % NF]);
      }
      s[sub] = mfma_bf16(rq4[g % 4], kf[st], s[sub]);
      dp[sub] = mfma_bf16(ro4[g % 4], vf[st], dp[sub]);
    };
    // Stat and di of the lane's 8 queries of quarter k (queries 16 k ..; elements 8 (k & 1)
    // .. + 7 of block k >> 1), loaded one phase before they are used.
    auto load_stats = [&](int k) {
#pragma unroll
      for (int gl = 0; gl < 2; ++gl) {
        sq[k & 1][gl] = *reinterpret_cast<const floatx4*>(sts + 16 * k + 8 * gl + 4 * h);
        dq4[k & 1][gl] = *reinterpret_cast<const floatx4*>(dis + 16 * k + 8 * gl + 4 * h);
      }
    };
    // Weight P and score gradient dS of element i of block sub, rounded to bf16 as the
    // gradient products use them.
    auto elem = [&](int sub, int i) {
      const int g = i >> 2, e = i & 3;
      const bool masked = MASKED && mykey > qbase + sub * 32 + 8 * g + 4 * h + e;
      const int k = 2 * sub + (i >> 3);
      bwd_elem<MODE, L2N>(s[sub][i], dp[sub][i], sq[k & 1][g & 1][e], dq4[k & 1][g & 1][e], masked, p, log2n, pv[i],
                          dsv[i]);
      if (i & 1) {
        pa[sub][i >> 3][(i & 7) - 1] = f2bf(pv[i - 1]);
        pa[sub][i >> 3][i & 7] = f2bf(pv[i]);
        da[sub][i >> 3][(i & 7) - 1] = f2bf(dsv[i - 1]);
        da[sub][i >> 3][i & 7] = f2bf(dsv[i]);
      }
    };
    // C step c = NDB * qq + db: dV += P^T dO and dK += dS^T Q over the tile's queries
    // 16 qq .. 16 qq + 15 and d block db; its fragments sit in ring slot c % 4.
    constexpr int NC = 4 * NDB;
    bf16x8 fc[4][2];
    auto c_load = [&](int c) {
      const int qq = c / NDB, db = c % NDB;
      fc[c % 4][0] = tr_frag_at(dOs + qq * 16 * D, tq_lo[db], tq_hi[db]);
      fc[c % 4][1] = tr_frag_at(Qs + qq * 16 * D, tq_lo[db], tq_hi[db]);
    };
    auto c_mma = [&](int c) {
      const int qq = c / NDB, db = c % NDB;
      dv[db] = mfma_bf16(pa[qq >> 1][qq & 1], fc[c % 4][0], dv[db]);
      dk[db] = mfma_bf16(da[qq >> 1][qq & 1], fc[c % 4][1], dk[db]);
    };

    // R1: S and dP of block 0; the copy of the next tile, one instruction pair per step. It
    // is issued unconditionally: past the last tile every row lies beyond the descriptors'
    // ranges (no memory is read, zeros land in the unused buffer set), and it has completed
    // by this tile's vmcnt(0).
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      s[sb] = floatx16{};
      dp[sb] = floatx16{};
    }
    load_stats(0);
#pragma unroll
    for (int g = 0; g < NF; ++g) {
      sdp_step(g);
      if (g < PW) {
        if constexpr (BUF) tile_dma2_part<D>(Qs0, dOs0, rq, rdo, qbase + BQ, wave, lane, g, ld);
        else tile_dma2_part<D>(Qs1, dOs1, rq, rdo, qbase + BQ, wave, lane, g, ld);
      }
      if (g == PW) {
        if constexpr (BUF) bwd_stat_dma(st0, di0, rst, rdi, qbase + BQ, wave, lane);
        else bwd_stat_dma(st1, di1, rst, rdi, qbase + BQ, wave, lane);
      }
      if (g == 0) step_order<2, 0, 4 + 4, 0>();
      else step_order<2, 0, 4, 0>();
    }
    // R2: S and dP of block 1 under elements 0..7 of block 0.
    constexpr int E2 = 8 / NF > 0 ? 8 / NF : 1;
    load_stats(1);
#pragma unroll
    for (int g = NF; g < 2 * NF; ++g) {
      sdp_step(g);
      const int st = g - NF;
#pragma unroll
      for (int k = 0; k < E2; ++k)
        if (E2 * st + k < 8) elem(0, E2 * st + k);
      if (g == 2 * NF - 3) c_load(0);
      if (g == 2 * NF - 2) c_load(1);
      if (g == 2 * NF - 1) c_load(2);
      if (g == NF) step_order<2, VE * E2, 4 + 4 + 4, 0>();
      else step_order<2, VE * E2, 4 + 4, 0>();
    }
    // C steps: quarter 0 under elements 8..15 of block 0, quarter 1 under 0..7 of block 1,
    // quarter 2 under 8..15 of block 1, quarter 3 alone. Quarters 0 and 1 read the stats of
    // the quarters weighed after them.
    constexpr int EC = 8 / NDB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c == 0) load_stats(2);
      if (c == NDB) load_stats(3);
      if (c + 3 < NC) c_load(c + 3);
      c_mma(c);
      const int qq = c / NDB, db = c % NDB;
      if (qq < 3) {
#pragma unroll
        for (int k = 0; k < EC; ++k) {
          const int idx = EC * db + k;  // quarter 0: 8..15 of block 0; 1: 0..7 of block 1; 2: 8..15
          elem(qq == 0 ? 0 : 1, qq == 1 ? idx : 8 + idx);
        }
        if (c == 0 || c == NDB) step_order<2, VE * EC, 4 + 4, 0>();
        else step_order<2, VE * EC, 4, 0>();
      } else {
        step_order<2, 0, 4, 0>();
      }
    }

    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this wave's copies of the next tile have landed
    __syncthreads();                     // the next buffer set is complete; this one is free
    {  // first fragments of the next tile
      const bf16* Qn = BUF ? Qs0 : Qs1;
      const bf16* dOn = BUF ? dOs0 : dOs1;
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        rq4[g] = ld8(Qn + row_off[g]);
        ro4[g] = ld8(dOn + row_off[g]);
      }
    }
  };

  // Tiles qstart and qstart + 1 cross the diagonal; the loop's back edge follows a buffer-1
  // tile only.
  int qt = qstart;
  tile(std::integral_constant<int, 0>{}, std::true_type{}, qt);
  if (qt + 1 < nq) {
    tile(std::integral_constant<int, 1>{}, std::true_type{}, qt + 1);
    qt += 2;
    while (qt < nq) {
      tile(std::integral_constant<int, 0>{}, std::false_type{}, qt);
      if (qt + 1 >= nq) break;
      tile(std::integral_constant<int, 1>{}, std::false_type{}, qt + 1);
      qt += 2;
    }
  }

  // dK = n * acc, dV = acc (flash.py:591-597), rounded to bf16.
  const float slope = (float)(1 << log2n);
  bf16* DK = reinterpret_cast<bf16*>(p.dk) + base;
  bf16* DV = reinterpret_cast<bf16*>(p.dv) + base;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = wk0 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (key < T_) {
        const size_t o = (size_t)key * ld + db * 32 + l32;
        DK[o] = f2bf(dk[db][i] * slope);
        DV[o] = f2bf(dv[db][i]);
      }
    }
  }
  };
  if constexpr (MODE == MODE_INRANGE) {
    run(blockIdx.x);
  } else {
    for (int L = blockIdx.x; L < nbh * nkb; L += gridDim.x) {
      run(L);
      __syncthreads();  // the next item's first copies overwrite both LDS buffer sets
    }
  }
  // The last workgroup (the lightest causal key block) also forms the sink gradient.
  if (blockIdx.x == gridDim.x - 1) attn_sink_grad(p, ceil_div(T_, SINK_ROWS));
}

// LDS layout of the 16-key dK/dV kernel's Q / dO tiles (64 rows of D bf16) and the lane
// mapping of its fragments, chosen with the bank-conflict counter so that both kinds of
// fragment read are conflict-free (each alternative listed cost 2-4 extra cycles per read):
//   D = 128: chunk c of row r at c ^ (4(r&3) + ((r>>2)&3)) (the attention kernels' swizzle);
//            MFMA row m of a 16-query block is tile row sigma(m) (0..7 -> {0..3, 8..11}, 8..15
//            -> {4..7, 12..15}); lane group g reads k chunk 4g + s at step s (not 4s + g);
//            the transposed reads' row quads are qoff(g) = 0, 8, 4, 12 (not 4g);
//   D = 64:  chunk c of row r at c ^ (r & 7) (the attention kernels' D = 64 swizzle costs 4
//            extra cycles per row-fragment read with every mapping tried); identity rows, k
//            chunk 4s + g, quads 4g.
// Lane group g then owns queries 16 b + quad(g) + i in register i of query block b.
template <int D>
struct Dkdv16Lay;
template <>
struct Dkdv16Lay<128> {
  static __device__ __forceinline__ int swz(int r) { return swz_chunk<16>(r); }
  static __device__ __forceinline__ int arow(int m) { return (m & 3) | ((m & 4) << 1) | ((m & 8) >> 1); }
  static __device__ __forceinline__ int dcol(int g, int s) { return 32 * g + 8 * s; }
  static __device__ __forceinline__ int quad(int g) { return 4 * (((g & 1) << 1) | (g >> 1)); }
};
template <>
struct Dkdv16Lay<64> {
  static __device__ __forceinline__ int swz(int r) { return r & 7; }
  static __device__ __forceinline__ int arow(int m) { return m; }
  static __device__ __forceinline__ int dcol(int g, int s) { return 32 * s + 8 * g; }
  static __device__ __forceinline__ int quad(int g) { return 4 * g; }
};

// dK/dV kernel for bf16 inputs built for two or more waves per SIMD: 16 keys per wave on
// v_mfma_f32_16x16x32_bf16, NW waves per workgroup (16 NW keys of one head). At D = 128 a
// wave's dK/dV accumulators take 64 registers (16 keys x 128 d x 2 / 64 lanes) and its K/V
// fragments 32, so with one 64-query tile's S and dP (32) it fits the 256 registers of a
// two-wave SIMD, where the 32-key kernel above needs about 410 and runs one wave per SIMD; at
// D = 64 half that, three waves per SIMD. The price is LDS traffic: every wave reads the whole
// Q and dO tile twice (row fragments for S and dP, transposed fragments for dK and dV), twice
// the bytes per MFMA of the 32-key form.
// Orientation: S = Q K^T with M = 16 queries, N = the wave's 16 keys, K = 32 d, so lane l owns
// key l % 16; P^T and dS^T feed dV += P^T dO and dK += dS^T Q as A operands (M = keys, K = 32
// queries: slots 0..3 from block 2c, 4..7 from block 2c + 1), with dO and Q read transposed
// (ds_read_b64_tr_b16); row order, k order and quads as in Dkdv16Lay.
// Per 64-query tile: 4 D / 32 steps of S, dP (one query block and 32 d each; the weights of
// block b run under the steps of block b + 1), then 2 D / 16 steps of dV, dK (one 32-query
// half and 16 d each; block 3's weights under the first half), the next tile's copy spread over
// the first steps, one barrier. Same work items (bwd_block_coords), tile streaming, masking
// and outputs as attn_bwd_bf16_kernel.
// Built with NW = 4 (64 keys per workgroup). At C4a 0.326-0.335 ms against 0.339-0.357 ms for
// the 32-key kernel in the same calls, and 0.339-0.346 ms with NW = 8 (128 keys, one workgroup
// per CU, its two waves per SIMD in step); at C3 (D = 64) 0.182-0.183 ms against 0.190-0.197.
// The 32-key kernel stays for the clipped and shifted variants.
template <int D>
constexpr int dkdv16_waves_per_simd() { return D == 64 ? 3 : 2; }
template <int D, int NW, int MODE, int L2N, int LAYOUT>
__global__ __launch_bounds__(64 * NW, dkdv16_waves_per_simd<D>() * 4 / NW) void attn_bwd_dkdv16_kernel(AttnBwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  typedef Dkdv16Lay<D> Lay;
  constexpr int BQ = BF_BQ, CPR = D / 8, NS = D / 32, NDB = D / 16;
  constexpr int PF = 2;                       // LDS fragments read PF steps ahead (3: no faster)
  constexpr int KB = 16 * NW;                 // keys per workgroup
  constexpr int NMASK = KB / BQ;              // query tiles that cross the diagonal
  constexpr int RPI = 64 / CPR;               // tile rows per copy instruction
  constexpr int PW = BQ / RPI / NW;           // copy instruction pairs per wave and tile
  constexpr int EA = 4 / NS;                  // weights per S/dP step (block b - 1)
  constexpr int CE = NDB / 4;                 // dV/dK steps per weight of block 3
  static_assert(KB % BQ == 0 && PW >= 1 && PW <= NS && EA >= 1 && CE >= 1, "work split");
  __shared__ __attribute__((aligned(16))) bf16 Qs0[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 Qs1[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dOs0[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dOs1[BQ * D];
  __shared__ __attribute__((aligned(16))) float st0[BQ];
  __shared__ __attribute__((aligned(16))) float st1[BQ];
  __shared__ __attribute__((aligned(16))) float di0[BQ];
  __shared__ __attribute__((aligned(16))) float di1[BQ];

  if (p.flag) {
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  const int nbh = p.B * p.H, nkb = ceil_div(T_, KB);
  int bh, kblk;
  bwd_block_coords(blockIdx.x, nbh, nkb, bh, kblk);
  const int k0 = kblk * KB;
  const size_t base = head_base(bh, p.H, T_, D, LAYOUT);
  const int ld = LAYOUT ? p.H * D : D;  // elements between positions
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + base;
  const bf16* K = reinterpret_cast<const bf16*>(p.k) + base;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + base;
  const bf16* dO = reinterpret_cast<const bf16*>(p.dO) + base;
  const int nbytes = head_bytes(T_, ld, D, 2);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)Q, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rdo = __builtin_amdgcn_make_buffer_rsrc((void*)dO, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rst =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.stat + (size_t)bh * T_), (short)0, T_ * 4, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rdi =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.di + (size_t)bh * T_), (short)0, T_ * 4, BUF_RSRC_WORD3);
  const int wk0 = k0 + wave * 16;  // this wave's first key
  const int mykey = wk0 + l16;
  const int log2n = p.log2n;
  const int nq = ceil_div(T_, BQ);
  const int qstart = k0 / BQ;

  // Copy instruction pair j of a 64-row Q / dO tile into LDS in this layout (as tile_dma2_part:
  // lane l of an instruction writes 16 bytes at base + 16 l, rows past T land as zeros; both
  // swizzles satisfy swz(RPI J + r) = swz(r) ^ swz(RPI J) for r < RPI).
  int dma_rowb = (lane / CPR) * ld * 2;
  int dma_chunkb = 16 * ((lane % CPR) ^ Lay::swz(lane / CPR));
  asm volatile("" : "+v"(dma_rowb), "+v"(dma_chunkb));
  auto dma_part = [&](bf16* la, bf16* lb, int r0, int j) {
    auto lla = LDS_PTR(bf16, la);
    auto llb = LDS_PTR(bf16, lb);
    asm volatile("" : "+s"(lla), "+s"(llb));
    const int J = wave * PW + j;
    const int voff = (r0 + RPI * J) * ld * 2 + dma_rowb + (dma_chunkb ^ (16 * Lay::swz(RPI * J)));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, lla + J * 512, 16, voff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rdo, llb + J * 512, 16, voff, 0, 0, 0);
  };
  auto lds_at = [](int row, int col) { return row * D + (((col >> 3) ^ Lay::swz(row)) << 3) + (col & 7); };

#pragma unroll
  for (int j = 0; j < PW; ++j) dma_part(Qs0, dOs0, qstart * BQ, j);
  bwd_stat_dma(st0, di0, rst, rdi, qstart * BQ, wave, lane);
  // K and V fragments of this wave's keys (B operands of S = Q K^T and dP = dO V^T): at step
  // s lane group g covers d = dcol(g, s) .. + 7 (the k order of the 32-deep steps is free as
  // long as both operands share it), so lane l holds K[mykey][dcol(g, s) + j]. Keys past T
  // are zero and always masked.
  bf16x8 kf[NS], vf[NS];
  {
    const size_t row = (size_t)min(mykey, T_ - 1) * ld;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kf[s] = ld8(K + row + Lay::dcol(g, s));
      vf[s] = ld8(V + row + Lay::dcol(g, s));
    }
    keep_own_row<NS>(kf, mykey < T_);
    keep_own_row<NS>(vf, mykey < T_);
  }
  floatx4 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = floatx4{};
    dv[db] = floatx4{};
  }
  // Per-lane LDS offsets (both swizzles repeat every 16 rows): row fragments of Q / dO for S
  // and dP (row arow(l16) of a query block, d = dcol(g, s)) and transposed fragments for dV and
  // dK (rows quad(g) + (0..3) of a 16-row half, columns 16 db + (0..15)).
  const int qoff = Lay::quad(g);
  int a_off[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) a_off[s] = lds_at(Lay::arow(l16), Lay::dcol(g, s));
  int t_off[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) t_off[db] = lds_at(qoff + (l16 >> 2), 16 * db + 4 * (lane & 3));

  constexpr int RING = PF + 1;
  bf16x8 aq[RING], ao[RING];  // row fragments of Q / dO, PF steps ahead
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < PF; ++t) {
    aq[t] = ld8(Qs0 + (t / NS) * 16 * D + a_off[t % NS]);
    ao[t] = ld8(dOs0 + (t / NS) * 16 * D + a_off[t % NS]);
  }
  constexpr int VE = bwd_valu_per_elem<MODE>();

  auto tile = [&](auto bufc, auto maskc, int qt) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool MASKED = decltype(maskc)::value;
    const bf16* Qs = BUF ? Qs1 : Qs0;
    const bf16* dOs = BUF ? dOs1 : dOs0;
    const float* sts = BUF ? st1 : st0;
    const float* dis = BUF ? di1 : di0;
    const int qbase = qt * BQ;

    floatx4 s[4], dp[4];
    floatx4 sv[2], dvv[2];  // stat and di of a block's queries (slot = block & 1)
    bf16x8 pa[2], da[2];
    float pw[4], dsx[4];
    bf16x8 cf[RING][2];    // transposed dO / Q fragments of the dV/dK steps, PF steps ahead

    auto a_step = [&](int t) {
      const int b = t / NS, st = t % NS, tn = t + PF;
      if (tn < 4 * NS) {
        aq[tn % RING] = ld8(Qs + (tn / NS) * 16 * D + a_off[tn % NS]);
        ao[tn % RING] = ld8(dOs + (tn / NS) * 16 * D + a_off[tn % NS]);
      }
      s[b] = mfma16_bf16(aq[t % RING], kf[st], s[b]);
      dp[b] = mfma16_bf16(ao[t % RING], vf[st], dp[b]);
    };
    auto load_stats = [&](int b) {
      sv[b & 1] = *reinterpret_cast<const floatx4*>(sts + 16 * b + qoff);
      dvv[b & 1] = *reinterpret_cast<const floatx4*>(dis + 16 * b + qoff);
    };
    // Weight P and score gradient dS of element i of query block b (query 16 b + qoff + i).
    auto elem = [&](int b, int i) {
      const bool masked = MASKED && mykey > qbase + 16 * b + qoff + i;
      bwd_elem<MODE, L2N>(s[b][i], dp[b][i], sv[b & 1][i], dvv[b & 1][i], masked, p, log2n, pw[i], dsx[i]);
      const int c = b >> 1, j0 = 4 * (b & 1);
      if (i & 1) {
        pa[c][j0 + i - 1] = f2bf(pw[i - 1]);
        pa[c][j0 + i] = f2bf(pw[i]);
        da[c][j0 + i - 1] = f2bf(dsx[i - 1]);
        da[c][j0 + i] = f2bf(dsx[i]);
      }
    };
    // dV/dK step u: query half c = u / NDB (queries 32 c ..), d block db = u % NDB.
    auto c_load = [&](int u) {
      const int c = u / NDB, db = u % NDB;
      cf[u % RING][0] = tr_frag_at(dOs + 32 * c * D, t_off[db], t_off[db] + 16 * D);
      cf[u % RING][1] = tr_frag_at(Qs + 32 * c * D, t_off[db], t_off[db] + 16 * D);
    };
    auto c_step = [&](int u) {
      const int c = u / NDB, db = u % NDB;
      dv[db] = mfma16_bf16(pa[c], cf[u % RING][0], dv[db]);
      dk[db] = mfma16_bf16(da[c], cf[u % RING][1], dk[db]);
    };

#pragma unroll
    for (int b = 0; b < 4; ++b) {
      s[b] = floatx4{};
      dp[b] = floatx4{};
    }
    // S, dP steps: block b's NS steps carry the weights of block b - 1 (EA elements each) and
    // load block b's stat and di into the other slot; block 0's carry the copy of the next
    // tile (issued unconditionally: past the last tile its rows lie beyond the descriptors'
    // ranges and zeros land in the unused buffer set).
    load_stats(0);
#pragma unroll
    for (int t = 0; t < 4 * NS; ++t) {
      const int b = t / NS, st = t % NS;
      if (st == 0 && b >= 1) load_stats(b);
      a_step(t);
      if (b == 0) {
        if (st < PW) {
          if constexpr (BUF) dma_part(Qs0, dOs0, qbase + BQ, st);
          else dma_part(Qs1, dOs1, qbase + BQ, st);
        }
        if (st == NS - 1) {
          if constexpr (BUF) bwd_stat_dma(st0, di0, rst, rdi, qbase + BQ, wave, lane);
          else bwd_stat_dma(st1, di1, rst, rdi, qbase + BQ, wave, lane);
        }
        step_order_r<2, 0>(t + PF < 4 * NS ? 2 : 0);
      } else {
#pragma unroll
        for (int e = 0; e < EA; ++e) elem(b - 1, EA * st + e);
        if (t >= 4 * NS - PF) c_load(t - (4 * NS - PF));
        // LDS reads: the fragments PF steps ahead (2), the block's stats (2) at its first
        // step, the first dV/dK fragments (4) at the last PF steps.
        step_order_r<2, VE * EA>((t + PF < 4 * NS ? 2 : 0) + (st == 0 ? 2 : 0) + (t >= 4 * NS - PF ? 4 : 0));
      }
    }
    // dV, dK steps: the first half (blocks 0, 1) under the weights of block 3.
#pragma unroll
    for (int u = 0; u < 2 * NDB; ++u) {
      if (u + PF < 2 * NDB) c_load(u + PF);
      c_step(u);
      if (u < NDB && u % CE == 0) {
        elem(3, u / CE);
        step_order_r<2, VE>(u + PF < 2 * NDB ? 4 : 0);
      } else {
        step_order_r<2, 0>(u + PF < 2 * NDB ? 4 : 0);
      }
    }

    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this wave's copies of the next tile have landed
    __syncthreads();                     // the next buffer set is complete; this one is free
    {
      const bf16* Qn = BUF ? Qs0 : Qs1;
      const bf16* dOn = BUF ? dOs0 : dOs1;
#pragma unroll
      for (int t = 0; t < PF; ++t) {
        aq[t] = ld8(Qn + (t / NS) * 16 * D + a_off[t % NS]);
        ao[t] = ld8(dOn + (t / NS) * 16 * D + a_off[t % NS]);
      }
    }
  };

  // The first NMASK tiles cross the diagonal; the rest alternate buffer sets.
  int qt = qstart;
  tile(std::integral_constant<int, 0>{}, std::true_type{}, qt);
  if constexpr (NMASK == 2) {
    if (qt + 1 < nq) tile(std::integral_constant<int, 1>{}, std::true_type{}, qt + 1);
  }
  qt += NMASK;
  while (qt < nq) {
    tile(std::integral_constant<int, NMASK & 1>{}, std::false_type{}, qt);
    if (++qt >= nq) break;
    tile(std::integral_constant<int, (NMASK + 1) & 1>{}, std::false_type{}, qt);
    ++qt;
  }

  // dK = n * acc, dV = acc (flash.py:591-597), rounded to bf16: register i of d block db
  // holds key wk0 + 4 g + i, column 16 db + l16.
  const float slope = (float)(1 << log2n);
  bf16* DK = reinterpret_cast<bf16*>(p.dk) + base;
  bf16* DV = reinterpret_cast<bf16*>(p.dv) + base;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = wk0 + 4 * g + i;
    if (key < T_) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const size_t o = (size_t)key * ld + 16 * db + l16;
        DK[o] = f2bf(dk[db][i] * slope);
        DV[o] = f2bf(dv[db][i]);
      }
    }
  }
  // The last workgroup (the lightest causal key block) also forms the sink gradient.
  if (blockIdx.x == gridDim.x - 1) attn_sink_grad(p, ceil_div(T_, SINK_ROWS));
}

// dQ kernel for bf16 inputs (query-stationary; no atomics): one workgroup = 4 waves = 128
// queries of one (b, h), 32 per wave. Scores are formed transposed, S^T = K Q^T and
// dP^T = V dO^T (Q and dO fragments held in registers, so each lane owns one query and its
// stat / di are per-lane scalars); dS^T feeds dQ^T += K^T dS^T directly as the B operand,
// with K^T fragments read transposed from the K tile. K/V stream through LDS in 64-key tiles
// that ping-pong between two buffer sets, each copied during the previous tile's first steps.
// Per tile:
//   R1  S^T, dP^T of keys 0..31 | next tile's copy (MFMA | VMEM)
//   R2  S^T, dP^T of keys 32..63 | dS of 0..31   (MFMA | VALU)
//   R3  dQ^T over keys 0..31     | dS of 32..63  (MFMA | VALU)
//   R4  dQ^T over keys 32..63                    (MFMA)
// The output is dq = round(round(n * acc) * dq_scale) (flash.py:592 and the q_s chain rule).
//
// Before the tiles the kernel forms this workgroup's di (written for the dK/dV kernel, which
// runs after it) and its partial sum of mass * di for the sink gradient (flash.py:694-705,
// 721-723). Unshifted variants take di = sum_d dO o from the rounded output, as
// flash.py:633 does. The shifted fallback saves no f32 copy of its output (the reference's
// precise_output, flash.py:322, exists to make this sum exact); it takes
// di = sum_j p_ij dP_ij from a first pass over the keys with the same f32 weights p and
// products dP that its score gradients use, so that sum_j p_ij (dP_ij - di_i) vanishes to
// f32 rounding however the weights are spread. In exact arithmetic both are <dO_i, o_i>.
// Waves per SIMD the dQ kernel is built for: at D = 64 the in-range kernel with n fixed at
// compile time fits 168 VGPRs (16 bytes spilled) and runs three (C3 dQ 0.158 -> 0.152 ms,
// measured A/B on one box); the other variants spill far more at that bound and keep two.
template <int D, int MODE, int L2N>
constexpr int dq_waves_per_simd() { return D == 64 && MODE == MODE_INRANGE && L2N > 0 ? 3 : 2; }

template <int D, int MODE, int L2N, int LAYOUT>
__global__ __launch_bounds__(256, (dq_waves_per_simd<D, MODE, L2N>())) void attn_bwd_dq_kernel(AttnBwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr int BK = 64, CPR = D / 8, NDB = D / 32, NF = D / 16;
  constexpr int PW = 64 * CPR / 64 / 4;  // copy instruction pairs per wave and tile
  __shared__ __attribute__((aligned(16))) bf16 Ks0[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Ks1[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Vs0[BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Vs1[BK * D];
  __shared__ float red[4];

  if (p.flag) {
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  const int nqb = ceil_div(T_, 128);
  const int nbh = p.B * p.H;
  const int ld = LAYOUT ? p.H * D : D;  // elements between positions
  const int log2n = p.log2n;
  const int nbytes = head_bytes(T_, ld, D, 2);

  // Per-lane swizzled offsets (the swizzle repeats every 16 rows).
  const int trow = (lane & 15) >> 2;
  int row_off[NF];  // row fragments of K / V: row l32, k chunk 2 st + h
#pragma unroll
  for (int st = 0; st < NF; ++st) row_off[st] = swz_at<CPR>(l32, 16 * st + 8 * h);
  int tk_lo[NDB], tk_hi[NDB];  // transposed K fragments: rows 4h + (0..3), 4h + 8 + (0..3)
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tk_lo[db] = swz_at<CPR>(4 * h + trow, tr_col(db * 32, lane));
    tk_hi[db] = swz_at<CPR>(4 * h + 8 + trow, tr_col(db * 32, lane));
  }
  constexpr int VE = bwd_valu_per_elem<MODE>();

  // One 128-query block qb of head bh.
  auto run = [&](int bh, int qb) __attribute__((always_inline)) {
  const int head = bh % p.H;
  const size_t base = head_base(bh, p.H, T_, D, LAYOUT);
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + base;
  const bf16* K = reinterpret_cast<const bf16*>(p.k) + base;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + base;
  const bf16* dO = reinterpret_cast<const bf16*>(p.dO) + base;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)K, (short)0, nbytes, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)V, (short)0, nbytes, BUF_RSRC_WORD3);
  const int q0 = qb * 128 + wave * 32;
  const int myq = q0 + l32;
  const int ntiles = (min(qb * 128 + 127, T_ - 1)) / BK + 1;  // key tiles up to the last query

  tile_dma2<D>(Ks0, Vs0, rk, rv, 0, wave, lane, ld);
  // Q and dO fragments of this lane's query (B operands of S^T = K Q^T, dP^T = V dO^T);
  // queries past T carry stat = 0, so their weights and score gradients are zero.
  bf16x8 qf[NF], of[NF];
  const bool live = myq < T_;
  {
    const size_t row = (size_t)min(myq, T_ - 1) * ld + 8 * h;
#pragma unroll
    for (int s = 0; s < NF; ++s) {
      qf[s] = ld8(Q + row + 16 * s);
      of[s] = ld8(dO + row + 16 * s);
    }
    keep_own_row<NF>(qf, live);
    keep_own_row<NF>(of, live);
  }
  const float stq = live ? p.stat[(size_t)bh * T_ + myq] : 0.0f;
  float diq = 0.0f;
  if constexpr (MODE != MODE_SHIFTED) {
    // di = sum_d dO o over the rounded output (flash.py:633); the two lane halves hold
    // alternate 8-element chunks of the row.
    const bf16* O = reinterpret_cast<const bf16*>(p.o) + base + (size_t)min(myq, T_ - 1) * ld;
    bf16x8 ovs[NF];
#pragma unroll
    for (int st = 0; st < NF; ++st) ovs[st] = ld8(O + 16 * st + 8 * h);
    keep_own_row<NF>(ovs, live);
    float s = 0.0f;
#pragma unroll
    for (int st = 0; st < NF; ++st) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s += (float)of[st][j] * (float)ovs[st][j];
    }
    diq = s + xor32(s);
  }
  const float nsdi = -stq * diq;  // in range: -stat di of this lane's query
  floatx16 dqa[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dqa[db] = floatx16{};
  float di_acc = 0.0f;  // shifted fallback: this lane's share of sum_j p_ij dP_ij

  bf16x8 rk2[2], rv2[2];  // row fragments of K / V, one step ahead (R1, R2)
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
  rk2[0] = ld8(Ks0 + row_off[0]);
  rv2[0] = ld8(Vs0 + row_off[0]);

  // One key tile. BUF selects the LDS buffer set, MASKED the tiles that cross the diagonal,
  // DIPASS the shifted fallback's first pass (weights and dP only, summed into di_acc).
  auto tile = [&](auto bufc, auto maskc, auto dipassc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool MASKED = decltype(maskc)::value;
    constexpr bool DIPASS = decltype(dipassc)::value;
    const bf16* Ks = BUF ? Ks1 : Ks0;
    const bf16* Vs = BUF ? Vs1 : Vs0;
    const int kb0 = kt * BK;

    floatx16 s[2], dp[2];
    bf16x8 da[2][2];
    float pv[16], dsv[16];
    auto sdp_step = [&](int g) {
      const int blk = g / NF, st = g % NF;
      const int gn = g + 1;
      if (gn < 2 * NF) {
        rk2[gn % 2] = ld8(Ks + (gn / NF) * 32 * D + row_off[gn % NF]);
        rv2[gn % 2] = ld8(Vs + (gn / NF) * 32 * D + row_off[gn % NF]);
      }
      s[blk] = mfma_bf16(rk2[g % 2], qf[st], s[blk]);
      dp[blk] = mfma_bf16(rv2[g % 2], of[st], dp[blk]);
    };
    // Score gradient of key element i of block blk (this lane's query), rounded to bf16; in
    // the first pass of the shifted fallback, the weight times dP instead.
    auto elem = [&](int blk, int i) {
      const bool masked = MASKED && kb0 + blk * 32 + 8 * (i >> 2) + 4 * h + (i & 3) > myq;
      if constexpr (MODE == MODE_INRANGE) {
        // dS = p (dP - di) r with p = w stat (flash.py:350-356), formed as
        // (w r) fma(stat, dP, -stat di): the lane's query fixes stat and di, so the product
        // takes one instruction less per score (the same real number, f32 operations in
        // another order).
        float r;
        const float w = pow2n<L2N>(rho_fast(s[blk][i], r), log2n);
        dsv[i] = masked ? 0.0f : (w * r) * __builtin_fmaf(stq, dp[blk][i], nsdi);
      } else {
        bwd_elem<MODE, L2N>(s[blk][i], dp[blk][i], stq, diq, masked, p, log2n, pv[i], dsv[i]);
      }
      if constexpr (DIPASS) {
        di_acc += pv[i] * dp[blk][i];
      } else if (i & 1) {
        da[blk][i >> 3][(i & 7) - 1] = f2bf(dsv[i - 1]);
        da[blk][i >> 3][i & 7] = f2bf(dsv[i]);
      }
    };
    // dQ^T += K^T dS^T over one 32-key block, one d block per step (two 16-key halves);
    // fragments one step ahead.
    bf16x8 ft[2][2];
    auto dq_load = [&](int blk, int db, bf16x8 (&f)[2]) {
      const bf16* kb = Ks + blk * 32 * D;
      f[0] = tr_frag_at(kb, tk_lo[db], tk_hi[db]);
      f[1] = tr_frag_at(kb + 16 * D, tk_lo[db], tk_hi[db]);
    };

    // R1: S^T and dP^T of keys 0..31, with the copy of the next tile into the other buffer
    // set (free since the barrier that ended the previous tile) spread over its steps: issued
    // in one burst, the copies of the CU's eight waves queue on the vector memory path and
    // stall the waves. Past the last tile the rows lie beyond the descriptors' ranges (no
    // memory is read; zeros land in the unused buffer set).
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      s[b] = floatx16{};
      dp[b] = floatx16{};
    }
    const int r_next = kt + 1 < ntiles ? kb0 + BK : T_ + BK;
#pragma unroll
    for (int g = 0; g < NF; ++g) {
      sdp_step(g);
      if (g < PW) {
        if constexpr (BUF) tile_dma2_part<D>(Ks0, Vs0, rk, rv, r_next, wave, lane, g, ld);
        else tile_dma2_part<D>(Ks1, Vs1, rk, rv, r_next, wave, lane, g, ld);
      }
      step_order<2, 0, 4, 0>();
    }
    // R2: S^T and dP^T of keys 32..63 under dS of keys 0..31.
    constexpr int E2 = 16 / NF;
#pragma unroll
    for (int g = NF; g < 2 * NF; ++g) {
      sdp_step(g);
#pragma unroll
      for (int k = 0; k < E2; ++k) elem(0, E2 * (g - NF) + k);
      if (!DIPASS && g == 2 * NF - 1) dq_load(0, 0, ft[0]);
      step_order<2, VE * E2, 4 + 4, 0>();
    }
    if constexpr (DIPASS) {
#pragma unroll
      for (int i = 0; i < 16; ++i) elem(1, i);
    } else {
      // R3: dQ^T over keys 0..31 under dS of keys 32..63.
      constexpr int E3 = 16 / NDB;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int c = db & 1;
        if (db + 1 < NDB) dq_load(0, db + 1, ft[c ^ 1]);
        else dq_load(1, 0, ft[c ^ 1]);
        dqa[db] = mfma_bf16(ft[c][0], da[0][0], dqa[db]);
        dqa[db] = mfma_bf16(ft[c][1], da[0][1], dqa[db]);
#pragma unroll
        for (int k = 0; k < E3; ++k) elem(1, E3 * db + k);
        step_order<2, VE * E3, 4, 0>();
      }
      // R4: dQ^T over keys 32..63.
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int c = (db + NDB) & 1;
        if (db + 1 < NDB) dq_load(1, db + 1, ft[c ^ 1]);
        dqa[db] = mfma_bf16(ft[c][0], da[1][0], dqa[db]);
        dqa[db] = mfma_bf16(ft[c][1], da[1][1], dqa[db]);
        step_order<2, 0, 4, 0>();
      }
    }

    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this wave's copies of the next tile have landed
    __syncthreads();                     // the next tile is complete; this buffer set is free
    {
      const bf16* Kn = BUF ? Ks0 : Ks1;
      const bf16* Vn = BUF ? Vs0 : Vs1;
      rk2[0] = ld8(Kn + row_off[0]);
      rv2[0] = ld8(Vn + row_off[0]);
    }
  };

  // Key tiles 0 .. 2 qb - 1 lie wholly before this workgroup's queries; tiles 2 qb and
  // 2 qb + 1 cross the diagonal.
  const int nfull = min(2 * qb, ntiles);
  auto sweep = [&](auto dipassc) {
    int kt = 0;
    for (; kt < nfull; kt += 2) {
      tile(std::integral_constant<int, 0>{}, std::false_type{}, dipassc, kt);
      tile(std::integral_constant<int, 1>{}, std::false_type{}, dipassc, kt + 1);
    }
    if (kt < ntiles) {
      tile(std::integral_constant<int, 0>{}, std::true_type{}, dipassc, kt);
      if (kt + 1 < ntiles) tile(std::integral_constant<int, 1>{}, std::true_type{}, dipassc, kt + 1);
    }
  };
  if constexpr (MODE == MODE_SHIFTED) {
    sweep(std::true_type{});
    diq = di_acc + xor32(di_acc);
    __syncthreads();  // every wave is done with the last tile's fragments
    tile_dma2<D>(Ks0, Vs0, rk, rv, 0, wave, lane, ld);
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    __syncthreads();
    rk2[0] = ld8(Ks0 + row_off[0]);
    rv2[0] = ld8(Vs0 + row_off[0]);
  }
  // di for the dK/dV kernel, and this block's share of the sink gradient: the sink's weight
  // relative to the row, mass = rho(b)^n stat (unshifted, 1/Z statistic) or (rho(b) stat)^n.
  if (live && h == 0) p.di[(size_t)bh * T_ + myq] = diq;
  if (p.sink) {
    float b = p.sink[head];
    if constexpr (MODE == MODE_CLIPPED) b = fminf(b, p.clamp);
    const float rb = rho_exact(b);
    const bool inv_stat = MODE == MODE_INRANGE || (MODE == MODE_CLIPPED && p.inv_stat);
    const float mass = inv_stat ? pow2n<L2N>(rb, log2n) * stq : pow2n<L2N>(rb * stq, log2n);
    float part = live && h == 0 ? mass * diq : 0.0f;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
    if (lane == 0) red[wave] = part;
    __syncthreads();
    if (threadIdx.x == 0) p.sink_part[(size_t)bh * nqb + qb] = red[0] + red[1] + red[2] + red[3];
  }
  sweep(std::false_type{});

  if (live) {
    const float slope = (float)(1 << log2n);
    bf16* DQ = reinterpret_cast<bf16*>(p.dq) + base + (size_t)myq * ld;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 ob;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16 dqs = f2bf(dqa[db][4 * g + e] * slope);
          ob[e] = f2bf((float)dqs * p.dq_scale);
        }
        *reinterpret_cast<bf16x4*>(DQ + db * 32 + 8 * g + 4 * h) = ob;
      }
    }
  }
  };
  if constexpr (MODE == MODE_INRANGE) {
    run(blockIdx.x, nqb - 1 - blockIdx.y);  // heaviest causal rows first
  } else {
    for (int L = blockIdx.x; L < nbh * nqb; L += gridDim.x) {
      run(L % nbh, nqb - 1 - L / nbh);
      __syncthreads();  // the next item's first copies overwrite both LDS buffer sets
    }
  }
}

// ---------------------------------------------------------------------------
// post: dq and the per-head sink gradient
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_post_kernel(AttnBwdParams p, size_t total, int nblk, int D) {
  const float slope = (float)(1 << p.log2n);
  // 8 consecutive elements per thread (total is a multiple of D, itself a multiple of 8).
  const size_t n8 = total / 8;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
    const floatx4 a0 = *reinterpret_cast<const floatx4*>(p.dq_acc + 8 * i);
    const floatx4 a1 = *reinterpret_cast<const floatx4*>(p.dq_acc + 8 * i + 4);
    T out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const T dqs = (T)((j < 4 ? a0[j] : a1[j - 4]) * slope);  // kernel output dq_s (flash.py:592)
      out[j] = (T)((float)dqs * p.dq_scale);                   // chain rule through q_s
    }
    // dq_acc is (B, H, T, D); dq is stored in the call's layout.
    size_t dst = 8 * i;
    if (p.layout) {
      const size_t row = dst / D;
      const int col = (int)(dst - row * D);
      const int bh = (int)(row / p.T), t = (int)(row - (size_t)bh * p.T);
      dst = head_base(bh, p.H, p.T, D, 1) + (size_t)t * row_stride(p.H, D, 1) + col;
    }
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(reinterpret_cast<T*>(p.dq) + dst) = *reinterpret_cast<const uint4*>(out);
    } else {
      *reinterpret_cast<uint4*>(reinterpret_cast<T*>(p.dq) + dst) = *reinterpret_cast<const uint4*>(out);
      *reinterpret_cast<uint4*>(reinterpret_cast<T*>(p.dq) + dst + 4) = *reinterpret_cast<const uint4*>(out + 4);
    }
  }
  if (blockIdx.x == 0) attn_sink_grad(p, nblk);
}

// Grid of a fallback (grid-stride) kernel: every work item gets its own workgroup when the
// variant was chosen on the host; when it is one branch of the device guard it usually exits
// at once, so it is launched as a small grid (a multiple of 8, so work item % 8 stays the XCD).
static int fallback_grid(const AttnBwdParams& p, int items) {
  return p.flag ? std::min(items, FALLBACK_GRID) : items;
}

// bf16, one variant: the dQ kernel (which also writes di and the sink partials) or the dK/dV
// kernel (which reads di).
template <int D, int LAYOUT>
static hipError_t launch_bwd_bf16_l(const AttnBwdParams& p, int mode, bool dq, hipStream_t st) {
  const int nbh = p.B * p.H, nkb = ceil_div(p.T, BWD_BK), nqb = ceil_div(p.T, 128);
  dim3 block(256);
  if (dq) {
    switch (mode) {
      case MODE_INRANGE: {
        KTimer t("attn_bwd_dq_inrange", st);
        dim3 qgrid(nbh, nqb);
        if (p.log2n == 4) hipLaunchKernelGGL((attn_bwd_dq_kernel<D, MODE_INRANGE, 4, LAYOUT>), qgrid, block, 0, st, p);
        else hipLaunchKernelGGL((attn_bwd_dq_kernel<D, MODE_INRANGE, 0, LAYOUT>), qgrid, block, 0, st, p);
      } break;
      case MODE_CLIPPED: {
        KTimer t("attn_bwd_dq_clipped", st);
        hipLaunchKernelGGL((attn_bwd_dq_kernel<D, MODE_CLIPPED, 0, LAYOUT>), dim3(fallback_grid(p, nbh * nqb)), block,
                           0, st, p);
      } break;
      case MODE_SHIFTED: {
        KTimer t("attn_bwd_dq_shifted", st);
        hipLaunchKernelGGL((attn_bwd_dq_kernel<D, MODE_SHIFTED, 0, LAYOUT>), dim3(fallback_grid(p, nbh * nqb)), block,
                           0, st, p);
      } break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (mode) {
      case MODE_INRANGE: {
        // 16 keys per wave, 4-wave workgroups of 64 keys (two per CU at D = 128, three at 64).
        KTimer t("attn_bwd_inrange", st);
        dim3 grid16(nbh * ceil_div(p.T, 64));
        if (p.log2n == 4) hipLaunchKernelGGL((attn_bwd_dkdv16_kernel<D, 4, MODE_INRANGE, 4, LAYOUT>), grid16, block, 0, st, p);
        else hipLaunchKernelGGL((attn_bwd_dkdv16_kernel<D, 4, MODE_INRANGE, 0, LAYOUT>), grid16, block, 0, st, p);
      } break;
      case MODE_CLIPPED: {
        KTimer t("attn_bwd_clipped", st);
        hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_CLIPPED, 0, LAYOUT>), dim3(fallback_grid(p, nbh * nkb)), block,
                           0, st, p);
      } break;
      case MODE_SHIFTED: {
        KTimer t("attn_bwd_shifted", st);
        hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_SHIFTED, 0, LAYOUT>), dim3(fallback_grid(p, nbh * nkb)), block,
                           0, st, p);
      } break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

template <int D>
static hipError_t launch_bwd_bf16(const AttnBwdParams& p, int mode, bool dq, hipStream_t st) {
  return p.layout ? launch_bwd_bf16_l<D, 1>(p, mode, dq, st) : launch_bwd_bf16_l<D, 0>(p, mode, dq, st);
}

// f32: the key-stationary kernel with dQ atomics.
template <int D>
static hipError_t launch_bwd_f32(const AttnBwdParams& p, int mode, hipStream_t st) {
  const int nbh = p.B * p.H, nkb = ceil_div(p.T, BWD_BK);
  dim3 block(256);
  switch (mode) {
    case MODE_INRANGE: {
      KTimer t("attn_bwd_inrange", st);
      dim3 grid(nbh, nkb);
      if (p.log2n == 4) hipLaunchKernelGGL((attn_bwd_kernel<float, D, MODE_INRANGE, 4>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((attn_bwd_kernel<float, D, MODE_INRANGE, 0>), grid, block, 0, st, p);
    } break;
    case MODE_CLIPPED: {
      KTimer t("attn_bwd_clipped", st);
      hipLaunchKernelGGL((attn_bwd_kernel<float, D, MODE_CLIPPED, 0>), dim3(fallback_grid(p, nbh * nkb)), block, 0, st,
                         p);
    } break;
    case MODE_SHIFTED: {
      KTimer t("attn_bwd_shifted", st);
      hipLaunchKernelGGL((attn_bwd_kernel<float, D, MODE_SHIFTED, 0>), dim3(fallback_grid(p, nbh * nkb)), block, 0, st,
                         p);
    } break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int attn_bwd_sink_blocks(int T) { return ceil_div(T, SINK_ROWS); }

// modes: list of variants to launch (each exits early unless the guard selects it).
hipError_t launch_attn_bwd(const AttnBwdParams& p, int D, bool bf16_io, const int* modes, int nmodes,
                           hipStream_t st) {
  const int nblk = attn_bwd_sink_blocks(p.T);
  hipError_t e = hipSuccess;
  if (bf16_io) {
    // dQ first (it writes di), then dK/dV; the sink partials come from the dQ kernel.
    for (int pass = 0; pass < 2 && e == hipSuccess; ++pass)
      for (int m = 0; m < nmodes && e == hipSuccess; ++m)
        e = D == 64 ? launch_bwd_bf16<64>(p, modes[m], pass == 0, st) : launch_bwd_bf16<128>(p, modes[m], pass == 0, st);
  } else {
    {
      KTimer t("attn_bwd_pre", st);
      hipLaunchKernelGGL((attn_bwd_pre_kernel<float>), dim3(p.B * p.H, nblk), dim3(256), 0, st, p, D);
    }
    e = hipGetLastError();
    for (int m = 0; m < nmodes && e == hipSuccess; ++m)
      e = D == 64 ? launch_bwd_f32<64>(p, modes[m], st) : launch_bwd_f32<128>(p, modes[m], st);
  }
  if (e != hipSuccess || bf16_io) return e;  // bf16: the dK/dV kernel formed the sink gradient
  // f32: dq from the accumulator, and the sink gradient.
  const size_t total = (size_t)p.B * p.H * p.T * D;
  const int blocks = (int)std::max<size_t>(std::min<size_t>((total / 8 + 255) / 256, 16384), 1);
  {
    KTimer t("attn_bwd_post", st);
    hipLaunchKernelGGL((attn_bwd_post_kernel<float>), dim3(blocks), dim3(256), 0, st, p, total, nblk, D);
  }
  return hipGetLastError();
}

}  // namespace alg
