// Causal algebraic attention backward for gfx950.
//
// Replaces src/algebraic/kernels/flash.py:333-361 (tile gradients), 515-627 (fused and
// resident backward schedules), 630-645 (di), 694-726 (sink VJP) and
// src/algebraic/kernels/head_resident.py:91-119.
//
// Three launches:
//   pre   di = sum_d dO*o per row (from the rounded output in range, the f32 output when
//         shifted; flash.py:633), zero the f32 dQ accumulator, per-(b,h,block) partial sums
//         of mass*di for the sink gradient (flash.py:694-705, 721-723).
//   main  one workgroup = 4 waves = 128 keys of one (b,h); dK/dV accumulate in registers
//         while the kernel streams 64-query tiles of Q and dO through LDS. Scores are
//         formed as S = Q K^T so a lane owns one key column; P^T and dS^T feed dV += P^T dO
//         and dK += dS^T Q directly as MFMA A operands, with dO/Q fragments transposed by
//         ds_read_b64_tr_b16. dS is staged in LDS ([key][query]) and each wave forms one
//         quarter of the tile's dQ = dS K over the workgroup's 128 keys, added to the f32
//         accumulator with one atomic per element per key block (no per-key-block dQ
//         partials in HBM, unlike flash.py:537-544).
//   post  dq = round(round(n * acc) * dq_scale) and the per-head sink gradient.
#include "attn_common.h"

namespace alg {

constexpr int BWD_BK = 128;  // keys per workgroup
// Queries per streamed tile: 64, or 32 where 64 would not fit in LDS (f32 with D=128).
template <typename T, int D>
constexpr int bwd_bq() { return (sizeof(T) == 4 && D == 128) ? 32 : 64; }
constexpr int PRE_ROWS = 256;  // rows per pre-kernel workgroup

// ---------------------------------------------------------------------------
// pre: di, dq_acc = 0, sink partials
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_pre_kernel(AttnBwdParams p, int D) {
  const int bh = blockIdx.x;
  const int head = bh % p.H;
  const int T_ = p.T;
  bool shifted = p.mode == MODE_SHIFTED;
  if (p.flag) shifted = *p.flag == 0;
  const bool precise = shifted && p.o_precise != nullptr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.y * PRE_ROWS;
  const int n = 1 << p.log2n;
  float b = p.sink ? p.sink[head] : 0.0f;
  if (p.mode == MODE_CLIPPED && !p.flag) b = fminf(b, p.clamp);
  const float rb = rho_exact(b);
  const bool inv_stat = !shifted && (p.mode != MODE_CLIPPED || p.inv_stat);
  const float rbn = ipow_rt(rb, n);
  float part = 0.0f;
  // 8 elements per lane, D/8 lanes per row (vector loads of dO, o; vector zero-fill of dq_acc).
  const int lpr = D / 8, rpw = 64 / lpr;
  const int sub = lane / lpr, li = lane - sub * lpr;
  const int rend = min(row0 + PRE_ROWS, T_);
  for (int r0 = row0 + wave * rpw; r0 < rend; r0 += 4 * rpw) {
    const int r = r0 + sub;
    const bool ok = r < rend;
    float s = 0.0f;
    if (ok) {
      const size_t off = ((size_t)bh * T_ + r) * D + li * 8;
      float dov[8], ov[8];
      if constexpr (sizeof(T) == 2) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.dO) + off);
#pragma unroll
        for (int j = 0; j < 8; ++j) dov[j] = (float)a[j];
      } else {
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.dO) + off);
        const floatx4 a1 = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.dO) + off + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { dov[j] = a0[j]; dov[4 + j] = a1[j]; }
      }
      if (precise || sizeof(T) == 4) {
        const float* src = precise ? p.o_precise + off : reinterpret_cast<const float*>(p.o) + off;
        const floatx4 b0 = *reinterpret_cast<const floatx4*>(src);
        const floatx4 b1 = *reinterpret_cast<const floatx4*>(src + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { ov[j] = b0[j]; ov[4 + j] = b1[j]; }
      } else {
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.o) + off);
#pragma unroll
        for (int j = 0; j < 8; ++j) ov[j] = (float)b[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += dov[j] * ov[j];
      const floatx4 z = {};
      *reinterpret_cast<floatx4*>(p.dq_acc + off) = z;
      *reinterpret_cast<floatx4*>(p.dq_acc + off + 4) = z;
    }
    for (int m = 1; m < lpr; m <<= 1) s += __shfl_xor(s, m, 64);
    if (ok && li == 0) {
      p.di[(size_t)bh * T_ + r] = s;
      const float st = p.stat[(size_t)bh * T_ + r];
      const float mass = inv_stat ? rbn * st : ipow_rt(rb * st, n);
      part += mass * s;
    }
  }
  for (int m = 1; m < 64; m <<= 1) part += __shfl_xor(part, m, 64);
  __shared__ float red[4];
  if (lane == 0) red[wave] = part;
  __syncthreads();
  if (threadIdx.x == 0) p.sink_part[(size_t)bh * gridDim.y + blockIdx.y] = red[0] + red[1] + red[2] + red[3];
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
  static __device__ __forceinline__ void load(uint4 (&r)[PER], const T* src, int r0, int T_) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = min(idx / CPR, R - 1), col = (idx - (idx / CPR) * CPR) * CH;
      r[c] = *reinterpret_cast<const uint4*>(src + (size_t)min(r0 + row, T_ - 1) * D + col);
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
  const int bh = blockIdx.x;
  const int k0 = blockIdx.y * BWD_BK;  // blockIdx.y = 0 has the most causal work
  const size_t base = (size_t)bh * T_ * D;
  const T* Q = reinterpret_cast<const T*>(p.q) + base;
  const T* K = reinterpret_cast<const T*>(p.k) + base;
  const T* V = reinterpret_cast<const T*>(p.v) + base;
  const T* dO = reinterpret_cast<const T*>(p.dO) + base;
  const float* stat = p.stat + (size_t)bh * T_;
  const float* di = p.di + (size_t)bh * T_;
  float* dq_acc = p.dq_acc + base;
  const int wk0 = k0 + wave * 32;    // this wave's first key
  const int mykey = wk0 + l32;
  const int log2n = p.log2n;

  {
    typedef RowTile<T, D, BWD_BK> KT;
    uint4 kr[KT::PER];
    KT::load(kr, K, k0, T_);
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
      const size_t o = (size_t)mykey * D + 16 * s + 8 * h;
      kf[s] = mykey < T_ ? ld8(reinterpret_cast<const bf16*>(K) + o) : z;
      vf[s] = mykey < T_ ? ld8(reinterpret_cast<const bf16*>(V) + o) : z;
    } else {
      floatx4 z = {};
      const size_t o = (size_t)mykey * D + 8 * s + 4 * h;
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
    QT::load(qr, Q, qbase, T_);
    QT::load(dr, dO, qbase, T_);
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
  T* DK = reinterpret_cast<T*>(p.dk) + base;
  T* DV = reinterpret_cast<T*>(p.dv) + base;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = wk0 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (key < T_) {
        const size_t o = (size_t)key * D + db * 32 + l32;
        DK[o] = (T)(dk[db][i] * slope);
        DV[o] = (T)(dv[db][i]);
      }
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

constexpr int BF_BQ = 64;  // queries per streamed tile (bf16 kernel)

// Asynchronous copy of the query tile at qbase (q_s, dO, stat, di) into LDS landing buffers
// with global_load_lds: lane l of a wave instruction writes 16 (or 4) bytes at base + 16 l
// (4 l), so each lane fetches the logical chunk the swizzle places there. Rows past T read
// row T-1 (made inert when the tile is committed).
template <int D>
__device__ __forceinline__ void bwd_tile_copy(bf16* pq, bf16* pdo, float* pst, float* pdi, const bf16* Q,
                                              const bf16* dO, const float* stat, const float* di, int qbase, int T_,
                                              int wave) {
  constexpr int CPR = D / 8, RPI = 64 / CPR, PW = BF_BQ * CPR / 64 / 4;  // PW instructions per wave
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int J = wave * PW + j;
    const int row = RPI * J + lane / CPR;
    const int c = (lane % CPR) ^ swz_chunk<CPR>(row);
    const size_t off = (size_t)min(qbase + row, T_ - 1) * D + 8 * c;
    __builtin_amdgcn_global_load_lds(Q + off, LDS_PTR(void, pq + J * 512), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(dO + off, LDS_PTR(void, pdo + J * 512), 16, 0, 0);
  }
  const int row = min(qbase + lane, T_ - 1);
  if (wave == 0) __builtin_amdgcn_global_load_lds(stat + row, LDS_PTR(void, pst), 4, 0, 0);
  if (wave == 1) __builtin_amdgcn_global_load_lds(di + row, LDS_PTR(void, pdi), 4, 0, 0);
}

// Same decomposition as attn_bwd_kernel (128 keys per workgroup, 32 per wave; dK/dV in
// registers; dQ via the staged dS and f32 atomics), arranged for one wave per SIMD:
//  * the tile body has no branches: S and dP of both 32-query blocks, then both blocks'
//    weights and score gradients (masking by select), then dV and dK, so the scheduler can
//    overlap the MFMAs of one block with the VALU work of the other;
//  * the next tile is copied into LDS landing buffers by direct copies issued at the top of
//    the iteration (no staging registers) and moved into the working tiles after the dS
//    barrier; the dQ atomics come last, a full tile before the next wait on the counter;
//  * every LDS access is a per-lane swizzled offset computed once plus an immediate;
//  * the dQ atomics are buffer atomics whose range check drops rows past T.
template <int D, int MODE, int L2N>
__global__ __launch_bounds__(256, 1) void attn_bwd_bf16_kernel(AttnBwdParams p) {
  static_assert(D == 64 || D == 128, "head_dim");
  constexpr int BQ = BF_BQ, CPR = D / 8, SCPR = BQ / 8, NDB = D / 32, NF = D / 16;
  __shared__ __attribute__((aligned(16))) bf16 Ks[BWD_BK * D];
  __shared__ __attribute__((aligned(16))) bf16 Qs[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dOs[BQ * D];
  __shared__ __attribute__((aligned(16))) bf16 dSs[BWD_BK * BQ];
  __shared__ __attribute__((aligned(16))) float st_s[BQ];
  __shared__ __attribute__((aligned(16))) float di_s[BQ];
  __shared__ __attribute__((aligned(16))) bf16 pre_q[BQ * D];  // landing buffers
  __shared__ __attribute__((aligned(16))) bf16 pre_do[BQ * D];
  __shared__ __attribute__((aligned(16))) float pre_st[BQ];
  __shared__ __attribute__((aligned(16))) float pre_di[BQ];

  if (p.flag) {
    const bool in_range = *p.flag != 0;
    if ((MODE == MODE_SHIFTED) == in_range) return;
  }
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T_ = p.T;
  const int bh = blockIdx.x;
  const int k0 = blockIdx.y * BWD_BK;  // blockIdx.y = 0 has the most causal work
  const size_t base = (size_t)bh * T_ * D;
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + base;
  const bf16* K = reinterpret_cast<const bf16*>(p.k) + base;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + base;
  const bf16* dO = reinterpret_cast<const bf16*>(p.dO) + base;
  const float* stat = p.stat + (size_t)bh * T_;
  const float* di = p.di + (size_t)bh * T_;
  float* dq_acc = p.dq_acc + base;
  const int wk0 = k0 + wave * 32;  // this wave's first key
  const int mykey = wk0 + l32;
  const int log2n = p.log2n;
  const int nq = ceil_div(T_, BQ);
  const int qstart = k0 / BQ;

  bwd_tile_copy<D>(pre_q, pre_do, pre_st, pre_di, Q, dO, stat, di, qstart * BQ, T_, wave);
  {
    typedef RowTile<bf16, D, BWD_BK> KT;  // keys past T: finite stand-ins whose dS is zero
    uint4 kr[KT::PER];
    KT::load(kr, K, k0, T_);
    KT::store(Ks, 0, kr);
  }
  // K and V fragments of this wave's keys: B operands of S = Q K^T and dP = dO V^T.
  bf16x8 kf[NF], vf[NF];
#pragma unroll
  for (int s = 0; s < NF; ++s) {
    const bf16x8 z = {};
    const size_t o = (size_t)mykey * D + 16 * s + 8 * h;
    kf[s] = mykey < T_ ? ld8(K + o) : z;
    vf[s] = mykey < T_ ? ld8(V + o) : z;
  }
  floatx16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = floatx16{};
    dv[db] = floatx16{};
  }

  // Per-lane swizzled offsets: both swizzles repeat every 16 rows, so every access below is
  // one of these plus a multiple of 16 rows (an immediate offset).
  constexpr int NQH = BQ / 32;    // 32-query slices of a tile (dQ phase)
  constexpr int WPH = 4 / NQH;    // waves per slice
  constexpr int DBW = NDB / WPH;  // 32-wide d blocks per wave
  static_assert(DBW >= 1, "tile shape");
  const int qs = wave / WPH;
  const int db0 = (wave % WPH) * DBW;
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
  const int ts_lo = swz_at<SCPR>(8 * h + trow, tr_col(qs * 32, lane));  // dS, dQ phase
  const int ts_hi = swz_at<SCPR>(8 * h + 4 + trow, tr_col(qs * 32, lane));
  int tk_lo[DBW], tk_hi[DBW];  // K, dQ phase
#pragma unroll
  for (int j = 0; j < DBW; ++j) {
    tk_lo[j] = swz_at<CPR>(8 * h + trow, tr_col((db0 + j) * 32, lane));
    tk_hi[j] = swz_at<CPR>(8 * h + 4 + trow, tr_col((db0 + j) * 32, lane));
  }
  // dS writes: row wave*32 + l32, columns 32 sub + 8g + 4h. A column shift is not a constant
  // offset under the swizzle (only multiples of 16 rows are), so each block has its own.
  int ds_off[2][4];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int g = 0; g < 4; ++g) ds_off[sub][g] = swz_at<SCPR>(wave * 32 + l32, sub * 32 + 8 * g + 4 * h);
  const int lane_off = (4 * h * D + l32) * 4;  // dQ atomics (bytes)

  // Landing buffers -> working tiles (same swizzled layout: a straight 16-byte copy); rows
  // past T get stat = 0, which makes their weights and score gradients exactly zero.
  auto commit = [&](int qbase) {
    constexpr int CH = BQ * D / 8;
#pragma unroll
    for (int c = threadIdx.x; c < CH; c += 256) {
      reinterpret_cast<uint4*>(Qs)[c] = reinterpret_cast<const uint4*>(pre_q)[c];
      reinterpret_cast<uint4*>(dOs)[c] = reinterpret_cast<const uint4*>(pre_do)[c];
    }
    if (threadIdx.x < BQ) {
      const bool live = qbase + (int)threadIdx.x < T_;
      st_s[threadIdx.x] = live ? pre_st[threadIdx.x] : 0.0f;
      di_s[threadIdx.x] = live ? pre_di[threadIdx.x] : 0.0f;
    }
  };
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
  commit(qstart * BQ);
  __syncthreads();

  for (int qt = qstart; qt < nq; ++qt) {
    const int qbase = qt * BQ;
    const bool more = qt + 1 < nq;
    if (more) bwd_tile_copy<D>(pre_q, pre_do, pre_st, pre_di, Q, dO, stat, di, qbase + BQ, T_, wave);
    // S = Q K^T and dP = dO V^T for both 32-query blocks (lane = key).
    floatx16 s[2], dp[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      s[sub] = floatx16{};
      dp[sub] = floatx16{};
#pragma unroll
      for (int st = 0; st < NF; ++st) {
        s[sub] = mfma_bf16(*reinterpret_cast<const bf16x8*>(Qs + sub * 32 * D + row_off[st]), kf[st], s[sub]);
        dp[sub] = mfma_bf16(*reinterpret_cast<const bf16x8*>(dOs + sub * 32 * D + row_off[st]), vf[st], dp[sub]);
      }
    }
    // Weights P and score gradients dS (rounded to bf16 as the gradient products use them);
    // blocks that cross the diagonal mask keys after the query (all of them for blocks
    // wholly before this wave's keys).
    bf16x8 pa[2][2], da[2][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int sq0 = qbase + sub * 32;
      const bool diag = wk0 + 31 > sq0;
      float pv[16], dsv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const floatx4 stq = *reinterpret_cast<const floatx4*>(st_s + sub * 32 + 8 * g + 4 * h);
        const floatx4 diq = *reinterpret_cast<const floatx4*>(di_s + sub * 32 + 8 * g + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * g + e;
          const bool masked = diag && mykey > sq0 + 8 * g + 4 * h + e;
          bwd_elem<MODE, L2N>(s[sub][i], dp[sub][i], stq[e], diq[e], masked, p, log2n, pv[i], dsv[i]);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pa[sub][0][j] = f2bf(pv[j]);
        pa[sub][1][j] = f2bf(pv[8 + j]);
        da[sub][0][j] = f2bf(dsv[j]);
        da[sub][1][j] = f2bf(dsv[8 + j]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 v4;
#pragma unroll
        for (int e = 0; e < 4; ++e) v4[e] = f2bf(dsv[4 * g + e]);
        *reinterpret_cast<bf16x4*>(dSs + ds_off[sub][g]) = v4;  // staged [key][query]
      }
    }
    // dV += P^T dO and dK += dS^T Q (transposed dO / Q fragments from LDS).
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const bf16* qb = Qs + sub * 32 * D;
      const bf16* ob = dOs + sub * 32 * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        dv[db] = mfma_bf16(pa[sub][0], tr_frag_at(ob, tq_lo[db], tq_hi[db]), dv[db]);
        dv[db] = mfma_bf16(pa[sub][1], tr_frag_at(ob + 16 * D, tq_lo[db], tq_hi[db]), dv[db]);
        dk[db] = mfma_bf16(da[sub][0], tr_frag_at(qb, tq_lo[db], tq_hi[db]), dk[db]);
        dk[db] = mfma_bf16(da[sub][1], tr_frag_at(qb + 16 * D, tq_lo[db], tq_hi[db]), dk[db]);
      }
    }
    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this wave's copies of the next tile have landed
    __syncthreads();                     // dS complete; working tiles no longer read
    if (more) commit(qbase + BQ);
    // dQ tile = dS K over this workgroup's keys; each wave takes 32 queries x DBW d blocks.
    floatx16 dqa[DBW];
#pragma unroll
    for (int j = 0; j < DBW; ++j) dqa[j] = floatx16{};
#pragma unroll
    for (int ks = 0; ks < BWD_BK / 16; ++ks) {
      const bf16x8 a0 = tr_frag_at(dSs + ks * 16 * BQ, ts_lo, ts_hi);
#pragma unroll
      for (int j = 0; j < DBW; ++j) {
        const bf16x8 b0 = tr_frag_at(Ks + ks * 16 * D, tk_lo[j], tk_hi[j]);
        dqa[j] = mfma_bf16(a0, b0, dqa[j]);
      }
    }
    // Buffer atomics over this slice's rows: the row offset is part of the range-checked
    // VGPR offset, so rows at or past T (beyond num_records) are dropped by the hardware;
    // the d-block offset is the scalar offset.
    const int rowbase = qbase + qs * 32;
    const int live_rows = max(0, T_ - rowbase);
    const __amdgpu_buffer_rsrc_t dqr = __builtin_amdgcn_make_buffer_rsrc(dq_acc + (size_t)rowbase * D, (short)0,
                                                                         live_rows * D * 4, BUF_RSRC_WORD3);
#pragma unroll
    for (int j = 0; j < DBW; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(dqa[j][i], dqr, lane_off + (8 * (i >> 2) + (i & 3)) * D * 4,
                                                        (db0 + j) * 128, 0);
    }
    __syncthreads();  // dS consumed; the next tile is in the working tiles
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
        const size_t o = (size_t)key * D + db * 32 + l32;
        DK[o] = f2bf(dk[db][i] * slope);
        DV[o] = f2bf(dv[db][i]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// post: dq and the per-head sink gradient
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_post_kernel(AttnBwdParams p, size_t total, int nblk) {
  const float slope = (float)(1 << p.log2n);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const T dqs = (T)(p.dq_acc[i] * slope);       // kernel output dq_s (flash.py:592)
    reinterpret_cast<T*>(p.dq)[i] = (T)((float)dqs * p.dq_scale);  // chain rule through q_s
  }
  if (blockIdx.x == 0 && p.dbeta) {
    bool shifted = p.mode == MODE_SHIFTED;
    if (p.flag) shifted = *p.flag == 0;
    for (int hh = threadIdx.x; hh < p.H; hh += blockDim.x) {
      if (!p.sink) { p.dbeta[hh] = 0.0f; continue; }
      float s = 0.0f;
      for (int b = 0; b < p.B; ++b)
        for (int k = 0; k < nblk; ++k) s += p.sink_part[(size_t)(b * p.H + hh) * nblk + k];
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
}

template <int D>
static hipError_t launch_bwd_main_bf16(const AttnBwdParams& p, int mode, hipStream_t st) {
  dim3 grid(p.B * p.H, ceil_div(p.T, BWD_BK)), block(256);
  switch (mode) {
    case MODE_INRANGE: {
      KTimer t("attn_bwd_inrange", st);
      if (p.log2n == 4) hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_INRANGE, 4>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_INRANGE, 0>), grid, block, 0, st, p);
    } break;
    case MODE_CLIPPED: { KTimer t("attn_bwd_clipped", st); hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_CLIPPED, 0>), grid, block, 0, st, p); } break;
    case MODE_SHIFTED: { KTimer t("attn_bwd_shifted", st); hipLaunchKernelGGL((attn_bwd_bf16_kernel<D, MODE_SHIFTED, 0>), grid, block, 0, st, p); } break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_bwd_main(const AttnBwdParams& p, int mode, hipStream_t st) {
  if constexpr (sizeof(T) == 2) return launch_bwd_main_bf16<D>(p, mode, st);
  dim3 grid(p.B * p.H, ceil_div(p.T, BWD_BK)), block(256);
  switch (mode) {
    case MODE_INRANGE: {
      KTimer t("attn_bwd_inrange", st);
      if (p.log2n == 4) hipLaunchKernelGGL((attn_bwd_kernel<T, D, MODE_INRANGE, 4>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((attn_bwd_kernel<T, D, MODE_INRANGE, 0>), grid, block, 0, st, p);
    } break;
    case MODE_CLIPPED: { KTimer t("attn_bwd_clipped", st); hipLaunchKernelGGL((attn_bwd_kernel<T, D, MODE_CLIPPED, 0>), grid, block, 0, st, p); } break;
    case MODE_SHIFTED: { KTimer t("attn_bwd_shifted", st); hipLaunchKernelGGL((attn_bwd_kernel<T, D, MODE_SHIFTED, 0>), grid, block, 0, st, p); } break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int attn_bwd_sink_blocks(int T) { return ceil_div(T, PRE_ROWS); }

// modes: list of main-kernel variants to launch (each exits early unless the guard selects it).
hipError_t launch_attn_bwd(const AttnBwdParams& p, int D, bool bf16_io, const int* modes, int nmodes,
                           hipStream_t st) {
  const int nblk = attn_bwd_sink_blocks(p.T);
  dim3 pgrid(p.B * p.H, nblk);
  {
    KTimer t("attn_bwd_pre", st);
    if (bf16_io) hipLaunchKernelGGL((attn_bwd_pre_kernel<bf16>), pgrid, dim3(256), 0, st, p, D);
    else hipLaunchKernelGGL((attn_bwd_pre_kernel<float>), pgrid, dim3(256), 0, st, p, D);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  for (int m = 0; m < nmodes; ++m) {
    if (bf16_io) e = D == 64 ? launch_bwd_main<bf16, 64>(p, modes[m], st) : launch_bwd_main<bf16, 128>(p, modes[m], st);
    else e = D == 64 ? launch_bwd_main<float, 64>(p, modes[m], st) : launch_bwd_main<float, 128>(p, modes[m], st);
    if (e != hipSuccess) return e;
  }
  const size_t total = (size_t)p.B * p.H * p.T * D;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
  {
    KTimer t("attn_bwd_post", st);
    if (bf16_io) hipLaunchKernelGGL((attn_bwd_post_kernel<bf16>), dim3(blocks), dim3(256), 0, st, p, total, nblk);
    else hipLaunchKernelGGL((attn_bwd_post_kernel<float>), dim3(blocks), dim3(256), 0, st, p, total, nblk);
  }
  return hipGetLastError();
}

}  // namespace alg
