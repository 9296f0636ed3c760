// Attention prologue and range guard for gfx950 (src/algebraic/kernels/flash.py:823-849).
//
//   prep      q_s = round(q * alpha) (flash.py:833); per-workgroup maxima of ||q_s||^2,
//             ||k||^2 (f32 row sums) and |v| (flash.py:841-849). NaN propagates, so a NaN
//             input fails the guard as the reference's comparisons do.
//   finalize  one workgroup reduces the maxima, writes sink/c broadcast to (H,)
//             (flash.py:826-828) and the guard flag (1 = in range) that the forward and
//             backward kernels read on the device (the lax.cond of flash.py:853-856).
#include "launchers.h"

namespace alg {

__device__ __forceinline__ float nanmax(float a, float b) { return (a > b || a != a) ? a : b; }

// Head dim D and whether the guard maxima are wanted are fixed per launch, so the kernel
// branches once into a straight-line body: all PREP_U rows' loads are issued before any is
// waited for, and the row sums are unrolled shuffles.
template <typename T, int D, bool GUARD>
__device__ __forceinline__ void attn_prep_body(const PrepParams& p) {
  constexpr int CH = 16 / sizeof(T);
  constexpr int lpr = D / CH;               // lanes per row
  constexpr int rpw = 64 / lpr;             // rows per wave per step
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / lpr, li = lane - sub * lpr;
  float mq = 0.0f, mk = 0.0f, mv = 0.0f;
  // Each lane loads PREP_U rows before reducing any (more bytes in flight per lane).
  constexpr int PREP_U = 4;
  const size_t step = (size_t)gridDim.x * 4 * rpw;
  for (size_t r0 = ((size_t)blockIdx.x * 4 + wave) * rpw; r0 < p.rows; r0 += step * PREP_U) {
    T qv[PREP_U][CH], kv[PREP_U][CH], vv[PREP_U][CH];
#pragma unroll
    for (int u = 0; u < PREP_U; ++u) {
      const size_t r = r0 + u * step + sub;
      const size_t off = (r < p.rows ? r : p.rows - 1) * p.D + li * CH;
      *reinterpret_cast<uint4*>(qv[u]) = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.q) + off);
      if constexpr (GUARD) {
        *reinterpret_cast<uint4*>(kv[u]) = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.k) + off);
        *reinterpret_cast<uint4*>(vv[u]) = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.v) + off);
      }
    }
#pragma unroll
    for (int u = 0; u < PREP_U; ++u) {
      const size_t r = r0 + u * step + sub;
      const bool ok = r < p.rows;
      const size_t off = r * p.D + li * CH;
      float sq = 0.0f, sk = 0.0f, av = 0.0f;
      if (ok) {
        T out[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          out[j] = (T)((float)qv[u][j] * p.alpha);
          const float f = (float)out[j];
          sq += f * f;
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<T*>(p.q_s) + off) = *reinterpret_cast<uint4*>(out);
        if constexpr (GUARD) {
#pragma unroll
          for (int j = 0; j < CH; ++j) {
            const float kf = (float)kv[u][j];
            sk += kf * kf;
            av = nanmax(av, __builtin_fabsf((float)vv[u][j]));
          }
        }
      }
      // Row sums across the lanes of one row.
#pragma unroll
      for (int m = 1; m < lpr; m <<= 1) {
        sq += __shfl_xor(sq, m, 64);
        sk += __shfl_xor(sk, m, 64);
      }
      mq = nanmax(mq, sq);
      mk = nanmax(mk, sk);
      mv = nanmax(mv, av);
    }
  }
  for (int m = 32; m >= 1; m >>= 1) {
    mq = nanmax(mq, __shfl_xor(mq, m, 64));
    mk = nanmax(mk, __shfl_xor(mk, m, 64));
    mv = nanmax(mv, __shfl_xor(mv, m, 64));
  }
  __shared__ float red[4][3];
  if (lane == 0) { red[wave][0] = mq; red[wave][1] = mk; red[wave][2] = mv; }
  __syncthreads();
  if (threadIdx.x < 3) {
    float m = red[0][threadIdx.x];
    for (int w = 1; w < 4; ++w) m = nanmax(m, red[w][threadIdx.x]);
    p.part[blockIdx.x * 3 + threadIdx.x] = m;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void attn_prep_kernel(PrepParams p) {
  if (p.D == 128) {
    if (p.want_guard) attn_prep_body<T, 128, true>(p);
    else attn_prep_body<T, 128, false>(p);
  } else {
    if (p.want_guard) attn_prep_body<T, 64, true>(p);
    else attn_prep_body<T, 64, false>(p);
  }
}



__device__ __forceinline__ float wave_nanmax(float m) {
  for (int k = 32; k >= 1; k >>= 1) m = nanmax(m, __shfl_xor(m, k, 64));
  return m;
}

__global__ __launch_bounds__(256) void attn_guard_kernel(GuardParams g) {
  __shared__ float red[4][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float mq = 0.0f, mk = 0.0f, mv = 0.0f, ms = 0.0f;
  if (g.want_guard) {
    for (int i = threadIdx.x; i < g.nblocks; i += 256) {
      mq = nanmax(mq, g.part[3 * i]);
      mk = nanmax(mk, g.part[3 * i + 1]);
      mv = nanmax(mv, g.part[3 * i + 2]);
    }
  }
  for (int hh = threadIdx.x; hh < g.H; hh += 256) {
    if (g.sink_logit) {
      const float s = g.sink_logit[g.sink_count == 1 ? 0 : hh] / g.c;
      if (g.sink_out) g.sink_out[hh] = s;
      ms = nanmax(ms, __builtin_fabsf(s));
    }
  }
  mq = wave_nanmax(mq);
  mk = wave_nanmax(mk);
  mv = wave_nanmax(mv);
  ms = wave_nanmax(ms);
  if (lane == 0) { red[wave][0] = mq; red[wave][1] = mk; red[wave][2] = mv; red[wave][3] = ms; }
  __syncthreads();
  if (threadIdx.x == 0 && g.flag) {
    for (int w = 1; w < 4; ++w) {
      mq = nanmax(mq, red[w][0]);
      mk = nanmax(mk, red[w][1]);
      mv = nanmax(mv, red[w][2]);
      ms = nanmax(ms, red[w][3]);
    }
    bool ok = (mq * mk <= g.q2k2_bound) && (mv <= g.v_bound);
    if (g.sink_logit) ok = ok && (ms <= g.sink_bound);
    *g.flag = g.want_guard ? (ok ? 1 : 0) : 1;
  }
}

int attn_prep_blocks(size_t rows) {
  size_t b = (rows + 63) / 64;
  return (int)(b < 1024 ? (b ? b : 1) : 1024);
}

hipError_t launch_attn_prep(const PrepParams& p, bool bf16_io, GuardParams g, hipStream_t st) {
  const int nb = attn_prep_blocks(p.rows);
  {
    KTimer t("attn_prep", st);
    if (bf16_io) hipLaunchKernelGGL((attn_prep_kernel<bf16>), dim3(nb), dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_prep_kernel<float>), dim3(nb), dim3(256), 0, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  g.part = p.part;
  g.nblocks = nb;
  return launch_attn_guard(g, st);
}

hipError_t launch_attn_guard(const GuardParams& g, hipStream_t st) {
  {
    KTimer t("attn_guard", st);
    hipLaunchKernelGGL(attn_guard_kernel, dim3(1), dim3(256), 0, st, g);
  }
  return hipGetLastError();
}

}  // namespace alg
