// Row RMS normalisation with a learned gain for gfx950: the model's final norm before the
// head (src/algebraic/model.py:208, rms_norm at src/algebraic/algebraic.py:76-83) and its VJP.
//
// One wave per row of d elements: lane l holds the 16-byte chunks l, l + 64, ... (d/8 chunks
// per row, d a multiple of 8, at most RN_MAXC * 512 elements); the row's sum of squares is a
// wave reduction. Forward: tau = 1/sqrt(mean(x^2) + eps) (f32), y = round((x tau) g), tau kept
// for the VJP. VJP (JAX autodiff of the same expression, in f32): a = g dy,
// dx = round(a tau - x tau^3 sum(a x) / d); dgain = sum over rows of dy x tau, as per-workgroup
// partials (the workgroup's waves summed in order) reduced per column in block order.
#include "launchers.h"

#pragma clang fp contract(off)

namespace alg {

namespace {

constexpr int RN_MAXC = 8;  // 16-byte chunks per lane: d <= 4096

template <typename T>
__device__ __forceinline__ void cvt8(const uint4& raw, float (&x)[8]) {
  if constexpr (sizeof(T) == 2) {
    bf16 v[8];
    *reinterpret_cast<uint4*>(v) = raw;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
  }
}

__device__ __forceinline__ float wave_sum(float s) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s += __shfl_xor(s, m, 64);
  return s;
}

}  // namespace

__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(RmsNormParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.d / 8;
  float g[RN_MAXC][8];
#pragma unroll
  for (int c = 0; c < RN_MAXC; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < 8; ++e) g[c][e] = (ch < nch && p.gain) ? p.gain[8 * ch + e] : 1.0f;
  }
  const float inv_d = 1.0f / (float)p.d;
  for (int row = blockIdx.x * 4 + wave; row < p.rows; row += gridDim.x * 4) {
    const bf16* xr = p.x + (size_t)row * p.d;
    float x[RN_MAXC][8];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < RN_MAXC; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        cvt8<bf16>(*reinterpret_cast<const uint4*>(xr + 8 * ch), x[c]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[c][e] * x[c][e];
      }
    }
    ss = wave_sum(ss);
    const float tau = 1.0f / sqrtf(ss * inv_d + p.eps);
    bf16* yr = p.y + (size_t)row * p.d;
#pragma unroll
    for (int c = 0; c < RN_MAXC; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        bf16 out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = f2bf(__fmul_rn(__fmul_rn(x[c][e], tau), g[c][e]));
        *reinterpret_cast<uint4*>(yr + 8 * ch) = *reinterpret_cast<uint4*>(out);
      }
    }
    if (lane == 0) p.tau[row] = tau;
  }
}

__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(RmsNormParams p) {
  __shared__ float red[4][RN_MAXC * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.d / 8;
  float g[RN_MAXC][8], acc[RN_MAXC][8];
#pragma unroll
  for (int c = 0; c < RN_MAXC; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      g[c][e] = (ch < nch && p.gain) ? p.gain[8 * ch + e] : 1.0f;
      acc[c][e] = 0.0f;
    }
  }
  const float inv_d = 1.0f / (float)p.d;
  for (int row = blockIdx.x * 4 + wave; row < p.rows; row += gridDim.x * 4) {
    const bf16* xr = p.x + (size_t)row * p.d;
    const bf16* dyr = p.dy + (size_t)row * p.d;
    const float tau = p.tau[row];
    float x[RN_MAXC][8], a[RN_MAXC][8];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < RN_MAXC; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        float dy[8];
        cvt8<bf16>(*reinterpret_cast<const uint4*>(xr + 8 * ch), x[c]);
        cvt8<bf16>(*reinterpret_cast<const uint4*>(dyr + 8 * ch), dy);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[c][e] += __fmul_rn(dy[e], __fmul_rn(x[c][e], tau));
          a[c][e] = __fmul_rn(g[c][e], dy[e]);
          s += __fmul_rn(a[c][e], x[c][e]);
        }
      }
    }
    s = wave_sum(s);
    const float coef = __fmul_rn(__fmul_rn(__fmul_rn(tau, tau), tau), s) * inv_d;
    bf16* dxr = p.dx + (size_t)row * p.d;
#pragma unroll
    for (int c = 0; c < RN_MAXC; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        bf16 out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = f2bf(__fsub_rn(__fmul_rn(a[c][e], tau), __fmul_rn(x[c][e], coef)));
        *reinterpret_cast<uint4*>(dxr + 8 * ch) = *reinterpret_cast<uint4*>(out);
      }
    }
  }
  if (!p.gpart) return;
#pragma unroll
  for (int c = 0; c < RN_MAXC; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][8 * ch + e] = acc[c][e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < p.d; i += 256)
    p.gpart[(size_t)i * gridDim.x + blockIdx.x] = red[0][i] + red[1][i] + red[2][i] + red[3][i];
}

// dgain[i] = sum over blocks of gpart[i][block], one workgroup per column, fixed-order tree.
__global__ __launch_bounds__(256) void rms_norm_gain_reduce_kernel(const float* gpart, int nblocks, float* dgain) {
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
  if (threadIdx.x == 0) dgain[i] = red[0];
}

int rms_norm_max_d() { return RN_MAXC * 512; }
int rms_norm_blocks(int rows) { return rows / 4 + 1 < 1024 ? rows / 4 + 1 : 1024; }

hipError_t launch_rms_norm_fwd(const RmsNormParams& p, hipStream_t st) {
  KTimer t("rms_norm_fwd", st);
  hipLaunchKernelGGL(rms_norm_fwd_kernel, dim3(rms_norm_blocks(p.rows)), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_rms_norm_bwd(const RmsNormParams& p, float* dgain, hipStream_t st) {
  const int nb = rms_norm_blocks(p.rows);
  {
    KTimer t("rms_norm_bwd", st);
    hipLaunchKernelGGL(rms_norm_bwd_kernel, dim3(nb), dim3(256), 0, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dgain) return e;
  KTimer t("rms_norm_gain_reduce", st);
  hipLaunchKernelGGL(rms_norm_gain_reduce_kernel, dim3(p.d), dim3(256), 0, st, p.gpart, nb, dgain);
  return hipGetLastError();
}

}  // namespace alg
