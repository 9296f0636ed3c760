// Row RMS normalisation with a learned gain for gfx950: the model's final norm before the
// head (src/algebraic/model.py:208, rms_norm at src/algebraic/algebraic.py:76-83) and its VJP.
//
// One wave per row of d elements: lane l holds the 16-byte chunks l, l + 64, ... (d/8 chunks
// per row, d a multiple of 8, at most RN_MAXC * 512 elements; the kernels are instantiated per
// chunk count so registers and LDS are sized to the width); the row's sum of squares is a
// wave reduction. Forward: tau = 1/sqrt(mean(x^2) + eps) (f32), y = round((x tau) g), tau kept
// for the VJP. VJP (JAX autodiff of the same expression, in f32): a = g dy,
// dx = round(a tau - x tau^3 sum(a x) / d); dgain = sum over rows of dy x tau, as per-workgroup
// partials (the workgroup's waves summed in order) reduced per column in block order.
#include "launchers.h"

#pragma clang fp contract(off)

namespace alg {

namespace {

constexpr int RN_MAXC = 8;  // 16-byte chunks per lane: d <= 4096

__device__ __forceinline__ void cvt8(const uint4& raw, float (&x)[8]) {
  bf16 v[8];
  *reinterpret_cast<uint4*>(v) = raw;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}

__device__ __forceinline__ float wave_sum(float s) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s += __shfl_xor(s, m, 64);
  return s;
}

// Row chunk c of this lane (chunk lane + 64 c), or zeros past the row's end.
template <int NC>
__device__ __forceinline__ void load_row(const bf16* r, int lane, int nch, uint4 (&raw)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
    raw[c] = ch < nch ? *reinterpret_cast<const uint4*>(r + 8 * ch) : make_uint4(0, 0, 0, 0);
  }
}

template <int NC>
__device__ __forceinline__ void load_gain(const float* gain, int lane, int nch, float (&g)[NC][8]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < 8; ++e) g[c][e] = (ch < nch && gain) ? gain[8 * ch + e] : 1.0f;
  }
}

}  // namespace

// One row per wave; NC = ceil(d / 512) chunks of 8 elements per lane, sized at compile time so
// the kernel keeps few registers and many waves (the row's loads) in flight.
template <int NC>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(RmsNormParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int nch = p.d / 8;
  uint4 raw[NC];
  load_row<NC>(p.x + (size_t)row * p.d, lane, nch, raw);
  float g[NC][8];
  load_gain<NC>(p.gain, lane, nch, g);
  float x[NC][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    cvt8(raw[c], x[c]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[c][e] * x[c][e];
  }
  ss = wave_sum(ss);
  const float tau = 1.0f / sqrtf(ss * (1.0f / (float)p.d) + p.eps);
  bf16* yr = p.y + (size_t)row * p.d;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
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

// Rows in a grid-stride loop (the gain gradient is a per-workgroup partial); the next row's
// x and dy are loaded while the current one is reduced and written.
template <int NC>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(RmsNormParams p) {
  __shared__ float red[4][NC * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = p.d / 8;
  float g[NC][8], acc[NC][8];
  load_gain<NC>(p.gain, lane, nch, g);
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[c][e] = 0.0f;
  const float inv_d = 1.0f / (float)p.d;
  const int stride = gridDim.x * 4;
  int row = blockIdx.x * 4 + wave;
  uint4 xr[NC], dyr[NC];
  if (row < p.rows) {
    load_row<NC>(p.x + (size_t)row * p.d, lane, nch, xr);
    load_row<NC>(p.dy + (size_t)row * p.d, lane, nch, dyr);
  }
  for (; row < p.rows; row += stride) {
    const float tau = p.tau[row];
    float x[NC][8], a[NC][8];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float dy[8];
      cvt8(xr[c], x[c]);
      cvt8(dyr[c], dy);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[c][e] += __fmul_rn(dy[e], __fmul_rn(x[c][e], tau));
        a[c][e] = __fmul_rn(g[c][e], dy[e]);
        s += __fmul_rn(a[c][e], x[c][e]);
      }
    }
    const int next = row + stride;
    if (next < p.rows) {
      load_row<NC>(p.x + (size_t)next * p.d, lane, nch, xr);
      load_row<NC>(p.dy + (size_t)next * p.d, lane, nch, dyr);
    }
    s = wave_sum(s);
    const float coef = __fmul_rn(__fmul_rn(__fmul_rn(tau, tau), tau), s) * inv_d;
    bf16* dxr = p.dx + (size_t)row * p.d;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
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
  for (int c = 0; c < NC; ++c) {
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

// Chunks per lane for width d: ceil(d / 512), 1..RN_MAXC (the width is checked by the caller).
static int rms_norm_nc(int d) { return (d / 8 + 63) / 64; }

#define RN_DISPATCH(KERNEL, GRID, ...)                                                          \
  switch (rms_norm_nc(p.d)) {                                                                 \
    case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 3: hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 4: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 5: hipLaunchKernelGGL(KERNEL<5>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 6: hipLaunchKernelGGL(KERNEL<6>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    case 7: hipLaunchKernelGGL(KERNEL<7>, GRID, dim3(256), 0, st, __VA_ARGS__); break;         \
    default: hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(256), 0, st, __VA_ARGS__); break;        \
  }

hipError_t launch_rms_norm_fwd(const RmsNormParams& p, hipStream_t st) {
  KTimer t("rms_norm_fwd", st);
  RN_DISPATCH(rms_norm_fwd_kernel, dim3((p.rows + 3) / 4), p);
  return hipGetLastError();
}

hipError_t launch_rms_norm_bwd(const RmsNormParams& p, float* dgain, hipStream_t st) {
  const int nb = rms_norm_blocks(p.rows);
  {
    KTimer t("rms_norm_bwd", st);
    RN_DISPATCH(rms_norm_bwd_kernel, dim3(nb), p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dgain) return e;
  KTimer t("rms_norm_gain_reduce", st);
  hipLaunchKernelGGL(rms_norm_gain_reduce_kernel, dim3(p.d), dim3(256), 0, st, p.gpart, nb, dgain);
  return hipGetLastError();
}

}  // namespace alg
