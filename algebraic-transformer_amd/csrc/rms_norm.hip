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

// Row chunk c of this lane (chunk lane + 64 c), or zeros past the row's end: buffer loads over
// the row's range, which return zeros past it, so every lane loads unconditionally and the
// row's loads issue back to back under one wait (a load per lane behind a range check
// compiles to a branch and a wait around each).
template <int NC>
__device__ __forceinline__ void load_row(const bf16* r, int lane, int nch, uint4 (&raw)[NC]) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)r, (short)0, nch * 16, BUF_RSRC_WORD3);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * (lane + 64 * c), 0, 0);
    raw[c] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// Gain of this lane's chunks (1 without a gain; zeros past the row's end, where x is zero).
template <int NC>
__device__ __forceinline__ void load_gain(const float* gain, int lane, int nch, float (&g)[NC][8]) {
  if (!gain) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) g[c][e] = 1.0f;
    return;
  }
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)gain, (short)0, nch * 32, BUF_RSRC_WORD3);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int off = 32 * (lane + 64 * c);
    const auto lo = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    const auto hi = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g[c][e] = __uint_as_float(lo[e]);
      g[c][4 + e] = __uint_as_float(hi[e]);
    }
  }
}

}  // namespace

// One row per wave; NC = ceil(d / 512) chunks of 8 elements per lane, sized at compile time so
// the kernel keeps few registers and many waves (the row's loads) in flight.
template <int NC>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(RmsNormParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
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

// Rows in a grid-stride loop, one row per wave at a time (the gain gradient is a
// per-workgroup partial). The gain sits in LDS and the per-element values (x, dy, a = g dy)
// are formed again from the raw row for the output, so a wave holds only its row's raw
// chunks and its gain-gradient accumulators: about 100 registers at d = 2048, four waves
// per SIMD, whose row loads keep enough bytes in flight without a software prefetch.
template <int NC>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(RmsNormParams p) {
  __shared__ __attribute__((aligned(16))) float gs[NC * 512];
  __shared__ float red[NC * 512];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nch = p.d / 8;
  {
    float g[NC][8];  // chunk lane + 64 c of the gain, as the rows are laid out
    load_gain<NC>(p.gain, lane, nch, g);
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) gs[8 * (lane + 64 * c) + e] = g[c][e];
    }
  }
  __syncthreads();
  float acc[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[c][e] = 0.0f;
  const float inv_d = 1.0f / (float)p.d;
  const int stride = gridDim.x * 4;
  for (int row = blockIdx.x * 4 + wave; row < p.rows; row += stride) {
    uint4 xr[NC], dyr[NC];
    load_row<NC>(p.x + (size_t)row * p.d, lane, nch, xr);
    load_row<NC>(p.dy + (size_t)row * p.d, lane, nch, dyr);
    const float tau = p.tau[row];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8], dy[8];
      cvt8(xr[c], x);
      cvt8(dyr[c], dy);
      const float* g = gs + 8 * (lane + 64 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[c][e] += __fmul_rn(dy[e], __fmul_rn(x[e], tau));
        s += __fmul_rn(__fmul_rn(g[e], dy[e]), x[e]);
      }
      __builtin_amdgcn_sched_barrier(0);  // one chunk's temporaries live at a time
    }
    s = wave_sum(s);
    const float coef = __fmul_rn(__fmul_rn(__fmul_rn(tau, tau), tau), s) * inv_d;
    bf16* dxr = p.dx + (size_t)row * p.d;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      // Re-convert from the raw chunks (keeping the converted values live across the row sum
      // would double the registers).
      asm volatile("" : "+v"(xr[c].x), "+v"(xr[c].y), "+v"(xr[c].z), "+v"(xr[c].w));
      asm volatile("" : "+v"(dyr[c].x), "+v"(dyr[c].y), "+v"(dyr[c].z), "+v"(dyr[c].w));
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        float x[8], dy[8];
        cvt8(xr[c], x);
        cvt8(dyr[c], dy);
        const float* g = gs + 8 * ch;
        bf16 out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          out[e] = f2bf(__fsub_rn(__fmul_rn(__fmul_rn(g[e], dy[e]), tau), __fmul_rn(x[e], coef)));
        *reinterpret_cast<uint4*>(dxr + 8 * ch) = *reinterpret_cast<uint4*>(out);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (!p.gpart) return;
  // The workgroup's partial: the waves' accumulators added in wave order.
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int ch = lane + 64 * c;
        if (ch < nch) {
#pragma unroll
          for (int e = 0; e < 8; ++e) red[8 * ch + e] = w == 0 ? acc[c][e] : red[8 * ch + e] + acc[c][e];
        }
      }
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < p.d; i += 256) p.gpart[(size_t)blockIdx.x * p.d + i] = red[i];  // row per block
}

// dgain[i] = sum over blocks of gpart[block][i], in two fixed-order stages with a thread per
// column (coalesced rows): the blocks in groups of RN_GROUP summed in block order into
// tmp[group][i], then the groups in group order (at most RN_GROUP groups: 1024 blocks).
// Each stage issues its RN_GROUP loads together (rows past the end are read clamped and not
// added) and then sums them in order.
constexpr int RN_GROUP = 32;
__device__ __forceinline__ float rn_sum_rows(const float* a, int r0, int r1, int d, int i) {
  float v[RN_GROUP];
#pragma unroll
  for (int k = 0; k < RN_GROUP; ++k) v[k] = a[(size_t)min(r0 + k, r1 - 1) * d + i];
  float s = v[0];
#pragma unroll
  for (int k = 1; k < RN_GROUP; ++k)
    if (r0 + k < r1) s += v[k];
  return s;
}
__global__ __launch_bounds__(256) void rms_norm_gain_part_kernel(const float* gpart, int nblocks, int d, float* tmp) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= d) return;
  const int b0 = blockIdx.y * RN_GROUP;
  tmp[(size_t)blockIdx.y * d + i] = rn_sum_rows(gpart, b0, min(nblocks, b0 + RN_GROUP), d, i);
}

__global__ __launch_bounds__(256) void rms_norm_gain_reduce_kernel(const float* tmp, int ngroups, int d, float* dgain) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= d) return;
  dgain[i] = rn_sum_rows(tmp, 0, ngroups, d, i);
}

int rms_norm_max_d() { return RN_MAXC * 512; }
int rms_norm_blocks(int rows) { return rows / 4 + 1 < 1024 ? rows / 4 + 1 : 1024; }
int rms_norm_gain_groups(int rows) { return (rms_norm_blocks(rows) + RN_GROUP - 1) / RN_GROUP; }
static_assert(1024 <= RN_GROUP * RN_GROUP, "the groups of the largest grid fit one second stage");

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
  // Workspace: gpart (nb rows of d) then, 256-byte aligned, the group sums (ngroups rows of d).
  const int ng = rms_norm_gain_groups(p.rows);
  float* tmp = p.gpart + ((size_t)nb * p.d + 63) / 64 * 64;
  KTimer t("rms_norm_gain_reduce", st);
  hipLaunchKernelGGL(rms_norm_gain_part_kernel, dim3((p.d + 255) / 256, ng), dim3(256), 0, st, p.gpart, nb, p.d, tmp);
  hipLaunchKernelGGL(rms_norm_gain_reduce_kernel, dim3((p.d + 255) / 256), dim3(256), 0, st, tmp, ng, p.d, dgain);
  return hipGetLastError();
}

}  // namespace alg
