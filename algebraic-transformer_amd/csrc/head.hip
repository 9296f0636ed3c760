// Fused tied-embedding algebraic likelihood head for gfx950.
//
// Replaces src/algebraic/kernels/fused_head.py:72-275 (forward statistics, telemetry,
// backward) including the XLA embedding-gradient matmul of fused_head.py:215.
//
// Forward (logits never stored):
//   z^T tile = E h^T per 128 vocab x 128 token tile (bf16 MFMA, f32 acc); epilogue
//   x = min(z/c, X), w = rho_fast(x)^n, per-token partial sums of w for this vocab tile,
//   and the target logit zt (fused_head.py:83-103). A statistics kernel reduces the
//   partials in a fixed order: stat = l^(-1/n) (fused_head.py:116), telemetry
//   pt = (rho(min(zt/c, X)) stat)^n and the objective mean(1 - pt) (fused_head.py:219-229).
// Backward:
//   the same tile product recomputes z; epilogue dz = s (p - y) r with p = (rho stat)^n,
//   s = g (n/c) / N, rounded to bf16 (fused_head.py:128-146) and stored vocab-major
//   (dZ^T, V x Npad) in a caller workspace; then dh = dZ E and dE = dZ^T h are two
//   bf16 MFMA GEMMs reading dZ^T and E/h in place (fused_head.py:147, 215).
#include "gemm_core.h"
#include "head_params.h"

namespace alg {



__global__ void head_zero_kernel(float* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// z^T = E h^T tile with the forward epilogue.
__global__ __launch_bounds__(256, 2) void head_fwd_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmSmem<KMAJOR, KMAJOR> sm;
  __shared__ float red[2][GT_N];
  const int m0 = blockIdx.y * GT_M;  // vocab
  const int n0 = blockIdx.x * GT_N;  // tokens
  GemmOperand A{p.E, p.d, p.V}, B{p.h, p.d, p.N};
  floatx16 acc[2][2];
  gemm_mainloop<KMAJOR, KMAJOR>(sm, A, B, m0, n0, p.d, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, l32 = lane & 31;
  const int log2n = p.log2n;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int col = wn * 64 + nb * 32 + l32;
    const int tok = n0 + col;
    const int tgt = tok < p.N ? p.targets[tok] : -1;
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = m0 + wm * 64 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        const float z = acc[mb][nb][i];
        const float x = fminf(z * p.inv_c, p.clamp);
        float t = rho_fast(x);
        for (int e = 0; e < log2n; ++e) t = t * t;
        if (v < p.V) part += t;
        if (v == tgt) p.zt[tok] = z;
      }
    }
    part += xor32(part);
    if (h == 0) red[wm][col] = part;
  }
  __syncthreads();
  if (threadIdx.x < GT_N) {
    const int tok = n0 + threadIdx.x;
    if (tok < p.N) p.partial[(size_t)blockIdx.y * p.N + tok] = red[0][threadIdx.x] + red[1][threadIdx.x];
  }
}

// Per-token statistics and telemetry (fused_head.py:116-117, 219-229).
__global__ __launch_bounds__(256) void head_stats_kernel(HeadParams p, int nvt) {
  __shared__ float red[256];
  const int tok = blockIdx.x * 256 + threadIdx.x;
  float miss = 0.0f;
  if (tok < p.N) {
    float l = 0.0f;
    for (int t = 0; t < nvt; ++t) l += p.partial[(size_t)t * p.N + tok];
    const int n = 1 << p.log2n;
    const float st = inv_root(l, n);
    p.stat[tok] = st;
    const float x = fminf(p.zt[tok] / p.c, p.clamp);
    const float pt = ipow_rt(rho_exact(x) * st, n);
    p.pt[tok] = pt;
    miss = 1.0f - pt;
  }
  red[threadIdx.x] = miss;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) p.obj_part[blockIdx.x] = red[0];
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

// z^T recomputed with the backward epilogue: dZ^T = bf16(s (p - y) r).
__global__ __launch_bounds__(256, 2) void head_dz_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmSmem<KMAJOR, KMAJOR> sm;
  const int m0 = blockIdx.y * GT_M;
  const int n0 = blockIdx.x * GT_N;
  GemmOperand A{p.E, p.d, p.V}, B{p.h, p.d, p.N};
  floatx16 acc[2][2];
  gemm_mainloop<KMAJOR, KMAJOR>(sm, A, B, m0, n0, p.d, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, l32 = lane & 31;
  const int log2n = p.log2n;
  const float scale = p.g[0] * ((float)(1 << log2n) * p.inv_c) / (float)p.N;  // fused_head.py:251
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int tok = n0 + wn * 64 + nb * 32 + l32;
    const bool live = tok < p.N;
    const int tgt = live ? p.targets[tok] : -1;
    const float st = live ? p.stat[tok] : 0.0f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = m0 + wm * 64 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (v >= p.V) continue;
        const float x = fminf(acc[mb][nb][i] * p.inv_c, p.clamp);
        float r;
        float t = rho_fast(x, r) * st;
        for (int e = 0; e < log2n; ++e) t = t * t;
        const float y = (v == tgt) ? 1.0f : 0.0f;
        const float dz = live ? (t - y) * r * scale : 0.0f;
        p.dzt[(size_t)v * p.Npad + tok] = f2bf(dz);
      }
    }
  }
}

// dh = dZ E: A = dZ^T stored [v][n] (m-contiguous), B = E stored [v][d] (n-contiguous).
__global__ __launch_bounds__(256, 2) void head_dh_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmSmem<MNMAJOR, MNMAJOR> sm;
  const int m0 = blockIdx.y * GT_M;  // tokens
  const int n0 = blockIdx.x * GT_N;  // d
  GemmOperand A{p.dzt, p.Npad, p.V}, B{p.E, p.d, p.V};
  floatx16 acc[2][2];
  gemm_mainloop<MNMAJOR, MNMAJOR>(sm, A, B, m0, n0, p.V, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int col = n0 + wn * 64 + nb * 32 + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tok = m0 + wm * 64 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (tok < p.N) p.dh[(size_t)tok * p.d + col] = f2bf(acc[mb][nb][i]);
      }
    }
}

// dE = dZ^T h: A = dZ^T stored [v][n] (k-contiguous), B = h stored [n][d] (n-contiguous).
__global__ __launch_bounds__(256, 2) void head_de_kernel(HeadParams p) {
  __shared__ __attribute__((aligned(16))) GemmSmem<KMAJOR, MNMAJOR> sm;
  const int m0 = blockIdx.y * GT_M;  // vocab
  const int n0 = blockIdx.x * GT_N;  // d
  GemmOperand A{p.dzt, p.Npad, p.V}, B{p.h, p.d, p.N};
  floatx16 acc[2][2];
  gemm_mainloop<KMAJOR, MNMAJOR>(sm, A, B, m0, n0, p.N, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int col = n0 + wn * 64 + nb * 32 + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = m0 + wm * 64 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (v < p.V) {
          const size_t o = (size_t)v * p.d + col;
          if (p.dE_f32) reinterpret_cast<float*>(p.dE)[o] = acc[mb][nb][i];
          else reinterpret_cast<bf16*>(p.dE)[o] = f2bf(acc[mb][nb][i]);
        }
      }
    }
}

int head_vocab_tiles(int V) { return (V + GT_M - 1) / GT_M; }
int head_token_tiles(int N) { return (N + GT_N - 1) / GT_N; }
int head_stat_blocks(int N) { return (N + 255) / 256; }

hipError_t launch_head_fwd(const HeadParams& p, hipStream_t st) {
  { KTimer t("head_zero", st); hipLaunchKernelGGL(head_zero_kernel, dim3((p.N + 255) / 256), dim3(256), 0, st, p.zt, p.N); }
  dim3 grid(head_token_tiles(p.N), head_vocab_tiles(p.V));
  { KTimer t("head_fwd", st); hipLaunchKernelGGL(head_fwd_kernel, grid, dim3(256), 0, st, p); }
  const int nb = head_stat_blocks(p.N);
  { KTimer t("head_stats", st); hipLaunchKernelGGL(head_stats_kernel, dim3(nb), dim3(256), 0, st, p, head_vocab_tiles(p.V)); }
  { KTimer t("head_obj", st); hipLaunchKernelGGL(head_obj_kernel, dim3(1), dim3(256), 0, st, p, nb); }
  return hipGetLastError();
}

hipError_t launch_head_bwd(const HeadParams& p, hipStream_t st) {
  dim3 g1(p.Npad / GT_N, head_vocab_tiles(p.V));
  { KTimer t("head_dz", st); hipLaunchKernelGGL(head_dz_kernel, g1, dim3(256), 0, st, p); }
  dim3 g2(p.d / GT_N, head_token_tiles(p.N));
  { KTimer t("head_dh", st); hipLaunchKernelGGL(head_dh_kernel, g2, dim3(256), 0, st, p); }
  dim3 g3(p.d / GT_N, head_vocab_tiles(p.V));
  { KTimer t("head_de", st); hipLaunchKernelGGL(head_de_kernel, g3, dim3(256), 0, st, p); }
  return hipGetLastError();
}

}  // namespace alg
