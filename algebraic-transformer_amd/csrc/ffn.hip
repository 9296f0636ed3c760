// ALU-GLU feed-forward for gfx950: the activation and its VJP fused into the epilogues of the
// products that produce and consume it (src/algebraic/model.py:185-193, ffn = "alu_glu";
// alu and its custom VJP: src/algebraic/algebraic.py:86-113).
//
// Forward: [gate | up] = h2 [w_g | w_u] as one product over the concatenated weights (a split
// operand: each wave's two 32-column blocks are the same columns f of w_g and of w_u), and the
// epilogue forms gate = round(.), up = round(.), act = alu(up), y = round(gate act); it stores
// y for the output product and gate, up for the backward.
// Backward: dy = round(dout w_d^T) with the epilogue forming d_gate = round(dy act),
// d_act = round(dy gate), d_up = round(d_act (0.5 (1 + u) + 0.5 u r^2)) (u, r recomputed from
// up), stored as one (N, 2F) matrix [d_gate | d_up] so dh2 and [dw_g | dw_u] are one product
// each. The remaining products (y w_d, dh2, the weight gradients) are plain GEMMs.
#include <cmath>

#include "gemm_core.h"
#include "head_params.h"
#include "launchers.h"

#pragma clang fp contract(off)

namespace alg {

typedef HeadGemm FC;  // 256 x 256 tiles, 8 waves (2 x 4)
constexpr int FNT = FC::THREADS;

namespace {

// alu(z) with the reference's negative-tail form; u, r returned for the derivative
// (algebraic.py:84-91). r is the hardware reciprocal square root, as the reference's
// lax.rsqrt; the tail's r^2 / (1 - u) (1 - u in (1, 2)) is a reciprocal multiply, within
// 2 ulp of the f32 quotient before the result is rounded to bf16. An IEEE sqrt and two IEEE
// divisions here cost about three times the VALU of the rest of the epilogue.
__device__ __forceinline__ float alu_f32(float z, float beta, float& u, float& r) {
  const float bz = __fmul_rn(beta, z);
  r = rsq(__fadd_rn(1.0f, __fmul_rn(bz, bz)));
  u = __fmul_rn(bz, r);
  const float one_plus_u =
      bz < 0.0f ? __fmul_rn(__fmul_rn(r, r), __builtin_amdgcn_rcpf(__fsub_rn(1.0f, u))) : __fadd_rn(1.0f, u);
  return __fmul_rn(__fmul_rn(0.5f, z), one_plus_u);
}

__device__ __forceinline__ float rb(float x) { return (float)f2bf(x); }

// Each wave stages its 128 x 64 block of bf16 values in its own 16 KiB share of the (idle)
// pipeline buffers, rows of 8 16-byte chunks XOR-swizzled by the row, so the accumulator's
// column-per-lane writes spread over the banks and the 16-byte row reads stay aligned; the
// global loads and stores of the epilogue then move 8 consecutive columns per lane.
__device__ __forceinline__ int stage_at(int r, int c) { return r * 64 + ((((c >> 3) ^ (r & 7)) & 7) << 3) + (c & 7); }

template <class Stage>
__device__ __forceinline__ bf16* wave_stage(Stage& s0, Stage& s1, int wm, int wn) {
  static_assert(FC::WM * FC::WN == 8 && FC::WTM == 128 && FC::WTN == 64, "staging assumes 8 waves of 128 x 64");
  static_assert(sizeof(Stage) >= 4 * 128 * 64 * sizeof(bf16), "a stage holds four waves' blocks");
  const int wi = wm * FC::WN + wn;  // 8 waves: 0..3 in s0, 4..7 in s1
  return reinterpret_cast<bf16*>(wi < 4 ? static_cast<void*>(&s0) : static_cast<void*>(&s1)) + (wi & 3) * 128 * 64;
}

}  // namespace

__global__ __launch_bounds__(FNT, 1) void ffn_gate_up_kernel(FfnParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, MNMAJOR, FC> s0, s1;
  const int nbm = (p.N + HT_M - 1) / HT_M, nbn = 2 * p.F / HT_N;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * HT_M, n0 = tn * HT_N;  // tokens, logical [gate | up] columns
  GemmOperand A{p.h2, p.d, p.N, p.d, (long)p.N * p.d};
  GemmOperand B{p.w_gu, 2L * p.F, p.d, 2 * p.F, 2L * p.d * p.F, (long)p.F};
  floatx16 acc[FC::MB][FC::NB];
  gemm_mainloop<KMAJOR, MNMAJOR, FC>(s0, s1, A, B, m0, n0, 0, p.d, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<FC>(wm, wn);
  // acc[.][0] is gate column f0 + l32, acc[.][1] up column f0 + l32 (f0 = n0/2 + 32 wn).
  __syncthreads();  // every wave is done reading the pipeline buffers
  bf16* stg = wave_stage(s0, s1, wm, wn);  // [row][0..31] gate, [row][32..63] up
#pragma unroll
  for (int mb = 0; mb < FC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      stg[stage_at(row, l32)] = f2bf(acc[mb][0][i]);
      stg[stage_at(row, 32 + l32)] = f2bf(acc[mb][1][i]);
    }
  }
  // 128 rows x 4 chunks of 8 columns: lane -> (row, chunk).
  const int f0 = n0 / 2 + wn * 32;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int idx = it * 64 + lane, row = idx >> 2, ch = idx & 3;
    const int tok = m0 + wm * FC::WTM + row;
    const bf16x8 gv = *reinterpret_cast<const bf16x8*>(stg + stage_at(row, 8 * ch));
    const bf16x8 uv = *reinterpret_cast<const bf16x8*>(stg + stage_at(row, 32 + 8 * ch));
    bf16x8 yv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float u, r;
      const float act = rb(alu_f32((float)uv[e], p.beta, u, r));
      yv[e] = f2bf(__fmul_rn((float)gv[e], act));
    }
    if (tok < p.N) {
      const size_t o = (size_t)tok * p.F + f0 + 8 * ch;
      *reinterpret_cast<bf16x8*>(p.y + o) = yv;
      *reinterpret_cast<bf16x8*>(p.gate + o) = gv;
      *reinterpret_cast<bf16x8*>(p.up + o) = uv;
    }
  }
}

__global__ __launch_bounds__(FNT, 1) void ffn_dy_kernel(FfnParams p) {
  __shared__ __attribute__((aligned(16))) GemmStage<KMAJOR, KMAJOR, FC> s0, s1;
  const int nbm = (p.N + HT_M - 1) / HT_M, nbn = (p.F + HT_N - 1) / HT_N;
  int tm, tn;
  xcd_tile(blockIdx.x, nbm, nbn, tm, tn);
  const int m0 = tm * HT_M, n0 = tn * HT_N;  // tokens, columns f
  GemmOperand A{p.dout, p.dm, p.N, p.dm, (long)p.N * p.dm};
  GemmOperand B{p.w_d, p.dm, p.F, p.dm, (long)p.F * p.dm};  // w_d (F, dm): [f][k]
  floatx16 acc[FC::MB][FC::NB];
  gemm_mainloop<KMAJOR, KMAJOR, FC>(s0, s1, A, B, m0, n0, 0, p.dm, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<FC>(wm, wn);
  __syncthreads();  // every wave is done reading the pipeline buffers
  bf16* stg = wave_stage(s0, s1, wm, wn);  // this wave's dy block, [row][0..63]
#pragma unroll
  for (int mb = 0; mb < FC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
#pragma unroll
      for (int nb = 0; nb < FC::NB; ++nb) stg[stage_at(row, nb * 32 + l32)] = f2bf(acc[mb][nb][i]);
    }
  }
  // 128 rows x 8 chunks of 8 columns: lane -> (row, chunk), in groups of GRP chunks per lane
  // whose gate/up loads are issued together (out-of-range chunks read chunk 0 and are not
  // stored): behind a per-chunk range check each load got a branch and a wait of its own.
  const int f0 = n0 + wn * FC::WTN;
  constexpr int GRP = 8;
#pragma unroll 1
  for (int g0 = 0; g0 < 16; g0 += GRP) {
    bf16x8 gvs[GRP], uvs[GRP];
#pragma unroll
    for (int k = 0; k < GRP; ++k) {
      const int idx = (g0 + k) * 64 + lane, row = idx >> 3, ch = idx & 7;
      const int tok = m0 + wm * FC::WTM + row, f = f0 + 8 * ch;
      const size_t o = tok < p.N && f < p.F ? (size_t)tok * p.F + f : 0;
      gvs[k] = *reinterpret_cast<const bf16x8*>(p.gate + o);
      uvs[k] = *reinterpret_cast<const bf16x8*>(p.up + o);
    }
#pragma unroll
    for (int k = 0; k < GRP; ++k) asm volatile("" : "+v"(gvs[k]), "+v"(uvs[k]));  // loads before the checks
#pragma unroll
  for (int k = 0; k < GRP; ++k) {
    const int idx = (g0 + k) * 64 + lane, row = idx >> 3, ch = idx & 7;
    const int tok = m0 + wm * FC::WTM + row, f = f0 + 8 * ch;
    if (tok >= p.N || f >= p.F) continue;  // F is a multiple of 128: chunks are whole
    const bf16x8 dyv = *reinterpret_cast<const bf16x8*>(stg + stage_at(row, 8 * ch));
    const bf16x8 gv = gvs[k], uv = uvs[k];
    bf16x8 dg, du;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float dy = (float)dyv[e];
      float u, r;
      const float act = rb(alu_f32((float)uv[e], p.beta, u, r));
      const float d_act = rb(__fmul_rn(dy, (float)gv[e]));
      const float deriv = __fadd_rn(__fmul_rn(0.5f, __fadd_rn(1.0f, u)), __fmul_rn(__fmul_rn(0.5f, u), __fmul_rn(r, r)));
      dg[e] = f2bf(__fmul_rn(dy, act));
      du[e] = f2bf(__fmul_rn(d_act, deriv));
    }
    const size_t od = (size_t)tok * 2 * p.F + f;
    *reinterpret_cast<bf16x8*>(p.d_gu + od) = dg;
    *reinterpret_cast<bf16x8*>(p.d_gu + od + p.F) = du;
  }
  }
}

// Plain products of the block (model.py:185-193: y w_d in the forward; [d_gate | d_up] [w_g |
// w_u]^T, h2^T [d_gate | d_up] and y^T dout in the backward): C = A B, one rounding to bf16 of
// the f32 sum, each operand read in its stored layout (AM, BM), so no transposed copy is made.
// Workgroups below g.full compute whole tiles, row-major inside each XCD's share; the rest
// compute k range (id - full) % split of tile full + (id - full) / split into an f32 tile of
// g.part, which ffn_gemm_tail_kernel sums in range order (ffn_gemm_plan).
template <int AM, int BM>
__global__ __launch_bounds__(FNT, 1) void ffn_gemm_kernel(FfnGemmParams g) {
  __shared__ __attribute__((aligned(16))) GemmStage<AM, BM, FC> s0, s1;
  const int nbn = (g.N + HT_N - 1) / HT_N;
  const int bid = blockIdx.x;
  int lin, kbeg = 0, kend = g.K, unit = -1;
  if (bid < g.full) {
    lin = g.full % 8 == 0 ? (bid % 8) * (g.full / 8) + bid / 8 : bid;
  } else {
    unit = bid - g.full;
    lin = g.full + unit / g.split;
    kbeg = (unit % g.split) * g.kchunk;
    kend = min(g.K, kbeg + g.kchunk);
  }
  const int tm = lin / nbn, tn = lin - tm * nbn;
  const int m0 = tm * HT_M, n0 = tn * HT_N;
  floatx16 acc[FC::MB][FC::NB];
  gemm_mainloop<AM, BM, FC>(s0, s1, g.A, g.B, m0, n0, kbeg, kend, acc);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  int wm, wn;
  wave_coords<FC>(wm, wn);
  if (unit >= 0) {  // one k range of a split tile: the whole f32 tile, row-major
    float* part = g.part + (size_t)unit * HT_M * HT_N;
#pragma unroll
    for (int mb = 0; mb < FC::MB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = wm * FC::WTM + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
#pragma unroll
        for (int nb = 0; nb < FC::NB; ++nb) part[r * HT_N + wn * FC::WTN + nb * 32 + l32] = acc[mb][nb][i];
      }
    return;
  }
  if (m0 + HT_M <= g.M && n0 + HT_N <= g.N) {  // interior tile: staged 16-byte row stores
    __syncthreads();  // every wave is done reading the pipeline buffers
    bf16* stg = wave_stage(s0, s1, wm, wn);
#pragma unroll
    for (int mb = 0; mb < FC::MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
#pragma unroll
        for (int nb = 0; nb < FC::NB; ++nb) stg[stage_at(row, nb * 32 + l32)] = f2bf(acc[mb][nb][i]);
      }
    }
    bf16* out = g.C + (size_t)(m0 + wm * FC::WTM) * g.ldc + n0 + wn * FC::WTN;
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int idx = it * 64 + lane, row = idx >> 3, ch = idx & 7;
      *reinterpret_cast<bf16x8*>(out + (size_t)row * g.ldc + 8 * ch) =
          *reinterpret_cast<const bf16x8*>(stg + stage_at(row, 8 * ch));
    }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < FC::MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = m0 + wm * FC::WTM + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (m >= g.M) continue;
#pragma unroll
      for (int nb = 0; nb < FC::NB; ++nb) {
        const int n = n0 + wn * FC::WTN + nb * 32 + l32;
        if (n < g.N) g.C[(size_t)m * g.ldc + n] = f2bf(acc[mb][nb][i]);
      }
    }
  }
}

// C of a split tile: its split f32 range tiles summed in range order, 32 rows of the tile per
// workgroup (grid: split tiles x HT_M / 32). N is a multiple of 8, so 8 columns that start
// inside the matrix lie inside it.
__global__ __launch_bounds__(256) void ffn_gemm_tail_kernel(FfnGemmParams g) {
  const int nbn = (g.N + HT_N - 1) / HT_N;
  const int lin = g.full + blockIdx.x;
  const int tm = lin / nbn, tn = lin - tm * nbn;
  const float* part = g.part + (size_t)blockIdx.x * g.split * HT_M * HT_N;
#pragma unroll
  for (int c = 0; c < 32 * HT_N / 8 / 256; ++c) {
    const int e = (threadIdx.x + 256 * c) * 8;
    const int r = blockIdx.y * 32 + e / HT_N, col = e % HT_N;
    const int m = tm * HT_M + r, n = tn * HT_N + col;
    if (m >= g.M || n >= g.N) continue;
    const size_t o = (size_t)r * HT_N + col;
    float4 a = *reinterpret_cast<const float4*>(part + o), b = *reinterpret_cast<const float4*>(part + o + 4);
    for (int k = 1; k < g.split; ++k) {
      const float* q = part + (size_t)k * HT_M * HT_N + o;
      const float4 x = *reinterpret_cast<const float4*>(q), y = *reinterpret_cast<const float4*>(q + 4);
      a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
      b.x += y.x; b.y += y.y; b.z += y.z; b.w += y.w;
    }
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16x8 o8;
#pragma unroll
    for (int t = 0; t < 8; ++t) o8[t] = f2bf(v[t]);
    *reinterpret_cast<bf16x8*>(g.C + (size_t)m * g.ldc + n) = o8;
  }
}

// Split plan: the tiles past the last complete round of 256 workgroups (all of them when there
// are fewer than 256) are split over k into S ranges when that is cheaper. Cost model, from
// the head products' measured rates: a round of 256 x 256 tiles costs 23.4 ns per k step of
// one element (48 us for K = 2048), and each split range tile costs its f32 tile written,
// read and summed (512 KiB at about 5 TB/s over the chip, 0.1 us) plus 5 us for the summing
// launch. A range keeps at least 1024 of K (so every range is non-empty).
FfnGemmPlan ffn_gemm_plan(int M, int N, int K) {
  FfnGemmPlan pl;
  pl.tiles = ((M + HT_M - 1) / HT_M) * ((N + HT_N - 1) / HT_N);
  pl.full = pl.tiles;
  pl.split = 1;
  pl.kchunk = 0;
  const int base = pl.tiles / 256 * 256, tail = pl.tiles - base;
  if (tail == 0) return pl;
  auto cost = [&](int s) {
    const double rounds = std::ceil(tail * (double)s / 256.0);
    return rounds * (K / (double)s) * 0.0234 + (s > 1 ? tail * s * 0.1 + 5.0 : 0.0);
  };
  int best = 1;
  double best_cost = cost(1);
  for (int s = 2; s <= 8 && K / s >= 1024; ++s) {
    const double c = cost(s);
    if (c < best_cost - 1e-9) { best = s; best_cost = c; }
  }
  if (best == 1) return pl;
  pl.full = base;
  pl.split = best;
  pl.kchunk = ((K + best - 1) / best + 127) / 128 * 128;
  return pl;
}

size_t ffn_gemm_workspace_bytes(const FfnGemmPlan& pl) {
  return pl.split > 1 ? (size_t)(pl.tiles - pl.full) * pl.split * HT_M * HT_N * sizeof(float) : 0;
}

hipError_t launch_ffn_gemm(const FfnGemmParams& g, int a_mode, int b_mode, hipStream_t st) {
  const int tiles = ((g.M + HT_M - 1) / HT_M) * ((g.N + HT_N - 1) / HT_N);
  const int grid = g.split > 1 ? g.full + (tiles - g.full) * g.split : tiles;
  {
    KTimer t("ffn_gemm", st);
    if (a_mode == KMAJOR && b_mode == KMAJOR) hipLaunchKernelGGL((ffn_gemm_kernel<KMAJOR, KMAJOR>), dim3(grid), dim3(FNT), 0, st, g);
    else if (a_mode == KMAJOR) hipLaunchKernelGGL((ffn_gemm_kernel<KMAJOR, MNMAJOR>), dim3(grid), dim3(FNT), 0, st, g);
    else if (b_mode == KMAJOR) hipLaunchKernelGGL((ffn_gemm_kernel<MNMAJOR, KMAJOR>), dim3(grid), dim3(FNT), 0, st, g);
    else hipLaunchKernelGGL((ffn_gemm_kernel<MNMAJOR, MNMAJOR>), dim3(grid), dim3(FNT), 0, st, g);
  }
  if (g.split > 1) {
    KTimer t("ffn_gemm_tail", st);
    hipLaunchKernelGGL(ffn_gemm_tail_kernel, dim3(tiles - g.full, HT_M / 32), dim3(256), 0, st, g);
  }
  return hipGetLastError();
}

hipError_t launch_ffn_fwd(const FfnParams& p, hipStream_t st) {
  const int tiles = ((p.N + HT_M - 1) / HT_M) * (2 * p.F / HT_N);
  KTimer t("ffn_gate_up", st);
  hipLaunchKernelGGL(ffn_gate_up_kernel, dim3(tiles), dim3(FNT), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_ffn_dy(const FfnParams& p, hipStream_t st) {
  const int tiles = ((p.N + HT_M - 1) / HT_M) * ((p.F + HT_N - 1) / HT_N);
  KTimer t("ffn_dy", st);
  hipLaunchKernelGGL(ffn_dy_kernel, dim3(tiles), dim3(FNT), 0, st, p);
  return hipGetLastError();
}

}  // namespace alg
