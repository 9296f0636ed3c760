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
  // 128 rows x 8 chunks of 8 columns: lane -> (row, chunk).
  const int f0 = n0 + wn * FC::WTN;
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int idx = it * 64 + lane, row = idx >> 3, ch = idx & 7;
    const int tok = m0 + wm * FC::WTM + row, f = f0 + 8 * ch;
    if (tok >= p.N || f >= p.F) continue;  // F is a multiple of 128: chunks are whole
    const size_t o = (size_t)tok * p.F + f;
    const bf16x8 dyv = *reinterpret_cast<const bf16x8*>(stg + stage_at(row, 8 * ch));
    const bf16x8 gv = *reinterpret_cast<const bf16x8*>(p.gate + o);
    const bf16x8 uv = *reinterpret_cast<const bf16x8*>(p.up + o);
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
