// bf16 MFMA GEMM main loop for gfx950, shared by the fused-head kernels.
//
// C[M][N] = sum_k A[m][k] B[k][n] with f32 accumulation, 128x128 workgroup tile, 64-deep
// k steps, 4 waves as 2x2, each wave 64x64 = 2x2 blocks of v_mfma_f32_32x32x16_bf16.
// Operands may be stored k-contiguous (fragments read with ds_read_b128) or m/n-contiguous
// (fragments read transposed with ds_read_b64_tr_b16), so every head product reads its
// operands in their natural HBM layout. Global tiles are double-buffered through LDS with
// one barrier per k step; rows outside the matrix are zero-filled.
#pragma once

#include "common.h"

namespace alg {

constexpr int GT_M = 128, GT_N = 128, GT_K = 64;
enum OperandMode { KMAJOR = 0, MNMAJOR = 1 };

struct GemmOperand {
  const bf16* ptr;
  long ld;        // leading dimension (elements) of the stored matrix
  int rows_valid; // stored rows beyond this are read as zero
};

template <int MODE>
struct TileShape;  // LDS tile shape for an operand of 128 (m or n) x 64 (k)
template <>
struct TileShape<KMAJOR> {   // stored [mn][k]: 128 rows of 64 k
  static constexpr int ROWS = 128, COLS = 64, PITCH = 72;
};
template <>
struct TileShape<MNMAJOR> {  // stored [k][mn]: 64 rows of 128 mn
  static constexpr int ROWS = 64, COLS = 128, PITCH = 136;
};

// Global -> registers for one 128x64 operand tile (4 x 16 bytes per thread).
template <int MODE>
__device__ __forceinline__ void gemm_load(uint4 (&r)[4], const GemmOperand& op, int mn0, int k0) {
  typedef TileShape<MODE> S;
  constexpr int CPR = S::COLS / 8;  // 16-byte chunks per stored row
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int idx = threadIdx.x + c * 256;
    const int row = idx / CPR, col = (idx - row * CPR) * 8;
    const int grow = (MODE == KMAJOR) ? mn0 + row : k0 + row;
    const int gcol = (MODE == KMAJOR) ? k0 + col : mn0 + col;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (grow < op.rows_valid) v = *reinterpret_cast<const uint4*>(op.ptr + (long)grow * op.ld + gcol);
    r[c] = v;
  }
}

template <int MODE>
__device__ __forceinline__ void gemm_store(bf16* tile, const uint4 (&r)[4]) {
  typedef TileShape<MODE> S;
  constexpr int CPR = S::COLS / 8;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int idx = threadIdx.x + c * 256;
    const int row = idx / CPR, col = (idx - row * CPR) * 8;
    *reinterpret_cast<uint4*>(tile + row * S::PITCH + col) = r[c];
  }
}

// Fragment of the 32-wide block starting at mn (tile-local) for k step ks (16 k).
template <int MODE>
__device__ __forceinline__ bf16x8 gemm_frag(const bf16* tile, int mn, int ks, int lane) {
  typedef TileShape<MODE> S;
  const int h = lane >> 5;
  if constexpr (MODE == KMAJOR) {
    return *reinterpret_cast<const bf16x8*>(tile + (mn + (lane & 31)) * S::PITCH + ks * 16 + 8 * h);
  } else {
    const int klo = ks * 16 + 8 * h;
    return lds_tr_frag(tile, S::PITCH, klo, klo + 4, mn, lane);
  }
}

template <int AM, int BM>
struct GemmSmem {
  bf16 a[2][TileShape<AM>::ROWS * TileShape<AM>::PITCH];
  bf16 b[2][TileShape<BM>::ROWS * TileShape<BM>::PITCH];
};

// Accumulate the (m0, n0) tile over k in [0, K). acc[mb][nb] is the wave's 32x32 block
// (wave rows wm*64 + mb*32, cols wn*64 + nb*32).
template <int AM, int BM>
__device__ __forceinline__ void gemm_mainloop(GemmSmem<AM, BM>& sm, const GemmOperand& A, const GemmOperand& B,
                                              int m0, int n0, int K, floatx16 (&acc)[2][2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
  const int nk = (K + GT_K - 1) / GT_K;
  uint4 ra[4], rb[4];
  gemm_load<AM>(ra, A, m0, 0);
  gemm_load<BM>(rb, B, n0, 0);
  gemm_store<AM>(sm.a[0], ra);
  gemm_store<BM>(sm.b[0], rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      gemm_load<AM>(ra, A, m0, (kt + 1) * GT_K);
      gemm_load<BM>(rb, B, n0, (kt + 1) * GT_K);
    }
#pragma unroll
    for (int ks = 0; ks < GT_K / 16; ++ks) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = gemm_frag<AM>(sm.a[cur], wm * 64 + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) bfr[j] = gemm_frag<BM>(sm.b[cur], wn * 64 + j * 32, ks, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      gemm_store<AM>(sm.a[cur ^ 1], ra);
      gemm_store<BM>(sm.b[cur ^ 1], rb);
    }
    __syncthreads();
  }
}

}  // namespace alg
