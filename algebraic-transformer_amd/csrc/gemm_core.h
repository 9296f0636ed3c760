// bf16 MFMA GEMM main loop for gfx950, shared by the fused-head kernels.
//
// C[M][N] = sum_k A[m][k] B[k][n] with f32 accumulation. A configuration fixes the
// workgroup tile TM x TN, 64-deep k steps and a WM x WN grid of waves; each wave owns a
// (TM/WM) x (TN/WN) sub-tile of 32x32 blocks computed with v_mfma_f32_32x32x16_bf16.
// Operands may be stored k-contiguous (fragments read with ds_read_b128) or m/n-contiguous
// (fragments read transposed with ds_read_b64_tr_b16), so every head product reads its
// operands in their natural HBM layout. Global tiles are double-buffered through LDS (the
// next tile's loads are in flight while the current one is consumed) with one barrier per
// k step; rows/columns outside the matrix are zero-filled.
#pragma once

#include "common.h"

namespace alg {

constexpr int GT_K = 64;
enum OperandMode { KMAJOR = 0, MNMAJOR = 1 };

template <int TM_, int TN_, int WM_, int WN_>
struct GemmCfg {
  static constexpr int TM = TM_, TN = TN_, WM = WM_, WN = WN_;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int WTM = TM / WM, WTN = TN / WN;  // wave sub-tile
  static constexpr int MB = WTM / 32, NB = WTN / 32;  // 32x32 blocks per wave
};

struct GemmOperand {
  const bf16* ptr;
  long ld;         // leading dimension (elements) of the stored matrix
  int rows_valid;  // stored rows at or beyond this are read as zero
  int cols_valid;  // stored columns at or beyond this are read as zero (multiple of 8)
};

// LDS tile of an operand covering TMN (m or n) x 64 (k).
template <int MODE, int TMN>
struct TileShape;
template <int TMN>
struct TileShape<KMAJOR, TMN> {   // stored [mn][k]
  static constexpr int ROWS = TMN, COLS = GT_K, PITCH = GT_K + 8;
};
template <int TMN>
struct TileShape<MNMAJOR, TMN> {  // stored [k][mn]
  static constexpr int ROWS = GT_K, COLS = TMN, PITCH = TMN + 8;
};

template <int MODE, int TMN, int NT>
struct OperandTile {
  typedef TileShape<MODE, TMN> S;
  static constexpr int CPR = S::COLS / 8;               // 16-byte chunks per stored row
  static constexpr int CHUNKS = S::ROWS * CPR / NT;     // per thread
  static constexpr int ELEMS = S::ROWS * S::PITCH;
  static_assert(S::ROWS * CPR % NT == 0, "tile/threads");

  // Global -> registers.
  static __device__ __forceinline__ void load(uint4 (&r)[CHUNKS], const GemmOperand& op, int mn0, int k0) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int idx = threadIdx.x + c * NT;
      const int row = idx / CPR, col = (idx - row * CPR) * 8;
      const int grow = (MODE == KMAJOR) ? mn0 + row : k0 + row;
      const int gcol = (MODE == KMAJOR) ? k0 + col : mn0 + col;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (grow < op.rows_valid && gcol < op.cols_valid)
        v = *reinterpret_cast<const uint4*>(op.ptr + (long)grow * op.ld + gcol);
      r[c] = v;
    }
  }
  // Registers -> LDS.
  static __device__ __forceinline__ void store(bf16* tile, const uint4 (&r)[CHUNKS]) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int idx = threadIdx.x + c * NT;
      const int row = idx / CPR, col = (idx - row * CPR) * 8;
      *reinterpret_cast<uint4*>(tile + row * S::PITCH + col) = r[c];
    }
  }
  // Fragment of the 32-wide block starting at tile-local mn for k step ks (16 k).
  static __device__ __forceinline__ bf16x8 frag(const bf16* tile, int mn, int ks, int lane) {
    if constexpr (MODE == KMAJOR) {
      return *reinterpret_cast<const bf16x8*>(tile + (mn + (lane & 31)) * S::PITCH + ks * 16 + 8 * (lane >> 5));
    } else {
      const int klo = ks * 16 + 8 * (lane >> 5);
      return lds_tr_frag(tile, S::PITCH, klo, klo + 4, mn, lane);
    }
  }
};

template <int AM, int BM, class C>
struct GemmSmem {
  bf16 a[2][OperandTile<AM, C::TM, C::THREADS>::ELEMS];
  bf16 b[2][OperandTile<BM, C::TN, C::THREADS>::ELEMS];
};

// Wave coordinates inside the workgroup tile.
template <class C>
__device__ __forceinline__ void wave_coords(int& wm, int& wn) {
  const int wave = threadIdx.x >> 6;
  wm = wave / C::WN;
  wn = wave % C::WN;
}

// Accumulate the (m0, n0) tile over k in [0, K). acc[mb][nb] is the wave's 32x32 block at
// rows wm*WTM + mb*32 and columns wn*WTN + nb*32 of the workgroup tile.
template <int AM, int BM, class C>
__device__ __forceinline__ void gemm_mainloop(GemmSmem<AM, BM, C>& sm, const GemmOperand& A, const GemmOperand& B,
                                              int m0, int n0, int K, floatx16 (&acc)[C::MB][C::NB]) {
  typedef OperandTile<AM, C::TM, C::THREADS> TA;
  typedef OperandTile<BM, C::TN, C::THREADS> TB;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  wave_coords<C>(wm, wn);
#pragma unroll
  for (int i = 0; i < C::MB; ++i)
#pragma unroll
    for (int j = 0; j < C::NB; ++j) acc[i][j] = floatx16{};
  const int nk = (K + GT_K - 1) / GT_K;
  uint4 ra[TA::CHUNKS], rb[TB::CHUNKS];
  TA::load(ra, A, m0, 0);
  TB::load(rb, B, n0, 0);
  TA::store(sm.a[0], ra);
  TB::store(sm.b[0], rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      TA::load(ra, A, m0, (kt + 1) * GT_K);
      TB::load(rb, B, n0, (kt + 1) * GT_K);
    }
#pragma unroll
    for (int ks = 0; ks < GT_K / 16; ++ks) {
      bf16x8 af[C::MB], bfr[C::NB];
#pragma unroll
      for (int i = 0; i < C::MB; ++i) af[i] = TA::frag(sm.a[cur], wm * C::WTM + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < C::NB; ++j) bfr[j] = TB::frag(sm.b[cur], wn * C::WTN + j * 32, ks, lane);
#pragma unroll
      for (int i = 0; i < C::MB; ++i)
#pragma unroll
        for (int j = 0; j < C::NB; ++j) acc[i][j] = mfma_bf16(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      TA::store(sm.a[cur ^ 1], ra);
      TB::store(sm.b[cur ^ 1], rb);
    }
    __syncthreads();
  }
}

// Map a linear workgroup id to (tile_m, tile_n) so that the workgroups one XCD runs
// (ids congruent mod 8 are dispatched to the same XCD) cover a compact group of tiles
// that share A row panels and B column panels in that XCD's L2.
__device__ __forceinline__ void xcd_tile(int bid, int nbm, int nbn, int& tm, int& tn) {
  const int total = nbm * nbn;
  int lin = bid;
  if (total % 8 == 0) lin = (bid % 8) * (total / 8) + bid / 8;
  constexpr int GROUP = 8;  // tiles of M per group, swept across N
  const int group_size = GROUP * nbn;
  const int g = lin / group_size;
  const int first_m = g * GROUP;
  const int gm = min(nbm - first_m, GROUP);
  const int r = lin - g * group_size;
  tm = first_m + r % gm;
  tn = r / gm;
}

}  // namespace alg
