// bf16 MFMA GEMM main loop for gfx950, shared by the fused-head kernels.
//
// C[M][N] = sum_k A[m][k] B[k][n] with f32 accumulation. Workgroup tile TM x TN (128 or 256
// each), 64-deep k steps, 4 waves as 2x2, each wave (TM/2) x (TN/2) = (TM/64) x (TN/64)
// blocks of v_mfma_f32_32x32x16_bf16. Operands may be stored k-contiguous (fragments read
// with ds_read_b128) or m/n-contiguous (fragments read transposed with ds_read_b64_tr_b16),
// so every head product reads its operands in their natural HBM layout. Global tiles are
// double-buffered through LDS (the next tile's loads are in flight while the current one is
// consumed) with one barrier per k step; rows/columns outside the matrix are zero-filled.
#pragma once

#include "common.h"

namespace alg {

constexpr int GT_K = 64;
enum OperandMode { KMAJOR = 0, MNMAJOR = 1 };

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

template <int MODE, int TMN>
struct OperandTile {
  typedef TileShape<MODE, TMN> S;
  static constexpr int CPR = S::COLS / 8;               // 16-byte chunks per stored row
  static constexpr int CHUNKS = S::ROWS * CPR / 256;    // per thread
  static constexpr int ELEMS = S::ROWS * S::PITCH;

  // Global -> registers.
  static __device__ __forceinline__ void load(uint4 (&r)[CHUNKS], const GemmOperand& op, int mn0, int k0) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int idx = threadIdx.x + c * 256;
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
      const int idx = threadIdx.x + c * 256;
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

template <int AM, int BM, int TM, int TN>
struct GemmSmem {
  bf16 a[2][OperandTile<AM, TM>::ELEMS];
  bf16 b[2][OperandTile<BM, TN>::ELEMS];
};

template <int TM, int TN>
struct WaveTile {
  static constexpr int MB = TM / 64, NB = TN / 64;  // 32x32 blocks per wave
};

// Accumulate the (m0, n0) tile over k in [0, K). acc[mb][nb] is the wave's 32x32 block at
// wave rows wm*(TM/2) + mb*32 and columns wn*(TN/2) + nb*32.
template <int AM, int BM, int TM, int TN>
__device__ __forceinline__ void gemm_mainloop(GemmSmem<AM, BM, TM, TN>& sm, const GemmOperand& A,
                                              const GemmOperand& B, int m0, int n0, int K,
                                              floatx16 (&acc)[TM / 64][TN / 64]) {
  typedef OperandTile<AM, TM> TA;
  typedef OperandTile<BM, TN> TB;
  constexpr int MB = TM / 64, NB = TN / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = floatx16{};
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
      bf16x8 af[MB], bfr[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i) af[i] = TA::frag(sm.a[cur], wm * (TM / 2) + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < NB; ++j) bfr[j] = TB::frag(sm.b[cur], wn * (TN / 2) + j * 32, ks, lane);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma_bf16(af[i], bfr[j], acc[i][j]);
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
