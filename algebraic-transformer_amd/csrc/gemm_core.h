// bf16 MFMA GEMM main loop for gfx950, shared by the fused-head kernels.
//
// C[M][N] = sum_k A[m][k] B[k][n] with f32 accumulation. A configuration fixes the
// workgroup tile TM x TN, 64-deep k steps and a WM x WN grid of waves; each wave owns a
// (TM/WM) x (TN/WN) sub-tile of 32x32 blocks computed with v_mfma_f32_32x32x16_bf16.
//
// Operands are stored either k-contiguous ([mn][k]; fragments read with ds_read_b128) or
// m/n-contiguous ([k][mn]; fragments read transposed with ds_read_b64_tr_b16), so every
// head product reads its operands in their natural HBM layout.
//
// Global -> LDS copies are buffer loads that write LDS (each lane of a wave instruction
// writes 16 bytes at base + 16*lane), so no VGPRs stage the tiles and the next tile's copy is
// in flight while the current one feeds the MFMAs; tiles are double-buffered with one barrier
// per k step. Because the copy writes rows without padding, 16-byte chunks are placed with an
// XOR swizzle that keeps the fragment reads free of bank conflicts:
//   k-contiguous rows (128 B):      chunk c of row r lives at chunk c ^ ((r >> 1) & 7)
//   mn-contiguous rows (2*TMN B):   chunk c of row r lives at chunk c ^ (4 * (r & 3))
// The pipelined loop covers the largest multiple of 128 in the k range; a remaining partial
// k tile is copied through registers with zero fill. Tiles that reach past the matrix edge in
// m or n stay on the pipelined loop with range-checked copies: every copy instruction gets a
// descriptor whose range ends at the operand's allocation, so reads past it return zeros, and
// the values read past a row's logical end (the next row's data) only reach output rows or
// columns outside the matrix, which the epilogues do not store.
#pragma once

#include <type_traits>

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
  int rows_valid;  // rows of the logical matrix
  int cols_valid;  // columns of the logical matrix (ld >= cols_valid rounded up to 8)
  long extent;     // elements readable from ptr (the allocation); a multiple of 8
  // Split m/n-contiguous operand: the logical columns alternate in 32-wide blocks between two
  // stored halves `split` elements apart (logical block 2b -> stored columns 32b.. of the first
  // half, block 2b+1 -> the same columns of the second half), so a product against [W1 | W2]
  // gives each wave matching W1 and W2 columns. 0: plain operand. Logical tile columns start at
  // mn0, stored ones at mn0 / 2.
  long split = 0;
};

// Stored element offset, relative to a tile's stored first column, of logical chunk c
// (8 columns) of an m/n-contiguous operand.
__device__ __forceinline__ long split_chunk_offset(const GemmOperand& op, int c) {
  if (!op.split) return 8L * c;
  const int blk = c >> 2;
  return (blk & 1) * op.split + (blk >> 1) * 32 + (c & 3) * 8;
}

// One operand tile covering TMN (m or n) x 64 (k) in LDS, unpadded and swizzled.
template <int MODE, int TMN, int NT>
struct OperandTile {
  static constexpr int ROWS = MODE == KMAJOR ? TMN : GT_K;   // stored rows in the tile
  static constexpr int CPR = (MODE == KMAJOR ? GT_K : TMN) / 8;  // 16-byte chunks per row
  static constexpr int ELEMS = ROWS * CPR * 8;
  static constexpr int WAVES = NT / 64;
  static constexpr int INSTR = ROWS * CPR / 64;             // wave copy instructions per tile
  static_assert(INSTR % WAVES == 0, "tile/waves");
  static constexpr int PER_WAVE = INSTR / WAVES;

  static constexpr int READS_PER_FRAG = MODE == KMAJOR ? 1 : 2;  // LDS instructions per fragment

  static __device__ __forceinline__ int swz(int row) {
    return MODE == KMAJOR ? ((row >> 1) & 7) : 4 * (row & 3);
  }
  // Element offset of logical (row, chunk) inside the tile.
  static __device__ __forceinline__ int at(int row, int chunk) { return (row * CPR + (chunk ^ swz(row))) * 8; }

  // Rows of the tile one wave instruction covers, and the swizzle period in rows.
  static constexpr int RPI = 64 / CPR;
  static_assert(CPR <= 64 && 64 % CPR == 0, "chunks per row");
  static constexpr int SWZ_PERIOD = MODE == KMAJOR ? 16 : 4;  // swz(row) depends on row mod this
  static_assert((RPI * PER_WAVE) % SWZ_PERIOD == 0 && (2 * RPI) % SWZ_PERIOD == 0,
                "the swizzle of instruction J must depend on J's parity only");

  // Per-lane byte offsets (relative to the instruction's first row and the tile's first
  // column) for even and odd instructions; computed once per kernel.
  static __device__ __forceinline__ void lane_offsets(const GemmOperand& op, uint32_t (&off)[2]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int row = RPI * par + lane / CPR;  // row inside the tile modulo the swizzle period
      const int c = (lane % CPR) ^ swz(row);   // logical chunk this lane fetches
      const long col = MODE == KMAJOR ? 8L * c : split_chunk_offset(op, c);
      off[par] = (uint32_t)(((lane / CPR) * op.ld + col) * 2);
    }
  }

  // Asynchronous global -> LDS copy of the tile at (mn0, k0); the tile must lie inside the
  // stored matrix. Lane `lane` of instruction J writes the physical chunk 64*J + lane.
  // `wave` must be wave-uniform (from readfirstlane) so the addressing stays scalar.
  // Instructions [J0, J1) of this wave's share (all of it by default).
  // The copies are buffer loads that write LDS: the descriptor's base is the tile's first
  // element (scalar), the instruction's row offset is the scalar offset, and the per-lane part
  // is one of the two lane offsets, so no per-instruction vector address is formed.
  // CHECKED (edge tiles): one descriptor per instruction, based at the instruction's first
  // row, whose range ends at the operand's allocation (the buffer range check covers the
  // per-lane offset only, not the scalar one), so chunks past the allocation read as zeros.
  template <bool CHECKED = false, int J0 = 0, int J1 = PER_WAVE>
  static __device__ __forceinline__ void copy(bf16* tile, const GemmOperand& op, const uint32_t (&off)[2], int wave,
                                              int mn0, int k0) {
    const int r0 = (MODE == KMAJOR) ? mn0 : k0;
    const int c0 = (MODE == KMAJOR) ? k0 : (op.split ? mn0 / 2 : mn0);
    if constexpr (!CHECKED) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(op.ptr + ((long)r0 * op.ld + c0)), (short)0, 0x7FFFFFFF, BUF_RSRC_WORD3);
#pragma unroll
      for (int j = J0; j < J1; ++j) {
        const int J = wave * PER_WAVE + j;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_PTR(void, tile + J * 512), 16, off[j & 1],
                                                 (int)(RPI * J * op.ld * 2), 0, 0);
      }
    } else {
#pragma unroll
      for (int j = J0; j < J1; ++j) {
        const int J = wave * PER_WAVE + j;
        const long first = (long)(r0 + RPI * J) * op.ld + c0;  // element offset of the instruction's base
        const long rest = op.extent - first;
        const int nrec = rest <= 0 ? 0 : (int)(rest >= 0x3FFFFFFF ? 0x7FFFFFFE : 2 * rest);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(op.ptr + (rest <= 0 ? 0 : first)), (short)0, nrec, BUF_RSRC_WORD3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_PTR(void, tile + J * 512), 16, off[j & 1], 0, 0, 0);
      }
    }
  }
  // Synchronous copy with zero fill (edge tiles, partial last k tile): elements outside the
  // stored matrix, or at k >= K, are zero (per element, so rows may end inside a chunk).
  static __device__ __forceinline__ void copy_zero_fill(bf16* tile, const GemmOperand& op, int mn0, int k0, int K) {
    for (int p = threadIdx.x; p < ROWS * CPR; p += NT) {
      const int row = p / CPR, c = p - row * CPR;
      const int grow = (MODE == KMAJOR) ? mn0 + row : k0 + row;
      const int gcol = (MODE == KMAJOR) ? k0 + 8 * c : mn0 + 8 * c;  // logical column
      const int col_end = (MODE == KMAJOR) ? min(K, op.cols_valid) : op.cols_valid;
      const bool row_ok = grow < op.rows_valid && ((MODE == KMAJOR) || grow < K);
      const int nv = row_ok ? min(8, col_end - gcol) : 0;  // live elements of this chunk
      const long scol = (MODE != KMAJOR && op.split) ? mn0 / 2 + split_chunk_offset(op, c) : gcol;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (nv > 0) v = *reinterpret_cast<const uint4*>(op.ptr + (long)grow * op.ld + scol);
      if (nv < 8) {  // keep elements [0, nv): two bf16 per 32-bit word
        unsigned int* w = reinterpret_cast<unsigned int*>(&v);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const unsigned int keep = nv >= 2 * q + 2 ? 0xffffffffu : (nv == 2 * q + 1 ? 0x0000ffffu : 0u);
          w[q] &= keep;
        }
      }
      *reinterpret_cast<uint4*>(tile + at(row, c)) = v;
    }
  }
  // Fragment of the 32-wide block starting at tile-local mn for k step ks (16 k).
  static __device__ __forceinline__ bf16x8 frag(const bf16* tile, int mn, int ks, int lane) {
    const int h = lane >> 5;
    if constexpr (MODE == KMAJOR) {
      return *reinterpret_cast<const bf16x8*>(tile + at(mn + (lane & 31), 2 * ks + h));
    } else {
      // ds_read_b64_tr_b16: lane i of each 16-lane group addresses row klo + i/4 at column
      // n0 + 4*(i%4) and receives column n0 + i for rows klo..klo+3 (see common.h).
      const int i = lane & 15;
      const int col = mn + ((lane >> 4) & 1) * 16 + 4 * (i & 3);
      const int r0 = ks * 16 + 8 * h + (i >> 2);
      const bf16* p0 = tile + at(r0, col >> 3) + (col & 7);
      const bf16* p1 = tile + at(r0 + 4, col >> 3) + (col & 7);
      bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p0));
      bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p1));
      bf16x8 r;
      r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
      r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
      return r;
    }
  }
};

// Scheduling template for one pipelined phase: NM independent MFMAs, NR LDS reads of the
// next phase's fragments and NG global->LDS copies. Reads are issued early (ceil(NR/8)
// after each of the first MFMAs) so they have landed by the time the next phase needs them;
// copies are spread one per MFMA so the vector memory queue never stalls the wave.
template <int NM, int NR, int NG = 0>
__device__ __forceinline__ void interleave_phase() {
  constexpr int PER = (NR + 7) / 8;
  constexpr int HEAD = (NR + PER - 1) / PER;  // MFMAs that carry reads
  static_assert(HEAD <= NM && NG <= NM, "phase shape");
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // one MFMA
    if (i < HEAD) __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);  // PER LDS reads
    if (i < NG) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);      // one copy
  }
  __builtin_amdgcn_sched_barrier(0);
}

// One pipeline stage (A and B tiles). The two stages are separate __shared__ objects so
// the compiler can tell reads of one stage from the DMA writes into the other and does not
// wait for the next tile's copy before reading the current one.
template <int AM, int BM, class C>
struct GemmStage {
  bf16 a[OperandTile<AM, C::TM, C::THREADS>::ELEMS];
  bf16 b[OperandTile<BM, C::TN, C::THREADS>::ELEMS];
};

// Wave coordinates inside the workgroup tile.
template <class C>
__device__ __forceinline__ void wave_coords(int& wm, int& wn) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  wm = wave / C::WN;
  wn = wave % C::WN;
}

// Accumulate the (m0, n0) tile over k in [kbeg, K). acc[mb][nb] is the wave's 32x32 block at
// rows wm*WTM + mb*32 and columns wn*WTN + nb*32 of the workgroup tile.
template <int AM, int BM, class C>
__device__ __forceinline__ void gemm_mainloop(GemmStage<AM, BM, C>& s0, GemmStage<AM, BM, C>& s1,
                                              const GemmOperand& A, const GemmOperand& B, int m0, int n0, int kbeg,
                                              int K, floatx16 (&acc)[C::MB][C::NB]) {
  typedef OperandTile<AM, C::TM, C::THREADS> TA;
  typedef OperandTile<BM, C::TN, C::THREADS> TB;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  wave_coords<C>(wm, wn);
#pragma unroll
  for (int i = 0; i < C::MB; ++i)
#pragma unroll
    for (int j = 0; j < C::NB; ++j) acc[i][j] = floatx16{};
  struct Frags {
    bf16x8 a[C::MB], b[C::NB];
  };
  // Fragments are read in the order the MFMAs consume them (all of B, then A row by row).
  auto load = [&](const GemmStage<AM, BM, C>& st, int ks, Frags& f) {
#pragma unroll
    for (int j = 0; j < C::NB; ++j) f.b[j] = TB::frag(st.b, wn * C::WTN + j * 32, ks, lane);
#pragma unroll
    for (int i = 0; i < C::MB; ++i) f.a[i] = TA::frag(st.a, wm * C::WTM + i * 32, ks, lane);
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < C::MB; ++i)
#pragma unroll
      for (int j = 0; j < C::NB; ++j) acc[i][j] = mfma_bf16(f.a[i], f.b[j], acc[i][j]);
  };
  const int klen = K - kbeg;
  const int kmain = klen >= 2 * GT_K ? klen - klen % (2 * GT_K) : 0;  // pipelined part
  const bool a_full = (AM == KMAJOR ? A.rows_valid : A.cols_valid) >= m0 + C::TM;
  const bool b_full = (BM == KMAJOR ? B.rows_valid : B.cols_valid) >= n0 + C::TN;
  if (kmain > 0) {
    uint32_t aoff[2], boff[2];
    TA::lane_offsets(A, aoff);
    TB::lane_offsets(B, boff);
    const int wave_u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nk = kmain / GT_K;  // even, >= 2
    // One k step, software-pipelined over its four 16-deep sub-steps: fragments of sub-step
    // ks+1 are read while ks multiplies. f0 holds sub-step 0 of `cur` on entry and sub-step 0
    // of `nxt` on exit. The barrier (after this wave's copies into `nxt` have landed, vmcnt)
    // comes before the last sub-step; after it no wave reads `cur` again, so the copy of tile
    // kt+2 into `cur` is issued right there, under the last sub-step's MFMAs: each copy has a
    // whole k step to land before the next barrier waits for it.
    auto pipelined = [&](auto checked) {
      constexpr bool CHK = decltype(checked)::value;
      auto copy_tile = [&](GemmStage<AM, BM, C>& st, int kt) {
        TA::template copy<CHK>(st.a, A, aoff, wave_u, m0, kbeg + kt * GT_K);
        TB::template copy<CHK>(st.b, B, boff, wave_u, n0, kbeg + kt * GT_K);
      };
      constexpr int NG = TA::PER_WAVE + TB::PER_WAVE;  // copy instructions per wave and tile
      Frags f0, f1;
      constexpr int NM = C::MB * C::NB;
      constexpr int NR = C::MB * TA::READS_PER_FRAG + C::NB * TB::READS_PER_FRAG;
      static_assert(NG <= NM, "one copy per MFMA at most");
      auto step = [&](GemmStage<AM, BM, C>& cur, GemmStage<AM, BM, C>& nxt, int kt, auto copyc) {
        __builtin_amdgcn_s_setprio(0);
        load(cur, 1, f1);
        mma(f0);
        interleave_phase<NM, NR>();
        load(cur, 2, f0);
        mma(f1);
        interleave_phase<NM, NR>();
        load(cur, 3, f1);
        mma(f0);
        interleave_phase<NM, NR>();
        __builtin_amdgcn_s_waitcnt(VMCNT0);
        __syncthreads();
        // Raised wave priority from the barrier to the end of the step: the waves that leave
        // the barrier first issue their copies and the next stage's first fragments ahead of
        // the other wave's sub-step MFMAs (measured: about 1 % on the head products).
        __builtin_amdgcn_s_setprio(1);
        if constexpr (decltype(copyc)::value) copy_tile(cur, kt + 2);
        load(nxt, 0, f0);
        mma(f1);
        interleave_phase<NM, NR, decltype(copyc)::value ? NG : 0>();
      };
      // The last k step: no copy.
      auto last = [&](const GemmStage<AM, BM, C>& cur) {
        load(cur, 1, f1);
        mma(f0);
        interleave_phase<NM, NR>();
        load(cur, 2, f0);
        mma(f1);
        interleave_phase<NM, NR>();
        load(cur, 3, f1);
        mma(f0);
        interleave_phase<NM, NR>();
        mma(f1);
      };
      copy_tile(s0, 0);
      copy_tile(s1, 1);
      // Wait for tile 0's copies only (tile 1's NG copy instructions are the younger ones):
      // tile 1 is first read after the barrier inside the first step, which waits for every
      // copy, so its load overlaps tile 0's first three sub-steps. The barrier is a plain
      // s_barrier: __syncthreads() would add a release fence, which waits for every copy.
      // Each wave has waited for its own tile-0 copies before it, so after it all of tile 0
      // is in LDS; the memory clobber keeps the fragment reads after it.
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(NG));
      asm volatile("s_barrier" ::: "memory");
      load(s0, 0, f0);
      int kt = 0;
      for (; kt + 2 < nk; kt += 2) {
        step(s0, s1, kt, std::true_type{});
        step(s1, s0, kt + 1, std::true_type{});
      }
      step(s0, s1, kt, std::false_type{});
      last(s1);
    };
    if (a_full && b_full) pipelined(std::false_type{});
    else pipelined(std::true_type{});
  }
  // Remaining partial k tiles (and short k ranges): register copies with zero fill.
  for (int k0 = kbeg + kmain; k0 < K; k0 += GT_K) {
    __syncthreads();
    TA::copy_zero_fill(s0.a, A, m0, k0, K);
    TB::copy_zero_fill(s0.b, B, n0, k0, K);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < GT_K / 16; ++ks) {
      Frags f;
      load(s0, ks, f);
      mma(f);
    }
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

// Row-major order inside each XCD's contiguous share of the tiles: the tiles an XCD runs
// together cover a few A row panels with every B column panel, so each A panel is streamed
// from memory once (for products whose A operand is large and B small).
__device__ __forceinline__ void xcd_tile_rowmajor(int bid, int nbm, int nbn, int& tm, int& tn) {
  const int total = nbm * nbn;
  const int lin = total % 8 == 0 ? (bid % 8) * (total / 8) + bid / 8 : bid;
  tm = lin / nbn;
  tn = lin - tm * nbn;
}

}  // namespace alg
