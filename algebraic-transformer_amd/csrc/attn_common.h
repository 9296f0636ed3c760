// Parameters and variant selection shared by the attention kernels.
#pragma once

#include "common.h"
#include "ktimer.h"

namespace alg {

#ifndef ALG_FALLBACK_GRID
#define ALG_FALLBACK_GRID 512
#endif
// Workgroups of a flag-checked fallback launch (grid-stride over its work items): with the flag
// clear every workgroup exits at once, so the launch costs its dispatch.
constexpr int FALLBACK_GRID = ALG_FALLBACK_GRID;

// Variants of the asinh-power kernel (src/algebraic/kernels/flash.py:59-73, 732-760, 850-852):
//   INRANGE  unshifted, unclipped, stat = 1/Z (the guarded "low" variant, bounded_scores)
//   CLIPPED  unshifted with x = min(s, clamp) (range_guard=False defaults); stat 1/Z or Z^(-1/n)
//   SHIFTED  running-max accumulation (the guarded "high" fallback or explicit shift=True)
enum AttnMode { MODE_INRANGE = 0, MODE_CLIPPED = 1, MODE_SHIFTED = 2 };

constexpr int FWD_BQ = 128;  // queries per forward workgroup (its guard partials: one set each)

struct AttnFwdParams {
  const void* q;       // (B,H,T,D) pre-scaled queries q_s = round(q * alpha)
  const void* k;       // (B,H,T,D)
  const void* v;       // (B,H,T,D)
  const float* sink;   // (H,) sink logit / c, or nullptr
  const int* flag;     // device guard flag (nonzero = in range) or nullptr (always run)
  void* o;             // (B,H,T,D) output in the input dtype
  float* o_precise;    // (B,H,T,D) f32 output (SHIFTED with precise output) or nullptr
  float* stat;         // (B,H,T) f32 row statistic
  int B, H, T;
  int log2n;           // n = 2^log2n
  float clamp;         // CLIPPED: positive-score clamp
  int fast_rho;        // SHIFTED: fast rho for the weights
  int inv_stat;        // CLIPPED: 1 -> stat = 1/Z, 0 -> stat = Z^(-1/n)
  int layout;          // storage of q, k, v, o (see head_base)
  // Guarded forward from unscaled queries (the bf16 in-range kernel's FROM_Q form): q holds
  // the raw queries; the kernel writes q_s = round(q * alpha) to q_s_out, its workgroup's
  // guard maxima (||q_s||^2 of its queries, ||k||^2 and |v| of the keys at the same positions)
  // to guard_part[3 * (bh * nqb + query block)], and reads the sink as sink_logit / sink_c
  // (sink_count 1: broadcast; the guard kernel that runs next writes the same value to sink).
  void* q_s_out = nullptr;
  float alpha = 1.0f;
  float* guard_part = nullptr;
  const float* sink_logit = nullptr;
  int sink_count = 0;
  float sink_c = 1.0f;
};

struct AttnBwdParams {
  const void* q;       // q_s
  const void* k;
  const void* v;
  const void* o;       // forward output in the input dtype (the di source, except on the
                       // bf16 shifted fallback, which forms di from its weights)
  const void* dO;      // (B,H,T,D) upstream cotangent in the input dtype
  const float* stat;   // (B,H,T)
  const float* sink;   // (H,) or nullptr
  const int* flag;
  float* di;           // (B,H,T) f32, written by the dQ kernel (bf16) or the pre kernel (f32)
  float* dq_acc;       // (B,H,T,D) f32 accumulator (workspace; f32 inputs only)
  float* sink_part;    // (B*H*nblk) f32 partial sums of mass*di (workspace)
  void* dq;            // (B,H,T,D) output
  void* dk;
  void* dv;
  float* dbeta;        // (H,) gradient w.r.t. sink/c
  int B, H, T;
  int log2n;
  float clamp;
  int fast_rho;
  int inv_stat;
  int mode;            // AttnMode selected by the host when flag is nullptr
  float dq_scale;      // chain-rule factor applied after the slope (alpha), or 1
  int layout;          // storage of q, k, v, o, dO, dq, dk, dv (see head_base)
};

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Storage of the (B, ., ., D) tensors of a call (q, k, v, o, dO, dq, dk, dv): 0 = (B, H, T, D),
// 1 = (B, T, H, D), the projection layout before the head transpose (model.py:167-169, 182).
// Per-row vectors (stat, di) and the internal f32 buffers (o_precise, dq_acc) stay (B, H, T, .).
// head_base is the element offset of position 0 of head bh = b*H + h; positions are
// row_stride elements apart.
__host__ __device__ inline size_t head_base(int bh, int H, int T, int D, int layout) {
  if (!layout) return (size_t)bh * T * D;
  const int b = bh / H, h = bh - b * H;
  return ((size_t)b * T * H + h) * D;
}
__host__ __device__ inline int row_stride(int H, int D, int layout) { return layout ? H * D : D; }
// Bytes from a head's base to the end of its last row (the range of a buffer descriptor whose
// out-of-range rows read as zeros).
__host__ __device__ inline int head_bytes(int T, int ld, int D, int esize) { return ((T - 1) * ld + D) * esize; }

// Unpadded bf16 LDS tiles with CPR 16-byte chunks per row (CPR = 16 for 256-byte rows, 8 for
// 128-byte rows). Chunk c of row r is stored at chunk c ^ swz_chunk<CPR>(r); the mask is
// chosen so that both access patterns of the kernels are free of bank conflicts:
//   * row fragments (ds_read_b128): 16 consecutive rows at one logical chunk land on 16
//     distinct 16-byte bank groups;
//   * transposed fragments (ds_read_b64_tr_b16): 4 consecutive rows (aligned to 4) x 4
//     consecutive chunks (aligned to 4) land on 16 distinct 16-byte bank groups.
template <int CPR>
__device__ __forceinline__ int swz_chunk(int row) {
  static_assert(CPR == 16 || CPR == 8, "row width");
  if constexpr (CPR == 16) return 4 * (row & 3) + ((row >> 2) & 3);
  else return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
}
// Element offset of (row, col) in a swizzled tile.
template <int CPR>
__device__ __forceinline__ int swz_at(int row, int col) {
  return row * (CPR * 8) + (((col >> 3) ^ swz_chunk<CPR>(row)) << 3) + (col & 7);
}
// Transposed 32x32x16 operand fragment from a swizzled tile M[k][n]: lane l receives
// M[k][ncol + l%32] for k = k_lo + (0..3) (slots 0..3) and k_hi + (0..3) (slots 4..7);
// k_lo and k_hi must be multiples of 4 (the ds_read_b64_tr_b16 lane layout is in common.h).
template <int CPR>
__device__ __forceinline__ bf16x8 swz_tr_frag(const bf16* tile, int k_lo, int k_hi, int ncol, int lane) {
  const int i = lane & 15;
  const int col = ncol + ((lane >> 4) & 1) * 16 + 4 * (i & 3);
  const bf16* p0 = tile + swz_at<CPR>(k_lo + (i >> 2), col);
  const bf16* p1 = tile + swz_at<CPR>(k_hi + (i >> 2), col);
  bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p0));
  bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p1));
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Transposed fragment from two precomputed swizzled offsets (ds_read_b64_tr_b16 at
// tile + lo and tile + hi). Both swizzles above repeat every 16 rows, so fragments 16·m rows
// apart share the per-lane offsets and differ only by a constant added to `tile`.
__device__ __forceinline__ bf16x8 tr_frag_at(const bf16* tile, int lo, int hi) {
  bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, tile + lo));
  bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, tile + hi));
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}
// Per-lane column of a transposed fragment read whose block starts at column ncol.
__device__ __forceinline__ int tr_col(int ncol, int lane) {
  return ncol + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
}

// Row padding (elements) of the f32 tiles, which keep a padded row-major layout.
constexpr int F32_PAD = 4;

// Copy of one 64-row tile (rows r0.., D columns) of two (T, D) bf16 matrices into LDS with
// range-checked buffer loads that write LDS directly: lane l of a wave instruction writes 16
// bytes at base + 16 l, so each lane fetches the logical chunk the swizzle places there. Rows
// at or past T lie beyond the descriptors' ranges and land as zeros. The destinations are
// passed through an empty asm so the compiler cannot tie these copies to a particular LDS
// array: it then inserts no wait for them before reads of the other buffer set. Every read
// of a copied tile is preceded by the explicit vmcnt(0) + barrier of the tile before it.
// Instruction J covers rows RPI J + r (r = lane / CPR); its swizzle is swz(r) ^ swz(RPI J), so
// every instruction's lane offset is one XOR of a per-lane chunk term with a wave-uniform
// value: two per-lane registers serve all of them.
// Both matrices have rows `ld` elements apart (ld = D for (B, H, T, D) storage, H*D for
// (B, T, H, D)); the descriptors' ranges end at the head's last row (head_bytes).
// ROWS (64 by default, or 32) is the tile height; the four waves share the copy instructions.
template <int D, int ROWS = 64, int NW = 4>
__device__ __forceinline__ void tile_dma2(bf16* la, bf16* lb, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                          int r0, int wave, int lane, int ld = D) {
  constexpr int CPR = D / 8, RPI = 64 / CPR, PW = ROWS * CPR / 64 / NW;  // PW instructions per wave
  static_assert(PW >= 1 && PW * NW * RPI == ROWS, "tile height");
  auto lla = LDS_PTR(bf16, la);
  auto llb = LDS_PTR(bf16, lb);
  asm volatile("" : "+s"(lla), "+s"(llb));
  const int r = lane / CPR;
  int rowb = r * ld * 2;                                        // per-lane row bytes
  int chunkb = 16 * ((lane % CPR) ^ swz_chunk<CPR>(r));         // per-lane chunk bytes
  asm volatile("" : "+v"(rowb), "+v"(chunkb));                  // computed here, not kept live
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int J = wave * PW + j;
    const int voff = (r0 + RPI * J) * ld * 2 + rowb + (chunkb ^ (16 * swz_chunk<CPR>(RPI * J)));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lla + J * 512, 16, voff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, llb + J * 512, 16, voff, 0, 0, 0);
  }
}
// Instruction pair j of tile_dma2 alone (lets a kernel spread a tile copy over several
// pipeline steps). NW waves share the copy instructions (4 by default).
template <int D, int ROWS = 64, int NW = 4>
__device__ __forceinline__ void tile_dma2_part(bf16* la, bf16* lb, __amdgpu_buffer_rsrc_t ra,
                                               __amdgpu_buffer_rsrc_t rb, int r0, int wave, int lane, int j,
                                               int ld = D) {
  constexpr int CPR = D / 8, RPI = 64 / CPR, PW = ROWS * CPR / 64 / NW;
  auto lla = LDS_PTR(bf16, la);
  auto llb = LDS_PTR(bf16, lb);
  asm volatile("" : "+s"(lla), "+s"(llb));
  const int r = lane / CPR;
  int rowb = r * ld * 2;
  int chunkb = 16 * ((lane % CPR) ^ swz_chunk<CPR>(r));
  asm volatile("" : "+v"(rowb), "+v"(chunkb));
  const int J = wave * PW + j;
  const int voff = (r0 + RPI * J) * ld * 2 + rowb + (chunkb ^ (16 * swz_chunk<CPR>(RPI * J)));
  __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lla + J * 512, 16, voff, 0, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, llb + J * 512, 16, voff, 0, 0, 0);
}

// Instruction order of one pipeline step: NM MFMAs, each followed by a share of the step's
// V VALU instructions, R LDS reads and W LDS writes; nothing moves across the step's end.
template <int NM, int V, int R, int W>
__device__ __forceinline__ void step_order() {
  constexpr int VP = (V + NM - 1) / NM, RP = (R + NM - 1) / NM, WP = (W + NM - 1) / NM;
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (RP > 0 && i * RP < R) __builtin_amdgcn_sched_group_barrier(0x100, RP, 0);
    if (VP > 0 && i * VP < V) __builtin_amdgcn_sched_group_barrier(0x002, VP, 0);
    if (WP > 0 && i * WP < W) __builtin_amdgcn_sched_group_barrier(0x200, WP, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// step_order with the LDS read count given as a value that folds to a constant once the
// caller's loop is unrolled.
template <int NM, int V>
__device__ __forceinline__ void step_order_r(int r) {
  switch (r) {
    case 0: step_order<NM, V, 0, 0>(); break;
    case 2: step_order<NM, V, 2, 0>(); break;
    case 4: step_order<NM, V, 4, 0>(); break;
    case 6: step_order<NM, V, 6, 0>(); break;
    default: step_order<NM, V, 8, 0>(); break;
  }
}

// Fragments of a lane's own row that may lie past T: the caller loads them from the row clamped
// to T - 1 (so every lane loads unconditionally and the loads issue together), and
// keep_own_row zeroes them on lanes whose row is past T. The empty asm keeps the compiler from
// moving the loads behind the lane check (a load per fragment behind a branch, each with a
// wait of its own).
template <int N>
__device__ __forceinline__ void keep_own_row(bf16x8 (&f)[N], bool live) {
#pragma unroll
  for (int s = 0; s < N; ++s) asm volatile("" : "+v"(f[s]));
  const bf16x8 z = {};
#pragma unroll
  for (int s = 0; s < N; ++s) f[s] = live ? f[s] : z;
}
}  // namespace alg
