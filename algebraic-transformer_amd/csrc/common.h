// Shared device helpers for the gfx950 algebraic attention / head kernels.
//
// MFMA lane layouts used throughout (wave64; verified on gfx950 with an in-bounds probe):
//   v_mfma_f32_32x32x16_bf16  A: lane l holds A[m = l%32][k = 8*(l/32) + j], j < 8
//                             B: lane l holds B[k = 8*(l/32) + j][n = l%32]
//                             C: lane l, reg i holds C[m = 8*(i/4) + 4*(l/32) + i%4][n = l%32]
//   v_mfma_f32_32x32x2f32     A: A[m = l%32][k = l/32], B: B[k = l/32][n = l%32], C as above.
//   v_mfma_f32_16x16x32_bf16  A: lane l holds A[m = l%16][k = 8*(l/16) + j], j < 8
//                             B: lane l holds B[k = 8*(l/16) + j][n = l%16]
//                             C: lane l, reg i holds C[m = 4*(l/16) + i][n = l%16]
// Any bijection of k onto (lane half, slot) gives the same product as long as A and B use
// the same one; the kernels exploit this to feed a C tile straight back as an operand.
//
//   ds_read_b64_tr_b16 (gfx950): inside each group of 16 lanes, lane i receives element i%4
//   of the 4-element (8-byte) chunk addressed by lane 4*e + i/4, for e = 0..3. So if lane j
//   of the group addresses &M[k0 + j/4][n0 + 4*(j%4)] of a row-major tile M[k][n], lane i
//   receives M[k0 + e][n0 + i], e = 0..3: a transposed operand fragment in one instruction.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// Word 3 of a raw buffer descriptor on gfx9-class targets: 32-bit data format, no swizzle.
#define BUF_RSRC_WORD3 0x00020000
// Cache-policy bit of buffer instructions (aux operand) marking an access non-temporal.
#define BUF_NT 2

namespace alg {
// s_waitcnt immediate for vmcnt(n) with expcnt/lgkmcnt left at their maxima (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int VMCNT0 = vmcnt_imm(0);
}  // namespace alg

namespace alg {

__device__ __forceinline__ floatx16 mfma_bf16(const bf16x8& a, const bf16x8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16_bf16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma_f32(float a, float b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Raw hardware reciprocal square root (v_rsq_f32); the only transcendental on the path.
__device__ __forceinline__ float rsq(float x) { return __builtin_amdgcn_rsqf(x); }

// Fast rho (flash.py:83-88): rho = x + (1+x^2) rsqrt(1+x^2); also returns r = rsqrt(1+x^2).
__device__ __forceinline__ float rho_fast(float x, float& r) {
  float rad = __builtin_fmaf(x, x, 1.0f);
  r = rsq(rad);
  return __builtin_fmaf(rad, r, x);
}
__device__ __forceinline__ float rho_fast(float x) {
  float r;
  return rho_fast(x, r);
}
// Stable rho (algebraic.py:31-35 / flash.py:76-80): |x| + sqrt(1+x^2), reciprocal for x < 0.
__device__ __forceinline__ float rho_exact(float x, float& r) {
  float rad = __builtin_fmaf(x, x, 1.0f);
  r = rsq(rad);
  float t = __builtin_fmaf(rad, r, __builtin_fabsf(x));
  return x >= 0.0f ? t : 1.0f / t;
}
__device__ __forceinline__ float rho_exact(float x) {
  float r;
  return rho_exact(x, r);
}

// x^n for n a power of two (repeated squaring; flash.py:95-104 for those n).
template <int N>
__device__ __forceinline__ float ipow(float x) {
  static_assert(N >= 1 && (N & (N - 1)) == 0, "power of two");
  if constexpr (N == 1) return x;
  else {
    float y = ipow<N / 2>(x);
    return y * y;
  }
}
// t^(2^L2N) with the exponent fixed at compile time (L2N > 0) or given at run time (L2N == 0).
template <int L2N>
__device__ __forceinline__ float pow2n(float t, int log2n) {
  if constexpr (L2N > 0) {
#pragma unroll
    for (int e = 0; e < L2N; ++e) t = t * t;
  } else {
    for (int e = 0; e < log2n; ++e) t = t * t;
  }
  return t;
}

// Runtime power-of-two exponent (cold paths only).
__device__ __forceinline__ float ipow_rt(float x, int n) {
  float out = x;
  while (n > 1) { out = out * out; n >>= 1; }
  return out;
}
// l^(-1/n) for n a power of two (flash.py:107-114): rsqrt, then y *= rsqrt(y).
__device__ __forceinline__ float inv_root(float l, int n) {
  float y = rsq(l);
  for (int k = n / 2; k > 1; k >>= 1) y = y * rsq(y);
  return y;
}

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }
// Two floats rounded to bf16 and packed (a in the low half). Built as a 2-vector so the
// compiler emits one v_cvt_pk_bf16_f32 (the shift-and-or form cost two conversions and a
// merge per pair).
__device__ __forceinline__ unsigned int pack_bf16x2(float a, float b) {
  typedef bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = f2bf(a);
  v[1] = f2bf(b);
  return __builtin_bit_cast(unsigned int, v);
}

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Load 8 consecutive bf16 (16 bytes) from global memory.
__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Transposed fragment read for a 32x32x16 operand from a row-major bf16 LDS tile M[k][n]
// with row pitch `pitch` elements. Lane l receives M[krow(h,j)][ncol + l%32] for the eight
// slots j, where the k rows are k_lo + (0..3) for slots 0..3 and k_hi + (0..3) for slots
// 4..7 (k_lo/k_hi may depend on the lane half h = l/32).
__device__ __forceinline__ bf16x8 lds_tr_frag(const bf16* tile, int pitch, int k_lo, int k_hi, int ncol,
                                              int lane) {
  const int i = lane & 15;
  const int n0 = ncol + ((lane >> 4) & 1) * 16;
  const bf16* p0 = tile + (k_lo + (i >> 2)) * pitch + n0 + 4 * (i & 3);
  const bf16* p1 = tile + (k_hi + (i >> 2)) * pitch + n0 + 4 * (i & 3);
  bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p0));
  bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, p1));
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Pack accumulator registers [i0, i0+8) of a C tile into a bf16 operand fragment.
__device__ __forceinline__ bf16x8 pack8(const floatx16& c, int i0) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = f2bf(c[i0 + j]);
  return r;
}

}  // namespace alg
