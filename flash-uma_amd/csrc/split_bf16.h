// fp32 products on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16).
//
// Every fp32 operand x is split exactly into three bf16 values, x = hi + mid + lo, each
// step rounding to nearest-even (hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid);
// both subtractions are exact in fp32 and the remainder after mid has at most 8 significant
// bits, so lo is exact).  A product a*b is then the sum of the nine exact partial products
// of the planes; the three of relative size 2^-24 and below (mid*lo, lo*mid, lo*lo) are
// dropped, leaving six MFMAs per 16-wide K step, accumulated in fp32:
//     a*b ~ hi*hi + hi*mid + mid*hi + hi*lo + mid*mid + lo*hi
// The dropped terms are below the fp32 rounding of the accumulation itself: measured against
// fp64 on the model's GEMM shapes, the split product's error is at or below that of the fp32
// MFMA (v_mfma_f32_32x32x2_f32) computing the same GEMM.
//
// At gfx950's rates (bf16 32x32x16: 32 cycles, fp32 32x32x2: 64 cycles per SIMD) the six
// products take 6 x 32 = 192 cycles per 32x32x16 block against 8 x 64 = 512 for fp32.
//
// LDS layout of one split operand tile (R rows x 16 k, one plane): bf16 rows of 32 bytes,
// two tile rows per 64-byte line; the four 16-byte chunks of a line are XOR-swizzled with
// ((line >> 1) ^ (line >> 2)) & 3, which keeps the MFMA fragment reads (32 consecutive rows,
// one chunk each) and the staging stores free of bank conflicts.
#pragma once
#include "fu_common.h"

namespace fu {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));

// bf16 element offset of 16-byte chunk c (0: k 0..7, 1: k 8..15) of tile row r in a plane
__device__ __forceinline__ int plane_off(int r, int c) {
  const int line = r >> 1;
  return line * 32 + 8 * (((r & 1) * 2 + c) ^ (((line >> 1) ^ (line >> 2)) & 3));
}

// Split 8 floats into three planes of packed bf16 pairs (two elements per conversion).
__device__ __forceinline__ void split3(const float4& a, const float4& b, uint4& H, uint4& Mi, uint4& L) {
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float2v v = {x[2 * t], x[2 * t + 1]};
    const unsigned hu = __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
    const float2v hf = {__builtin_bit_cast(float, hu << 16), __builtin_bit_cast(float, hu & 0xffff0000u)};
    const float2v r1 = v - hf;
    const unsigned mu = __builtin_bit_cast(unsigned, __builtin_convertvector(r1, bf16x2));
    const float2v mf = {__builtin_bit_cast(float, mu << 16), __builtin_bit_cast(float, mu & 0xffff0000u)};
    const float2v r2 = r1 - mf;
    (&H.x)[t] = hu;
    (&Mi.x)[t] = mu;
    (&L.x)[t] = __builtin_bit_cast(unsigned, __builtin_convertvector(r2, bf16x2));
  }
}

// Split 4 floats into three planes of 4 bf16 each (as split3).
__device__ __forceinline__ void split3_4(const float4& a, uint2& H, uint2& Mi, uint2& L) {
  uint4 h, m, l;
  split3(a, a, h, m, l);
  H = make_uint2(h.x, h.y);
  Mi = make_uint2(m.x, m.y);
  L = make_uint2(l.x, l.y);
}

__device__ __forceinline__ void st_planes4(__bf16* p0, int plane_stride, int off, const uint2& H, const uint2& Mi,
                                           const uint2& L) {
  *reinterpret_cast<uint2*>(p0 + off) = H;
  *reinterpret_cast<uint2*>(p0 + plane_stride + off) = Mi;
  *reinterpret_cast<uint2*>(p0 + 2 * plane_stride + off) = L;
}

__device__ __forceinline__ void st_planes(__bf16* p0, int plane_stride, int off, const uint4& H, const uint4& Mi,
                                          const uint4& L) {
  *reinterpret_cast<uint4*>(p0 + off) = H;
  *reinterpret_cast<uint4*>(p0 + plane_stride + off) = Mi;
  *reinterpret_cast<uint4*>(p0 + 2 * plane_stride + off) = L;
}

__device__ __forceinline__ void ld_planes(const __bf16* p0, int plane_stride, int off, bf16x8 (&f)[3]) {
#pragma unroll
  for (int p = 0; p < 3; ++p) f[p] = *reinterpret_cast<const bf16x8*>(p0 + p * plane_stride + off);
}

// The six partial products (plane of a, plane of b), smallest first.  Kernels issue product
// q for all of their accumulators before product q + 1, so consecutive MFMAs are independent.
constexpr int kSplitA[6] = {2, 1, 0, 1, 0, 0};
constexpr int kSplitB[6] = {0, 1, 2, 0, 1, 0};

__device__ __forceinline__ floatx16 mfma_bf16(const bf16x8& a, const bf16x8& b, const floatx16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}

// Matrix-core mode for every fp32 contraction of the library (fu_set_matmul_mode).
enum { FU_MATMUL_SPLIT_BF16 = 0, FU_MATMUL_FP32 = 1, FU_MATMUL_SPLIT_F16 = 2 };
int matmul_mode();

}  // namespace fu
