// fp32 products on the fp16 matrix cores (v_mfma_f32_32x32x16_f16): three MFMAs per 16-wide
// K step instead of the six of the bf16 split (split_bf16.h).
//
// Every fp32 operand row (a row of A, or a row of W, i.e. one output column) gets a power-of-two
// scale 2^e, and each element x of it is split into two fp16 values
//     x 2^e = hi + lo,   hi = fp16(x 2^e),   lo = fp16(x 2^e - hi)
// (round to nearest even; the subtraction is exact in fp32).  While lo is a normal fp16
// (|x 2^e| >= 2^-3) hi + lo carries 22 significant bits of x 2^e; below that it is within 2^-25
// of it.  A product is then
//     a b 2^(ea + eb) ~ hi_a hi_b + hi_a lo_b + lo_a hi_b
// with each partial product exact in the fp32 accumulator and the dropped lo_a lo_b of relative
// size 2^-22.  The accumulated output is multiplied by 2^-ea and 2^-eb afterwards (exact).
//
// Window.  The kernels stage a row in pieces (8 consecutive k of a row in the real GEMM, 4 of
// each of a_r and a_i in the complex layer).  A piece is inside the window at a scale when its
// largest scaled magnitude is at or above 2^-3 (or it is zero) and no piece overflowed (largest
// fp16 65504).  Inside it every element keeps 22 bits relative to the largest element of its
// piece: |error(x)| <= 2^-22 max(|x|, max |piece|) 2^-e.  A piece below the window has the
// absolute error 2^-25 2^-e of the scale instead, which matters only when it meets elements of
// the other operand that are large next to those its row's large pieces meet.  So a row is
// called flat when its smallest piece maximum (zero pieces included) is at least 2^-6 of its
// largest, and a tile is accepted from a pass unless an operand has a piece below the window
// while the other operand has a row that is not flat (or a piece overflowed).  The passes:
//  0. scales from the first chunk: the maximum m of the row's first 16 elements is mapped to
//     [2^6, 2^7) (256x of headroom above it), with no pass over the data; the pieces are
//     tracked as they are staged (A's are not when a pre-split weight's columns are all flat
//     with no piece below the window: the rule above can then not fail on A's account);
//  1. exact scales, from a pass over the rows: e = 14 - floor(log2 R), R the row's largest
//     magnitude (R 2^e in [2^14, 2^15)), so pieces down to 2^-17 R stay in the window.  Pass 0
//     is skipped for rows of up to F16_PREPASS_CHUNKS chunks and for a tile with a zero first
//     chunk (nothing to scale from);
//  2. for a tile that pass 1 cannot hold (a piece below 2^-17 of its row's maximum against a
//     rough other operand): exact scales, and the K loop runs twice, first with the products
//     hi_a lo'_b + lo'_a hi_b of the residuals scaled up, lo' = fp16((x 2^e - hi) 2^11),
//     accumulated, then multiplied by 2^-11 (exact), then hi_a hi_b added.  lo' is normal down
//     to |x 2^e| ~ 2^-13, so every element down to 2^-27 R keeps 22 bits:
//     |error(x)| <= 2^-22 |x| + 2^-50 R.
// The rules work on pieces, not elements: an element far below the largest one of its own
// piece that meets a large element of the other operand is not seen.  Rows whose magnitude
// changes by blocks or smoothly along K are covered.
// A row of zeros keeps e = 0.
#pragma once
#include "split_bf16.h"

namespace fu {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Split 8 floats (already scaled) into the hi and lo planes of packed fp16 pairs.
__device__ __forceinline__ void split2h(const float4& a, const float4& b, uint4& H, uint4& L) {
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float2v v = {x[2 * t], x[2 * t + 1]};
    const f16x2 h = __builtin_convertvector(v, f16x2);
    const float2v r = v - __builtin_convertvector(h, float2v);
    (&H.x)[t] = __builtin_bit_cast(unsigned, h);
    (&L.x)[t] = __builtin_bit_cast(unsigned, __builtin_convertvector(r, f16x2));
  }
}

// As split2h, with the lo pieces scaled by 2^11 (pass 2 of the window rules above: the
// residual x - hi is exact, and so is its product with a power of two).
__device__ __forceinline__ void split2h_up(const float4& a, const float4& b, uint4& H, uint4& L) {
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float2v v = {x[2 * t], x[2 * t + 1]};
    const f16x2 h = __builtin_convertvector(v, f16x2);
    const float2v r = (v - __builtin_convertvector(h, float2v)) * 2048.0f;
    (&H.x)[t] = __builtin_bit_cast(unsigned, h);
    (&L.x)[t] = __builtin_bit_cast(unsigned, __builtin_convertvector(r, f16x2));
  }
}

// Split 4 floats (already scaled) into 4 fp16 of each plane.
__device__ __forceinline__ void split2h_4(const float4& a, uint2& H, uint2& L) {
  uint4 h, l;
  split2h(a, a, h, l);
  H = make_uint2(h.x, h.y);
  L = make_uint2(l.x, l.y);
}

__device__ __forceinline__ void split2h_4_up(const float4& a, uint2& H, uint2& L) {
  uint4 h, l;
  split2h_up(a, a, h, l);
  H = make_uint2(h.x, h.y);
  L = make_uint2(l.x, l.y);
}

__device__ __forceinline__ void st_planes2(__bf16* p0, int plane_stride, int off, const uint4& H, const uint4& L) {
  *reinterpret_cast<uint4*>(p0 + off) = H;
  *reinterpret_cast<uint4*>(p0 + plane_stride + off) = L;
}

__device__ __forceinline__ void st_planes2_4(__bf16* p0, int plane_stride, int off, const uint2& H, const uint2& L) {
  *reinterpret_cast<uint2*>(p0 + off) = H;
  *reinterpret_cast<uint2*>(p0 + plane_stride + off) = L;
}

__device__ __forceinline__ void ld_planes2(const __bf16* p0, int plane_stride, int off, f16x8 (&f)[2]) {
  f[0] = *reinterpret_cast<const f16x8*>(p0 + off);
  f[1] = *reinterpret_cast<const f16x8*>(p0 + plane_stride + off);
}

// The three partial products (plane of a, plane of b), smallest first: lo*hi, hi*lo, hi*hi.
constexpr int kF16A[3] = {1, 0, 0};
constexpr int kF16B[3] = {0, 1, 0};

__device__ __forceinline__ floatx16 mfma_f16(const f16x8& a, const f16x8& b, const floatx16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
}

// 2^e for e in [-126, 127].
__device__ __forceinline__ float pow2i(int e) { return __uint_as_float((unsigned)(127 + e) << 23); }

__device__ __forceinline__ int f16_exp_of(float m, int target) {
  const int E = (int)((__float_as_uint(m) >> 23) & 0xff) - 127;  // floor(log2 m) for normal m
  const int e = target - E;
  return m > 0.0f ? (e < -126 ? -126 : e > 126 ? 126 : e) : 0;
}
// exact scale of a row whose largest magnitude is R: R 2^e in [2^14, 2^15)
__device__ __forceinline__ int f16_exp_row(float R) { return f16_exp_of(R, 14); }
// scale from a first chunk whose largest magnitude is m: m 2^e in [2^6, 2^7)
__device__ __forceinline__ int f16_exp_chunk(float m) { return f16_exp_of(m, 6); }
// a row whose scaled largest magnitude Rs left the window (Rs = 0: a row of zeros, in the window)
__device__ __forceinline__ bool f16_outside(float Rs) { return !(Rs < 32768.0f) || (Rs > 0.0f && Rs < 0.125f); }

// A staged piece whose largest scaled magnitude m (>= 0) is nonzero and below 2^-3: its lo
// pieces are fp16 subnormals, so the piece is outside the window (m = 0: zeros, exact).
__device__ __forceinline__ bool f16_lossy(float m) { return (__float_as_uint(m) - 1u) < 0x3dffffffu; }
// A row is flat when its smallest piece maximum (zero pieces included) is at least 2^-6 of its
// largest (a row of zeros is flat).
__device__ __forceinline__ bool f16_flat(float pmin, float pmax) { return pmin >= pmax * 0.015625f; }
// Window verdict bits of a tile (OR over its rows): a piece of A (W) below the window; a row of A
// (W) that is not flat; an overflowed piece.
constexpr unsigned F16_LOW_A = 1u, F16_ROUGH_A = 2u, F16_LOW_W = 4u, F16_ROUGH_W = 8u, F16_OVERFLOW = 16u;
// Pieces below the window count only against a rough other operand: a flat operand's elements
// that meet them are within 2^6 of those that meet its large pieces.
__device__ __forceinline__ bool f16_needs_exact(unsigned t) {
  return ((t & F16_LOW_A) && (t & F16_ROUGH_W)) || ((t & F16_LOW_W) && (t & F16_ROUGH_A));
}
// The residual factor of pass 2 and its inverse.
constexpr float F16_LO_UP = 2048.0f, F16_LO_DOWN = 1.0f / 2048.0f;

__device__ __forceinline__ float amax4(const float4& v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}
// largest magnitude of 8 values as a tree of three-operand maxima (v_max3 with |.| modifiers)
__device__ __forceinline__ float amax8(const float4& a, const float4& b) {
  const float m0 = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fabsf(a.z));
  const float m1 = fmaxf(fmaxf(fabsf(a.w), fabsf(b.x)), fabsf(b.y));
  const float m2 = fmaxf(fmaxf(fabsf(b.z), fabsf(b.w)), m0);
  return fmaxf(m1, m2);
}

// Rows (or operands) of up to this many 16-wide chunks get the exact scale from a pre-pass.
constexpr int F16_PREPASS_CHUNKS = 4;

// A pre-split real weight W (N, K) (fu_linear_weight_split), one after the other:
//  * fp16 planes in MFMA-fragment order: per (32-column block, 16-k chunk), 3 x 64 lanes x 16 B:
//    hi, lo and lo' = 2^11 lo of the column scaled by its exact power of two 2^e(n);
//  * the unscale factors 2^-e(n), one float per column of the 32-column blocks;
//  * one int per column of the 32-column blocks: bit 0 set when a piece (8 consecutive k from a
//    multiple of 8) of the column is nonzero and below the window at the column's scale, bit 1
//    when the column is not flat;
//  * one int (padded to 16 bytes): the OR of the column flags.
__host__ __device__ inline int64_t resident_frag_vectors(int32_t N, int32_t K) {
  return (int64_t)((N + 31) / 32) * (K / 16) * 3 * 64;
}
__host__ __device__ inline int64_t resident_cols(int32_t N) { return (int64_t)((N + 31) / 32) * 32; }

}  // namespace fu
