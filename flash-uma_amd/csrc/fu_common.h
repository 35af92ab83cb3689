// Shared definitions for the FlashUMA gfx950 kernels and their C-ABI entry points.
//
// Every entry point returns an int status (FU_OK or a negative FU_ERR_*), takes raw
// device pointers plus int64 sizes, and launches on the hipStream_t passed as void*.
// No entry point allocates device memory or synchronises the host.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <algorithm>
#include <type_traits>

#include "../../include/flashuma.h"

namespace fu {

// Last error message of the calling host thread; read through fu_last_error().
extern thread_local char g_last_error[512];

inline int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(FU_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return FU_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned int cdiv(int64_t a, int64_t b) { return static_cast<unsigned int>((a + b - 1) / b); }

// Largest grid dimension used by the 1-D launches; kernels grid-stride beyond it.
constexpr int64_t kMaxBlocks = 1 << 20;

// Workgroups of a launch are dealt round-robin over the 8 XCDs (each with its own L2).
// xcd_block renumbers them so that XCD k runs the k-th contiguous eighth of the logical
// workgroups (grid a multiple of 8; identity otherwise).
__device__ __forceinline__ int64_t xcd_block(int64_t b, int64_t nblocks) {
  return (nblocks & 7) == 0 ? (b & 7) * (nblocks >> 3) + (b >> 3) : b;
}

// Wave-per-edge kernels: this workgroup's contiguous edge range [e0, e1).  With the XCD
// renumbering, a receiver's CSR segment (consecutive edges) stays in one workgroup and each
// XCD walks one Morton-ordered eighth of the edges, so receiver and (spatially close)
// sender rows are re-read from that XCD's L2 rather than fetched by every XCD.
__device__ __forceinline__ void block_edge_range(int64_t E, int64_t& e0, int64_t& e1) {
  const int64_t nb = gridDim.x;
  const int64_t chunk = (E + nb - 1) / nb;
  e0 = xcd_block(blockIdx.x, nb) * chunk;
  e0 = e0 < E ? e0 : E;
  e1 = e0 + chunk < E ? e0 + chunk : E;
}

// Grid for block_edge_range: about 4 edges per wave of 4-wave workgroups, a multiple of 8.
inline unsigned int edge_grid(int64_t E) {
  int64_t nb = (E + 15) / 16;
  nb = nb < 8192 ? nb : 8192;
  return static_cast<unsigned int>(((nb + 7) / 8) * 8);
}

// 1 / (1 + exp(-x)).  The quotient is the hardware reciprocal (v_rcp_f32, 1 ulp) refined by
// one Newton-Raphson step, r + r (1 - y r) with fused multiply-adds, instead of the IEEE
// division sequence (5 % of a LayerNorm-SiLU GEMM launch); y = 1 + exp(-x) >= 1, and an
// infinite y (x below about -88) gives 0 as the division does.
__device__ __forceinline__ float sigmoidf_(float x) {
  const float y = 1.0f + expf(-x);
  const float r = __builtin_amdgcn_rcpf(y);
  return y < __builtin_huge_valf() ? fmaf(r, fmaf(-y, r, 1.0f), r) : 0.0f;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
// 16-byte load with the nontemporal hint (operands streamed once)
__device__ __forceinline__ float4 ld4_nt(const float* p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
// 16-byte store with the nontemporal hint (large write-once outputs)
__device__ __forceinline__ void st4_nt(float* p, float4 v) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<f4*>(p));
}

__device__ __forceinline__ float4 operator*(float4 a, float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float4 operator+(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 scale4(float4 a, float s) {
  return make_float4(a.x * s, a.y * s, a.z * s, a.w * s);
}

// Cross-lane exchanges without LDS traffic (gfx950):
//   swap_halves<32>(a, b): v_permlane32_swap; afterwards lanes 0-31 of the first result hold
//     a[0..31] and lanes 32-63 hold b[0..31], the second result holds a[32..63] | b[32..63];
//   swap_halves<16>(a, b): v_permlane16_swap, the same within each pair of 16-lane rows;
//   partner<H>(v) for H = 8, 2, 1: v of lane l ^ H (DPP row_ror:8, quad_perm); for H = 4:
//     v of lane 7 - (l mod 8) in l's 8-lane group (DPP row_half_mirror), which also pairs
//     every lane with bit 2 clear with one with bit 2 set inside the same 8-lane group.
template <int H>
__device__ __forceinline__ void swap_halves(float a, float b, float& lo, float& hi) {
  static_assert(H == 32 || H == 16, "swap_halves: H must be 32 or 16");
  if constexpr (H == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  }
}

template <int H>
__device__ __forceinline__ float partner(float v) {
  constexpr int ctrl = H == 8 ? 0x128 : H == 4 ? 0x141 : H == 2 ? 0x4E : 0xB1;
  static_assert(H == 8 || H == 4 || H == 2 || H == 1, "partner: H must be 8, 4, 2 or 1");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
}

// Sum over each aligned group of G lanes (G = 2, 4, ..., 64); every lane of a group receives
// the group total (the same value in every lane: each step adds commuted operand pairs).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 64) {
    float lo, hi;
    swap_halves<32>(v, v, lo, hi);
    v = lo + hi;
  }
  if constexpr (G >= 32) {
    float lo, hi;
    swap_halves<16>(v, v, lo, hi);
    v = lo + hi;
  }
  if constexpr (G >= 16) v += partner<8>(v);
  if constexpr (G >= 8) v += partner<4>(v);
  if constexpr (G >= 4) v += partner<2>(v);
  if constexpr (G >= 2) v += partner<1>(v);
  return v;
}

// Full-wavefront (64 lanes) sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace fu
