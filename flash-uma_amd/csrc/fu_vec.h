// Per-lane channel vectors for the wave-per-row kernels: a wave64 covers one C-wide feature
// row with CPL = C/64 consecutive channels per lane, so every row access is one coalesced
// 256*CPL-byte transaction.
#pragma once
#include "fu_common.h"

namespace fu {

template <int CPL>
struct Vec {
  float v[CPL];
  __device__ __forceinline__ float& operator[](int k) { return v[k]; }
  __device__ __forceinline__ const float& operator[](int k) const { return v[k]; }
};

template <int CPL>
__device__ __forceinline__ Vec<CPL> vload(const float* p) {
  Vec<CPL> r;
  if constexpr (CPL == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
  } else if constexpr (CPL == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r.v[0] = t.x; r.v[1] = t.y;
  } else {
#pragma unroll
    for (int k = 0; k < CPL; ++k) r.v[k] = p[k];
  }
  return r;
}

// vload with the nontemporal hint: for large read-once streams, so that they do not evict
// rows that other waves read again (the node rows of a gather).
template <int CPL>
__device__ __forceinline__ Vec<CPL> vload_nt(const float* p) {
  Vec<CPL> r;
  if constexpr (CPL == 4) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
  } else if constexpr (CPL == 2) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 t = __builtin_nontemporal_load(reinterpret_cast<const f2*>(p));
    r.v[0] = t.x; r.v[1] = t.y;
  } else {
#pragma unroll
    for (int k = 0; k < CPL; ++k) r.v[k] = __builtin_nontemporal_load(p + k);
  }
  return r;
}

// vstore with the nontemporal hint: for large write-once streams that no kernel re-reads
// while they could still sit in L2.
template <int CPL>
__device__ __forceinline__ void vstore_nt(float* p, const Vec<CPL>& a) {
  if constexpr (CPL == 4) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = {a.v[0], a.v[1], a.v[2], a.v[3]};
    __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
  } else if constexpr (CPL == 2) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a.v[0], a.v[1]};
    __builtin_nontemporal_store(v, reinterpret_cast<f2*>(p));
  } else {
#pragma unroll
    for (int k = 0; k < CPL; ++k) __builtin_nontemporal_store(a.v[k], p + k);
  }
}

template <int CPL>
__device__ __forceinline__ void vstore(float* p, const Vec<CPL>& a) {
  if constexpr (CPL == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(a.v[0], a.v[1], a.v[2], a.v[3]);
  } else if constexpr (CPL == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(a.v[0], a.v[1]);
  } else {
#pragma unroll
    for (int k = 0; k < CPL; ++k) p[k] = a.v[k];
  }
}

template <int CPL>
__device__ __forceinline__ Vec<CPL> vzero() {
  Vec<CPL> r;
#pragma unroll
  for (int k = 0; k < CPL; ++k) r.v[k] = 0.0f;
  return r;
}

template <int CPL>
__device__ __forceinline__ Vec<CPL> vmul(const Vec<CPL>& a, const Vec<CPL>& b) {
  Vec<CPL> r;
#pragma unroll
  for (int k = 0; k < CPL; ++k) r.v[k] = a.v[k] * b.v[k];
  return r;
}

template <int CPL>
__device__ __forceinline__ Vec<CPL> vadd(const Vec<CPL>& a, const Vec<CPL>& b) {
  Vec<CPL> r;
#pragma unroll
  for (int k = 0; k < CPL; ++k) r.v[k] = a.v[k] + b.v[k];
  return r;
}

template <int CPL>
__device__ __forceinline__ Vec<CPL> vscale(const Vec<CPL>& a, float s) {
  Vec<CPL> r;
#pragma unroll
  for (int k = 0; k < CPL; ++k) r.v[k] = a.v[k] * s;
  return r;
}

template <int CPL>
__device__ __forceinline__ float vdot(const Vec<CPL>& a, const Vec<CPL>& b) {
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) s += a.v[k] * b.v[k];
  return s;
}

// Recursive halving over lane bits H = V/2, V/4, ..., 1: at each step a lane keeps half of its
// values (the upper half if bit H of its index is set) and adds its partner's copy of that
// half, the partner having the opposite bit H and the same higher bits.  Afterwards lane l
// holds the sum of value (l mod V) over the V lanes that share l's bits above log2(V).
// H = 32 and 16 use the permlane swaps (both halves exchanged in one instruction, no
// selects), H <= 8 DPP moves.
template <int V>
__device__ __forceinline__ float halve_values(const float (&vals)[V], int lane) {
  if constexpr (V == 1) {
    return vals[0];
  } else {
    constexpr int H = V / 2;
    float nxt[H];
    if constexpr (H >= 16) {
#pragma unroll
      for (int k = 0; k < H; ++k) {
        float lo, hi;
        swap_halves<H>(vals[k], vals[k + H], lo, hi);
        nxt[k] = lo + hi;
      }
    } else {
      const bool upper = (lane & H) != 0;
#pragma unroll
      for (int k = 0; k < H; ++k) {
        const float send = upper ? vals[k] : vals[k + H];
        const float keep = upper ? vals[k + H] : vals[k];
        nxt[k] = keep + partner<H>(send);
      }
    }
    return halve_values<H>(nxt, lane);
  }
}

// Sum V per-lane values over all 64 lanes of a wave (V a power of two <= 64).  Lane l
// receives the total of value (l mod V).  Costs V - 1 exchanges plus 6 - log2 V full-wave
// steps, instead of 6 V for V independent reductions.
template <int V>
__device__ __forceinline__ float wave_multi_sum(const float (&vals)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
  float r = halve_values<V>(vals, lane);
  if constexpr (V < 64) {
    // the V-lane groups hold equal value sets: add them across the remaining lane bits
    if constexpr (V <= 16) {
      float lo, hi;
      swap_halves<16>(r, r, lo, hi);
      r = lo + hi;
    }
    if constexpr (V <= 32) {
      float lo, hi;
      swap_halves<32>(r, r, lo, hi);
      r = lo + hi;
    }
    static_assert(V >= 16, "wave_multi_sum: V below 16 needs more cross-group steps");
  }
  return r;
}

}  // namespace fu
