// The resident-panel split-fp16 GEMM pieces shared by fu_linear_resident (gemm_resident.hip)
// and fu_radial_gather_fwd (radial_gather.hip): a workgroup of 4 waves keeps one 128-row panel
// of A (K <= 128) split into fp16 planes in LDS and walks output tiles whose weight fragments
// come pre-split from global memory (split_f16.h: resident_frag_vectors).
#pragma once

#include "split_f16.h"

namespace fu {

constexpr int kResRows = 128;             // rows per workgroup (the panel)
constexpr int kResPlane = kResRows * 16;  // fp16 per plane (one 16-wide chunk of the panel)

// The workgroup's A panel into LDS: thread (r, h) holds k = 16 kc + 8 h .. + 7 of row r for
// every chunk kc (one piece per chunk); a row past M reads the last row, whose outputs are not
// stored.  Writes the fp16 planes of all chunks (or pass 2's residual planes) and the rows'
// unscale factors; returns whether the panel runs pass 2 (uniform over the workgroup).
template <int KC>
__device__ __forceinline__ bool resident_panel(const float* __restrict__ A, int64_t lda, const int* __restrict__ wsum,
                                               __bf16* sp, float* s_rinv, unsigned* s_need, int64_t row0, int64_t M) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = tid >> 1, h = tid & 1;
  const int64_t gr = row0 + r < M ? row0 + r : M - 1;
  const float* pa = A + gr * lda + 8 * h;
  float4 v[KC][2];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    v[kc][0] = ld4(pa + 16 * kc);
    v[kc][1] = ld4(pa + 16 * kc + 4);
  }
  float pm[KC];
  float R = 0.0f;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    pm[kc] = amax8(v[kc][0], v[kc][1]);
    R = fmaxf(R, pm[kc]);
  }
  R = fmaxf(R, __shfl_xor(R, 1));
  const int e = f16_exp_row(R);
  const float sc = pow2i(e);
  bool low = false;
  float pmin = R, pmax = 0.0f;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    low = low || f16_lossy(pm[kc] * sc);
    pmin = fminf(pmin, pm[kc]);
    pmax = fmaxf(pmax, pm[kc]);
  }
  pmin = fminf(pmin, __shfl_xor(pmin, 1));
  pmax = fmaxf(pmax, __shfl_xor(pmax, 1));
  const bool rough = !f16_flat(pmin, pmax);
  // pass 2 of split_f16.h for the whole panel when a piece below the window meets a rough
  // operand on the other side (the weight side from its summary word)
  const int ws = *wsum;
  const bool mine = (low && (ws & 2)) || ((ws & 1) && rough);
  const unsigned long long bal = __ballot(mine);
  if (lane == 0) s_need[wave] = bal != 0ull;
  if (h == 0) s_rinv[r] = pow2i(-e);
  __syncthreads();
  const bool need2 = (s_need[0] | s_need[1] | s_need[2] | s_need[3]) != 0u;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    uint4 H, L;
    const float4 a0 = scale4(v[kc][0], sc), a1 = scale4(v[kc][1], sc);
    if (need2)
      split2h_up(a0, a1, H, L);
    else
      split2h(a0, a1, H, L);
    st_planes2(sp + kc * 2 * kResPlane, kResPlane, plane_off(r, h), H, L);
  }
  __syncthreads();
  return need2;
}

// K loop of one wave over the products q in [Q0, Q1) of kF16A / kF16B for its NI x NJ blocks of
// 32 x 32 (rows wr + 32 i, weight column blocks cb[]): the weight's fragments straight from
// global memory, PD chunks ahead (for PD < KC, sched_barrier(0) keeps the scheduler from
// hoisting all of them, where they would not fit the registers; PD = KC leaves the order to
// the compiler), the A fragments from the resident planes.  LOP: the lo planes are lo'.
template <int KC, int Q0, int Q1, bool LOP, int NI, int NJ, int PD>
__device__ __forceinline__ void resident_kloop(const __bf16* sp, const uint4* __restrict__ wf, const int (&cb)[NJ],
                                               floatx16 (&acc)[NI][NJ], int wr, int fr, int fh) {
  f16x8 bq[KC][NJ][2];
  auto load_b = [&](int kc) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t base = ((int64_t)cb[j] * KC + kc) * 3 * 64;
      bq[kc][j][0] = __builtin_bit_cast(f16x8, wf[base]);
      bq[kc][j][1] = __builtin_bit_cast(f16x8, wf[base + (LOP ? 128 : 64)]);
    }
  };
#pragma unroll
  for (int kc = 0; kc < PD && kc < KC; ++kc) load_b(kc);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    if (kc + PD < KC) load_b(kc + PD);
    if constexpr (PD < KC) __builtin_amdgcn_sched_barrier(0);
    f16x8 aq[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i) ld_planes2(sp + kc * 2 * kResPlane, kResPlane, plane_off(wr + 32 * i + fr, fh), aq[i]);
#pragma unroll
    for (int q = Q0; q < Q1; ++q)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma_f16(aq[i][kF16A[q]], bq[kc][j][kF16B[q]], acc[i][j]);
    if constexpr (PD < KC) __builtin_amdgcn_sched_barrier(0);
  }
}

// The whole K reduction of one tile (pass 0, or pass 2's two loops), accumulators zeroed here.
template <int KC, int NI, int NJ, int PD>
__device__ __forceinline__ void resident_tile(const __bf16* sp, const uint4* __restrict__ wf, const int (&cb)[NJ],
                                              floatx16 (&acc)[NI][NJ], bool need2, int wr, int fr, int fh) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int t = 0; t < 16; ++t) acc[i][j][t] = 0.0f;
  if (!need2) {
    resident_kloop<KC, 0, 3, false, NI, NJ, PD>(sp, wf, cb, acc, wr, fr, fh);
  } else {
    resident_kloop<KC, 0, 2, true, NI, NJ, PD>(sp, wf, cb, acc, wr, fr, fh);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[i][j][t] *= F16_LO_DOWN;
    resident_kloop<KC, 2, 3, true, NI, NJ, PD>(sp, wf, cb, acc, wr, fr, fh);
  }
}


}  // namespace fu
