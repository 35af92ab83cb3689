// Radial output layer fused with the gather-rotate forward (lmax = 2, C = 128).
//
// Each block's radial output rad = h2 W3^T + b3 (model.py:149, K = C = 128, N = 12 C) is read
// exactly once in the forward, by the gather (ops/gather.py:114-154: X = rad * (D x[node]) per
// side, slot and channel).  The resident GEMM of gemm_resident.hip already holds one 128-row
// panel of h2 (128 edges) in LDS and walks every output column, so its epilogue can form the
// gather's outputs itself: rad never makes the HBM round trip into a separate gather kernel,
// which removes that kernel's launch and its 1.5 GB read of rad per block at bcc Fe.  rad is
// still written (the gather backward reads it).
//
// Column order.  The weight's 12 C rows are permuted (fu_radial_gather_perm) so that output
// tile t (96 columns, t = 0..15) holds three radial blocks of one side for 32 channels: side
// so = t / 8, channel group cg = (t / 2) % 4, blocks q = 3 (t % 2) + j, j = 0..2 (the m = 0 blocks
// q = 0, 1, 2 or the |m| = 1, 1, 2 blocks q = 3, 4, 5); column 96 t + 32 j + ch is radial column
// slot_rad(so, q) C + 32 cg + ch of the natural order.  Each of the 4 waves computes 32 rows of
// every tile (three 32 x 32 blocks: 48 accumulators, so that the epilogue's node rows and Wigner
// scalars fit beside them at two workgroups per CU).  In the epilogue a lane takes one edge
// (slice row) and 4 channels: it reads the edge's node row pieces (9 or 8 coefficients x 16
// bytes) and Wigner scalars, rotates them exactly as the gather kernel does (same products in
// the same order, so X is bitwise the gather's) and writes rad and the tile's X slots as
// 16-byte pieces (8 lanes of one edge cover 128 contiguous bytes).
//
// The K loop and the panel are those of fu_linear_resident (split-fp16, weight fragments
// straight from global memory, pass 2 of split_f16.h for a panel the window rule sends there).
#include "edge_layout.h"
#include "split_f16.h"

namespace fu {
namespace rg {

constexpr int RBM = 128;          // rows (edges) per workgroup
constexpr int KC = 8;             // 16-wide K chunks: K = 128
constexpr int RPLANE = RBM * 16;  // fp16 per plane (one chunk of the panel)
constexpr int CH = 128;           // channels
constexpr int NT = 16;            // output tiles: 2 sides x 4 channel groups x 2 halves of the radial blocks
constexpr int TN = 96;            // columns per tile: 3 radial blocks x 32 channels
constexpr int RES3 = 96 + 8;      // floats per row of a wave's epilogue slice: 4 RES3 = 32 mod 64 banks

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
    st_planes2(sp + kc * 2 * RPLANE, RPLANE, plane_off(r, h), H, L);
  }
  __syncthreads();
  return need2;
}

// K loop of one wave over the products q in [Q0, Q1) of kF16A / kF16B for its 2 x NJ blocks of
// 32 x 32 (rows wr .. wr + 63, weight column blocks cb[]): the weight's fragments straight from
// global memory, PD chunks ahead (sched_barrier(0) keeps the scheduler from hoisting all of them:
// with 3 column blocks that does not fit the registers), the A fragments from the resident
// planes.  LOP: the lo planes are lo'.
template <int KC, int Q0, int Q1, bool LOP, int NI, int NJ, int PD = 2>
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
    __builtin_amdgcn_sched_barrier(0);
    f16x8 aq[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i) ld_planes2(sp + kc * 2 * RPLANE, RPLANE, plane_off(wr + 32 * i + fr, fh), aq[i]);
#pragma unroll
    for (int q = Q0; q < Q1; ++q)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma_f16(aq[i][kF16A[q]], bq[kc][j][kF16B[q]], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The whole K reduction of one tile (pass 0, or pass 2's two loops), accumulators zeroed here.
template <int KC, int NI, int NJ>
__device__ __forceinline__ void resident_tile(const __bf16* sp, const uint4* __restrict__ wf, const int (&cb)[NJ],
                                              floatx16 (&acc)[NI][NJ], bool need2, int wr, int fr, int fh) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int t = 0; t < 16; ++t) acc[i][j][t] = 0.0f;
  if (!need2) {
    resident_kloop<KC, 0, 3, false, NI, NJ>(sp, wf, cb, acc, wr, fr, fh);
  } else {
    resident_kloop<KC, 0, 2, true, NI, NJ>(sp, wf, cb, acc, wr, fr, fh);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[i][j][t] *= F16_LO_DOWN;
    resident_kloop<KC, 2, 3, true, NI, NJ>(sp, wf, cb, acc, wr, fr, fh);
  }
}


__device__ __forceinline__ float4 rot3(float w0, float w1, float w2, const float4& a, const float4& b,
                                       const float4& c) {
  return make_float4(w0 * a.x + w1 * b.x + w2 * c.x, w0 * a.y + w1 * b.y + w2 * c.y, w0 * a.z + w1 * b.z + w2 * c.z,
                     w0 * a.w + w1 * b.w + w2 * c.w);
}

__device__ __forceinline__ float4 rot5(const float* w, const float4 (&v)[9]) {
  return make_float4(w[0] * v[4].x + w[1] * v[5].x + w[2] * v[6].x + w[3] * v[7].x + w[4] * v[8].x,
                     w[0] * v[4].y + w[1] * v[5].y + w[2] * v[6].y + w[3] * v[7].y + w[4] * v[8].y,
                     w[0] * v[4].z + w[1] * v[5].z + w[2] * v[6].z + w[3] * v[7].z + w[4] * v[8].z,
                     w[0] * v[4].w + w[1] * v[5].w + w[2] * v[6].w + w[3] * v[7].w + w[4] * v[8].w);
}

__device__ __forceinline__ float4 mul4(const float4& a, const float4& b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

template <int LAYOUT>
__global__ __launch_bounds__(256, 2) void radial_gather_kernel(
    const float* __restrict__ A, int64_t lda, const uint4* __restrict__ W2, const float* __restrict__ cinv,
    const int* __restrict__ wsum, const float* __restrict__ bias, const float* __restrict__ x,
    const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j, const float* __restrict__ wig,
    const float* __restrict__ csd, const int64_t* __restrict__ batch, float* __restrict__ rad,
    float* __restrict__ X0, float* __restrict__ X1, float* __restrict__ X2, int64_t M) {
  __shared__ __attribute__((aligned(16))) __bf16 sp[KC * 2 * RPLANE];  // [chunk][hi, lo or lo'][plane]
  __shared__ float s_rinv[RBM];
  __shared__ unsigned s_need[4];
  __shared__ __attribute__((aligned(16))) float s_ep[4][8 * RES3];  // one slice per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * RBM;
  const bool need2 = resident_panel<KC>(A, lda, wsum, sp, s_rinv, s_need, row0, M);

  const int fr = lane & 31, fh = lane >> 5;
  const int wr = 32 * wave;                 // this wave's 32 rows of every tile
  const int rr = lane >> 3, c4 = lane & 7;  // epilogue: slice row (edge), channel quad
  const uint4* wf = W2 + lane;
  float* ep = s_ep[wave];
  // the node and system ids of the 4 edges this lane takes in the epilogues (rows
  // wr + 8 g8 + rr; a row past M takes the last edge, nothing of it is stored), both sides,
  // loaded once: every tile's slices then issue their row loads at once
  int32_t nid[2][4], bid[2][4];
#pragma unroll
  for (int g8 = 0; g8 < 4; ++g8) {
    const int64_t e = row0 + wr + 8 * g8 + rr;
    const int64_t ec = e < M ? e : M - 1;
    nid[0][g8] = (int32_t)idx_i[ec];
    nid[1][g8] = (int32_t)idx_j[ec];
  }
#pragma unroll
  for (int g8 = 0; g8 < 4; ++g8) {
    bid[0][g8] = (int32_t)batch[nid[0][g8]];
    bid[1][g8] = (int32_t)batch[nid[1][g8]];
  }
  for (int t = 0; t < NT; ++t) {
    // tile t: side so, channel group cg, radial blocks q = 3 hq .. 3 hq + 2 (hq 0: m = 0)
    const int so = t >> 3, cg = (t >> 1) & 3, hq = t & 1;
    int cb[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) cb[j] = 3 * t + j;
    floatx16 acc[1][3];
    resident_tile<KC, 1, 3>(sp, wf, cb, acc, need2, wr, fr, fh);
    const int ch = 32 * cg + 4 * c4;  // this lane's first channel
    const int col0 = t * TN + 4 * c4;
#pragma unroll
    for (int g8 = 0; g8 < 4; ++g8) {
      // one slice at a time: its loads are not hoisted above the previous slice's stores
      __builtin_amdgcn_sched_barrier(0);
      // lane (fr, fh) holds column fr of each block and rows 8 (s / 4) + 4 fh + s % 4
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) ep[(4 * fh + s) * RES3 + 32 * j + fr] = acc[0][j][4 * g8 + s];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int rb = wr + 8 * g8;  // first row of the slice in the panel
      const int64_t e = row0 + rb + rr;
      if (e < M) {
        const float rf = s_rinv[rb + rr];
        float4 rv[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const float4 a4 = ld4(ep + rr * RES3 + 32 * j + 4 * c4);
          const float4 cs = ld4(cinv + col0 + 32 * j);
          const float4 bv = bias ? ld4(bias + col0 + 32 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
          rv[j] = make_float4(a4.x * rf * cs.x + bv.x, a4.y * rf * cs.y + bv.y, a4.z * rf * cs.z + bv.z,
                              a4.w * rf * cs.w + bv.w);
        }
        float* re = rad + e * 12 * CH + ch;
#pragma unroll
        for (int j = 0; j < 3; ++j) st4_nt(re + slot_rad<LAYOUT>(so, 3 * hq + j) * CH, rv[j]);
        const int64_t node = so ? nid[1][g8] : nid[0][g8];
        const float* xn = x + node * 9 * CH + ch;
        const float* w = wig + e * 34;
        float4 v[9];
#pragma unroll
        for (int k = 1; k < 9; ++k) v[k] = ld4(xn + k * CH);
        if (hq == 0) {
          // X_m0 slots q = 0, 1, 2: rotated coefficients 0, 2, 6
          const float4 x0 = ld4(xn), c0 = ld4(csd + (int64_t)(so ? bid[1][g8] : bid[0][g8]) * CH + ch);
          v[0] = make_float4(x0.x + c0.x, x0.y + c0.y, x0.z + c0.z, x0.w + c0.w);
          float* o0 = X0 + e * 6 * CH + ch;
          st4_nt(o0 + slot_m0<LAYOUT>(so, 0) * CH, mul4(v[0], rv[0]));
          st4_nt(o0 + slot_m0<LAYOUT>(so, 1) * CH, mul4(rot3(w[3], w[4], w[5], v[1], v[2], v[3]), rv[1]));
          st4_nt(o0 + slot_m0<LAYOUT>(so, 2) * CH, mul4(rot5(w + 19, v), rv[2]));
        } else {
          // X_m1 slots q = 0..3: rotated coefficients 3, 7, 1, 5 (radial blocks 3, 4, 3, 4);
          // X_m2 slots q = 0, 1: coefficients 8, 4 (radial block 5)
          float* o1 = X1 + e * 8 * CH + ch;
          float* o2 = X2 + e * 4 * CH + ch;
          st4_nt(o1 + slot_m1<LAYOUT>(so, 0) * CH, mul4(rot3(w[6], w[7], w[8], v[1], v[2], v[3]), rv[0]));
          st4_nt(o1 + slot_m1<LAYOUT>(so, 2) * CH, mul4(rot3(w[0], w[1], w[2], v[1], v[2], v[3]), rv[0]));
          st4_nt(o1 + slot_m1<LAYOUT>(so, 1) * CH, mul4(rot5(w + 24, v), rv[1]));
          st4_nt(o1 + slot_m1<LAYOUT>(so, 3) * CH, mul4(rot5(w + 14, v), rv[1]));
          st4_nt(o2 + slot_m2<LAYOUT>(so, 0) * CH, mul4(rot5(w + 29, v), rv[2]));
          st4_nt(o2 + slot_m2<LAYOUT>(so, 1) * CH, mul4(rot5(w + 9, v), rv[2]));
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

}  // namespace rg

// Host side of the column order: perm[p] = natural radial column of permuted column p.
template <int LAYOUT>
static void radial_gather_perm_fill(int32_t* perm) {
  for (int t = 0; t < rg::NT; ++t)
    for (int j = 0; j < 3; ++j)
      for (int c = 0; c < 32; ++c)
        perm[t * rg::TN + 32 * j + c] = slot_rad<LAYOUT>(t >> 3, 3 * (t & 1) + j) * rg::CH + 32 * ((t >> 1) & 3) + c;
}

extern "C" int fu_radial_gather_perm(int32_t C, int32_t layout, int32_t* perm) {
  const char* who = "fu_radial_gather_perm";
  if (C != rg::CH) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d (the fused kernel takes C = 128)", who, C);
  if (layout != 0 && layout != 1) return set_error(FU_ERR_UNSUPPORTED, "%s: layout=%d (0 or 1)", who, layout);
  if (!perm) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (layout) radial_gather_perm_fill<1>(perm);
  else radial_gather_perm_fill<0>(perm);
  return FU_OK;
}

extern "C" int fu_radial_gather_fwd(const float* h2, int64_t ldh, const void* W2, const float* bias, const float* x,
                                    const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                                    const float* csd_emb, const int64_t* batch, float* rad, float* X_m0,
                                    float* X_m1, float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C, int32_t K,
                                    int32_t layout, void* stream) {
  const char* who = "fu_radial_gather_fwd";
  if (E < 0 || N < 0 || S < 1 || ldh < K || N > 0x7fffffffLL || S > 0x7fffffffLL)
    return set_error(FU_ERR_SHAPE, "%s: bad shape", who);
  if (C != rg::CH || K != 16 * rg::KC)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d K=%d (the fused kernel takes C = K = 128)", who, C, K);
  if (layout != 0 && layout != 1) return set_error(FU_ERR_UNSUPPORTED, "%s: layout=%d (0 or 1)", who, layout);
  if (E == 0) return FU_OK;
  if (!h2 || !W2 || !x || !idx_i || !idx_j || !wigner || !csd_emb || !batch || !rad || !X_m0 || !X_m1 || !X_m2)
    return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(h2) || ldh % 4 != 0 || !aligned16(W2) || (bias && !aligned16(bias)) || !aligned16(x) ||
      !aligned16(csd_emb) || !aligned16(rad) || !aligned16(X_m0) || !aligned16(X_m1) || !aligned16(X_m2))
    return set_error(FU_ERR_ALIGN, "%s: h2, W2, bias, x, csd_emb, rad and X must be 16-byte aligned (ldh % 4 == 0)",
                     who);
  const int Nc = 12 * C;
  const uint4* w2 = static_cast<const uint4*>(W2);
  const float* cinv = reinterpret_cast<const float*>(w2 + resident_frag_vectors(Nc, K));
  const int* summary = reinterpret_cast<const int*>(cinv + resident_cols(Nc)) + resident_cols(Nc);
  const dim3 grid((unsigned)cdiv(E, rg::RBM)), block(256);
  hipStream_t s = as_stream(stream);
  if (layout)
    hipLaunchKernelGGL(rg::radial_gather_kernel<1>, grid, block, 0, s, h2, ldh, w2, cinv, summary, bias, x, idx_i,
                       idx_j, wigner, csd_emb, batch, rad, X_m0, X_m1, X_m2, E);
  else
    hipLaunchKernelGGL(rg::radial_gather_kernel<0>, grid, block, 0, s, h2, ldh, w2, cinv, summary, bias, x, idx_i,
                       idx_j, wigner, csd_emb, batch, rad, X_m0, X_m1, X_m2, E);
  return check_launch(who);
}

}  // namespace fu
