// Radial output layer fused with the gather-rotate forward (C = 128; lmax 2 below, lmax 3 and 4
// further down, radial_gather_lmax_kernel).
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
// so = t / 8, channel group cg = (t / 2) % 4, and the blocks of degrees 0 and 1 ((l, |m|) =
// (0, 0), (1, 0), (1, 1)) for even t or of degree 2 ((2, 0), (2, 1), (2, 2)) for odd t; column
// 96 t + 32 j + ch is radial column slot_rad(so, q) C + 32 cg + ch of the natural order, q =
// tile_block(t % 2, j).  Grouping by degree lets a tile read each node coefficient it rotates
// once (rows 0..3 or 4..8; grouped by |m| instead, rows 1..8 were read by both tiles of a pair:
// 877 against 831 us at bcc Fe).  Each of the 4 waves computes 32 rows of every tile (three
// 32 x 32 blocks: 48 accumulators, so that the epilogue's node rows and Wigner scalars fit
// beside them at two workgroups per CU).  In the epilogue a lane takes one edge (slice row)
// and 4 channels: it reads the edge's node row pieces (4 or 5 coefficients x 16 bytes) and
// Wigner scalars, rotates them exactly as the gather kernel does (same products in the same
// order, so X is bitwise the gather's) and writes rad and the tile's X slots as 16-byte pieces
// (8 lanes of one edge cover 128 contiguous bytes).
//
// The K loop and the panel are those of fu_linear_resident (split-fp16, weight fragments
// straight from global memory, pass 2 of split_f16.h for a panel the window rule sends there).
#include "edge_layout.h"
#include "edge_lmax_layout.h"
#include "resident_panel.h"

namespace fu {
namespace rg {

constexpr int RBM = kResRows;     // rows (edges) per workgroup
constexpr int KC = 8;             // 16-wide K chunks: K = 128
constexpr int RPLANE = kResPlane;  // fp16 per plane (one chunk of the panel)
constexpr int CH = 128;           // channels
constexpr int NT = 16;            // output tiles (lmax 2): 2 sides x 4 channel groups x 2 degree groups
constexpr int TN = 96;            // columns per tile: 3 radial blocks x 32 channels
constexpr int RES3 = 96 + 8;      // floats per row of a wave's epilogue slice: 4 RES3 = 32 mod 64 banks

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

// radial block (slot q of a side) of column block j of a tile of degree group hq: degrees 0, 1
// (blocks (0, 0), (1, 0), (1, 1)) or degree 2 ((2, 0), (2, 1), (2, 2))
__host__ __device__ constexpr int tile_block(int hq, int j) { return hq == 0 ? (j < 2 ? j : 3) : (j == 0 ? 2 : j + 3); }

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
    // tile t: side so, channel group cg, the radial blocks of degrees 0, 1 (hq 0) or 2 (hq 1)
    const int so = t >> 3, cg = (t >> 1) & 3, hq = t & 1;
    int cb[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) cb[j] = 3 * t + j;
    floatx16 acc[1][3];
    resident_tile<KC, 1, 3, 2>(sp, wf, cb, acc, need2, wr, fr, fh);
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
        for (int j = 0; j < 3; ++j) st4_nt(re + slot_rad<LAYOUT>(so, tile_block(hq, j)) * CH, rv[j]);
        const int64_t node = so ? nid[1][g8] : nid[0][g8];
        const float* xn = x + node * 9 * CH + ch;
        const float* w = wig + e * 34;
        float4 v[9];
        if (hq == 0) {
          // degrees 0 and 1: X_m0 slots 0, 1 (rotated coefficients 0, 2), X_m1 slots 0, 2
          // (coefficients 3, 1)
#pragma unroll
          for (int k = 1; k < 4; ++k) v[k] = ld4(xn + k * CH);
          const float4 x0 = ld4(xn), c0 = ld4(csd + (int64_t)(so ? bid[1][g8] : bid[0][g8]) * CH + ch);
          v[0] = make_float4(x0.x + c0.x, x0.y + c0.y, x0.z + c0.z, x0.w + c0.w);
          float* o0 = X0 + e * 6 * CH + ch;
          float* o1 = X1 + e * 8 * CH + ch;
          st4_nt(o0 + slot_m0<LAYOUT>(so, 0) * CH, mul4(v[0], rv[0]));
          st4_nt(o0 + slot_m0<LAYOUT>(so, 1) * CH, mul4(rot3(w[3], w[4], w[5], v[1], v[2], v[3]), rv[1]));
          st4_nt(o1 + slot_m1<LAYOUT>(so, 0) * CH, mul4(rot3(w[6], w[7], w[8], v[1], v[2], v[3]), rv[2]));
          st4_nt(o1 + slot_m1<LAYOUT>(so, 2) * CH, mul4(rot3(w[0], w[1], w[2], v[1], v[2], v[3]), rv[2]));
        } else {
          // degree 2: X_m0 slot 2 (coefficient 6), X_m1 slots 1, 3 (coefficients 7, 5), X_m2
          // slots 0, 1 (coefficients 8, 4)
#pragma unroll
          for (int k = 4; k < 9; ++k) v[k] = ld4(xn + k * CH);
          float* o0 = X0 + e * 6 * CH + ch;
          float* o1 = X1 + e * 8 * CH + ch;
          float* o2 = X2 + e * 4 * CH + ch;
          st4_nt(o0 + slot_m0<LAYOUT>(so, 2) * CH, mul4(rot5(w + 19, v), rv[0]));
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

// ---------------------------------------------------------------------------------------
// lmax 3 and 4 (the reference block order extended by degree, edge_lmax_layout.h).  Tiles per
// side and channel group: degree group g = 0 (degrees 0 and 1: radial (0, 0), (1, 0), (1, 1)),
// then g = 1 .. L - 1 (degree g + 1: (l, 0), (l, 1), (l, 2)); tile t = ((so 4 + cg) L + g).
// The epilogue rotates each degree's node coefficients with the lmax gather's arithmetic
// (gather_fwd_block of edge_lmax.hip: rv = 0, rv += D[m][mp] v[mp] for mp = -l .. l).
// ---------------------------------------------------------------------------------------

// (l, |m|) of column block j of degree group g
__host__ __device__ constexpr int grp_l(int g, int j) { return g == 0 ? (j == 0 ? 0 : 1) : g + 1; }
__host__ __device__ constexpr int grp_am(int g, int j) { return g == 0 ? (j == 2 ? 1 : 0) : j; }

// X slots (l, m), |m| <= min(l, 2), of one edge side for degree l >= 1 from its node row
// pieces v (row l^2 + l + mp at v[l + mp]) and the radial values rv[|m|]
template <int L, int l>
__device__ __forceinline__ void lm_slots(const float4 (&v)[2 * l + 1], const float4* rv, const float* wl,
                                         const float* we, float* X0e, float* X1e, float* X2e, int so) {
  constexpr int mm = lm::mmx(l);
#pragma unroll
  for (int am = 0; am <= mm; ++am) {
#pragma unroll
    for (int s2 = 0; s2 < (am == 0 ? 1 : 2); ++s2) {
      const int m = s2 == 0 ? am : -am;
      float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int mp = -l; mp <= l; ++mp) {
        const float w = l <= 2 ? wl[lm::widx(l, m, mp)] : we[lm::widx(l, m, mp)];
        r.x += w * v[l + mp].x;
        r.y += w * v[l + mp].y;
        r.z += w * v[l + mp].z;
        r.w += w * v[l + mp].w;
      }
      float* base = am == 0 ? X0e : am == 1 ? X1e : X2e;
      st4_nt(base + lm::xblk(L, l, m, so) * CH, mul4(r, rv[am]));
    }
  }
}

template <int L, int l>
__device__ __forceinline__ void lm_degree(const float* xn, const float4* rv, const float* wl, const float* we,
                                          float* X0e, float* X1e, float* X2e, int so) {
  float4 v[2 * l + 1];
#pragma unroll
  for (int k = 0; k < 2 * l + 1; ++k) v[k] = ld4(xn + (l * l + k) * CH);
  lm_slots<L, l>(v, rv, wl, we, X0e, X1e, X2e, so);
}

template <int L>
__global__ __launch_bounds__(256, 2) void radial_gather_lmax_kernel(
    const float* __restrict__ A, int64_t lda, const uint4* __restrict__ W2, const float* __restrict__ cinv,
    const int* __restrict__ wsum, const float* __restrict__ bias, const float* __restrict__ x,
    const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j, const float* __restrict__ wig,
    const float* __restrict__ ext, const float* __restrict__ csd, const int64_t* __restrict__ batch,
    float* __restrict__ rad, float* __restrict__ X0, float* __restrict__ X1, float* __restrict__ X2, int64_t M) {
  constexpr int NK = lm::ncoef(L), EW = lm::extw(L), NTL = 8 * L;
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
  int32_t nid[2][4], bid[2][4];  // as in radial_gather_kernel
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
  for (int t = 0; t < NTL; ++t) {
    const int g = t % L, cg = (t / L) & 3, so = t / (4 * L);
    int cb[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) cb[j] = 3 * t + j;
    floatx16 acc[1][3];
    resident_tile<KC, 1, 3, 2>(sp, wf, cb, acc, need2, wr, fr, fh);
    const int ch = 32 * cg + 4 * c4;
    const int col0 = t * TN + 4 * c4;
#pragma unroll
    for (int g8 = 0; g8 < 4; ++g8) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) ep[(4 * fh + s) * RES3 + 32 * j + fr] = acc[0][j][4 * g8 + s];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int rb = wr + 8 * g8;
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
        float* re = rad + e * lm::wrad(L) * CH + ch;
#pragma unroll
        for (int j = 0; j < 3; ++j) st4_nt(re + lm::radblk(L, grp_l(g, j), grp_am(g, j), so) * CH, rv[j]);
        const float* xn = x + (int64_t)(so ? nid[1][g8] : nid[0][g8]) * NK * CH + ch;
        const float* wl = wig + e * 34;
        const float* we = ext + e * EW;
        float* X0e = X0 + e * lm::wx0(L) * CH + ch;
        float* X1e = X1 + e * lm::wx1(L) * CH + ch;
        float* X2e = X2 + e * lm::wx2(L) * CH + ch;
        if (g == 0) {
          // degree 0 (csd added) with radial block (0, 0), degree 1 with (1, 0), (1, 1)
          const float4 x0 = ld4(xn), c0 = ld4(csd + (int64_t)(so ? bid[1][g8] : bid[0][g8]) * CH + ch);
          const float4 v0 = make_float4(x0.x + c0.x, x0.y + c0.y, x0.z + c0.z, x0.w + c0.w);
          st4_nt(X0e + lm::xblk(L, 0, 0, so) * CH, mul4(v0, rv[0]));
          lm_degree<L, 1>(xn, rv + 1, wl, we, X0e, X1e, X2e, so);
        } else if (g == 1) {
          lm_degree<L, 2>(xn, rv, wl, we, X0e, X1e, X2e, so);
        } else if (g == 2) {
          lm_degree<L, 3>(xn, rv, wl, we, X0e, X1e, X2e, so);
        } else if constexpr (L >= 4) {
          lm_degree<L, 4>(xn, rv, wl, we, X0e, X1e, X2e, so);
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
        perm[t * rg::TN + 32 * j + c] = slot_rad<LAYOUT>(t >> 3, rg::tile_block(t & 1, j)) * rg::CH + 32 * ((t >> 1) & 3) + c;
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

// perm[p] = natural radial column of permuted column p, lmax 3 or 4
template <int L>
static void radial_gather_lmax_perm_fill(int32_t* perm) {
  for (int t = 0; t < 8 * L; ++t) {
    const int g = t % L, cg = (t / L) & 3, so = t / (4 * L);
    for (int j = 0; j < 3; ++j)
      for (int c = 0; c < 32; ++c)
        perm[t * rg::TN + 32 * j + c] =
            lm::radblk(L, rg::grp_l(g, j), rg::grp_am(g, j), so) * rg::CH + 32 * cg + c;
  }
}

extern "C" int fu_radial_gather_perm_lmax(int32_t C, int32_t lmax, int32_t* perm) {
  const char* who = "fu_radial_gather_perm_lmax";
  if (C != rg::CH) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d (the fused kernel takes C = 128)", who, C);
  if (lmax != 3 && lmax != 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d (3 or 4)", who, lmax);
  if (!perm) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (lmax == 3) radial_gather_lmax_perm_fill<3>(perm);
  else radial_gather_lmax_perm_fill<4>(perm);
  return FU_OK;
}

extern "C" int fu_radial_gather_fwd_lmax(const float* h2, int64_t ldh, const void* W2, const float* bias,
                                         const float* x, const int64_t* idx_i, const int64_t* idx_j,
                                         const float* wigner, const float* wig_ext, const float* csd_emb,
                                         const int64_t* batch, float* rad, float* X_m0, float* X_m1, float* X_m2,
                                         int64_t E, int64_t N, int64_t S, int32_t C, int32_t K, int32_t lmax,
                                         void* stream) {
  const char* who = "fu_radial_gather_fwd_lmax";
  if (E < 0 || N < 0 || S < 1 || ldh < K || N > 0x7fffffffLL || S > 0x7fffffffLL)
    return set_error(FU_ERR_SHAPE, "%s: bad shape", who);
  if (C != rg::CH || K != 16 * rg::KC)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d K=%d (the fused kernel takes C = K = 128)", who, C, K);
  if (lmax != 3 && lmax != 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d (3 or 4)", who, lmax);
  if (E == 0) return FU_OK;
  if (!h2 || !W2 || !x || !idx_i || !idx_j || !wigner || !wig_ext || !csd_emb || !batch || !rad || !X_m0 ||
      !X_m1 || !X_m2)
    return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(h2) || ldh % 4 != 0 || !aligned16(W2) || (bias && !aligned16(bias)) || !aligned16(x) ||
      !aligned16(csd_emb) || !aligned16(rad) || !aligned16(X_m0) || !aligned16(X_m1) || !aligned16(X_m2))
    return set_error(FU_ERR_ALIGN, "%s: h2, W2, bias, x, csd_emb, rad and X must be 16-byte aligned (ldh % 4 == 0)",
                     who);
  const int Nc = 6 * lmax * C;
  const uint4* w2 = static_cast<const uint4*>(W2);
  const float* cinv = reinterpret_cast<const float*>(w2 + resident_frag_vectors(Nc, K));
  const int* summary = reinterpret_cast<const int*>(cinv + resident_cols(Nc)) + resident_cols(Nc);
  const dim3 grid((unsigned)cdiv(E, rg::RBM)), block(256);
  hipStream_t s = as_stream(stream);
  if (lmax == 3)
    hipLaunchKernelGGL(rg::radial_gather_lmax_kernel<3>, grid, block, 0, s, h2, ldh, w2, cinv, summary, bias, x,
                       idx_i, idx_j, wigner, wig_ext, csd_emb, batch, rad, X_m0, X_m1, X_m2, E);
  else
    hipLaunchKernelGGL(rg::radial_gather_lmax_kernel<4>, grid, block, 0, s, h2, ldh, w2, cinv, summary, bias, x,
                       idx_i, idx_j, wigner, wig_ext, csd_emb, batch, rad, X_m0, X_m1, X_m2, E);
  return check_launch(who);
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
