// Edge kernels for lmax in {2, 3, 4} with mmax = 2: gather-rotate, rotate-scatter, the
// edge-degree embedding and the gate, forward and backward.  They restate the reference's
// lmax = 2 kernels (ops/gather.py:34-405, ops/scatter.py:45-481, ops/gating.py:32-185) for
// any degree, in the reference's column-block order extended degree by degree:
//
//   SH coefficient (l, m) of a node row sits at row l^2 + l + m; the edge frame keeps the
//   orders |m| <= min(l, 2).  Per edge, with side so = 0 (sender) / 1 (receiver):
//     X_m0 (2(L+1) blocks): (l, 0) at block 2l + so
//     X_m1 (4L blocks):     (l, +1) at 2(l-1) + so, (l, -1) at 2(L + l - 1) + so
//     X_m2 (4(L-1) blocks): (l, +2) at 2(l-2) + so, (l, -2) at 2(L - 1 + l - 2) + so
//     rad (6L blocks):      |m| = 0: 2l + so; 1: 2(L+1) + 2(l-1) + so; 2: 4L + 2 + 2(l-2) + so
//     Y_m0 = [gate_1 .. gate_L, y_0 .. y_L (m = 0)], Y_m1 = [R_1 .. R_L, I_1 .. I_L],
//     Y_m2 = [R_2 .. R_L, I_2 .. I_L]; Z and Zout as Y without the gates.
//   For L = 2 every block lands where the reference puts it (ops/gather.py:132-154,
//   ops/gating.py:63-103, ops/scatter.py:104-127).
//
// Wigner rows: the reference's 34 scalars give D^1 and D^2; the ext array (fu_wigner_ext_fwd)
// gives rows m = -2..2 of D^3 (5 x 7) and D^4 (5 x 9).
//
// Mapping (HBM-bound, like the lmax = 2 kernels): forward gather and backward scatter one
// wave64 per edge, lanes across channels, a contiguous XCD-aware edge range per workgroup; forward scatters one wave per receiver with fp64
// accumulators, segments in CSR order; backward gather node-centric (one wave per CSR
// segment of the node, as receiver and as sender), so no kernel uses atomics.  The l blocks
// are processed one at a time to bound registers.
#include "edge_lmax_layout.h"
#include "fu_vec.h"

namespace fu {
namespace lm {

template <int l>
__device__ __forceinline__ float dwig(const float* wl, const float* we, int m, int mp) {
  if constexpr (l <= 2) return wl[widx(l, m, mp)];
  else return we[widx(l, m, mp)];
}

__device__ __forceinline__ int wave_uniform() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

template <int L, int CPL>
__device__ __forceinline__ float* xslot(float* X0e, float* X1e, float* X2e, int l, int m, int so) {
  constexpr int C = 64 * CPL;
  const int am = m < 0 ? -m : m;
  float* base = am == 0 ? X0e : am == 1 ? X1e : X2e;
  return base + xblk(L, l, m, so) * C;
}

template <int L, int CPL>
__device__ __forceinline__ const float* zslot(const float* Z0e, const float* Z1e, const float* Z2e, int l, int m) {
  constexpr int C = 64 * CPL;
  const int am = m < 0 ? -m : m;
  const float* base = am == 0 ? Z0e : am == 1 ? Z1e : Z2e;
  return base + zblk(L, l, m) * C;
}

// ---------------------------------------------------------------------------------------
// Gather forward
// ---------------------------------------------------------------------------------------

// NT: the radial rows and the X stores (each touched once) carry the nontemporal hint
template <int L, int CPL, int l, bool NT = false>
__device__ __forceinline__ void gather_fwd_block(const float* xr, const float* wl, const float* we, const float* rade,
                                                 float* X0e, float* X1e, float* X2e, int so) {
  constexpr int C = 64 * CPL;
  Vec<CPL> v[2 * l + 1];
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) v[l + mp] = vload<CPL>(xr + (l * l + l + mp) * C);
#pragma unroll
  for (int am = 0; am <= mmx(l); ++am) {
    const Vec<CPL> r = NT ? vload_nt<CPL>(rade + radblk(L, l, am, so) * C) : vload<CPL>(rade + radblk(L, l, am, so) * C);
#pragma unroll
    for (int s = 0; s < (am == 0 ? 1 : 2); ++s) {
      const int m = s == 0 ? am : -am;
      Vec<CPL> rv = vzero<CPL>();
#pragma unroll
      for (int mp = -l; mp <= l; ++mp)
#pragma unroll
        for (int q = 0; q < CPL; ++q) rv[q] += dwig<l>(wl, we, m, mp) * v[l + mp][q];
      if constexpr (NT) vstore_nt(xslot<L, CPL>(X0e, X1e, X2e, l, m, so), vmul(rv, r));
      else vstore(xslot<L, CPL>(X0e, X1e, X2e, l, m, so), vmul(rv, r));
    }
  }
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void gather_fwd_lmax_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j,
    const float* __restrict__ wig, const float* __restrict__ ext, const float* __restrict__ rad,
    const float* __restrict__ csd, const int64_t* __restrict__ batch, float* __restrict__ X0,
    float* __restrict__ X1, float* __restrict__ X2, int64_t E) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_uniform(); e < e1; e += (blockDim.x >> 6)) {
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* rade = rad + e * wrad(L) * C + c;
    float* X0e = X0 + e * wx0(L) * C + c;
    float* X1e = X1 + e * wx1(L) * C + c;
    float* X2e = X2 + e * wx2(L) * C + c;
#pragma unroll
    for (int so = 0; so < 2; ++so) {
      const int64_t node = so ? idx_j[e] : idx_i[e];
      const float* xr = x + node * K * C + c;
      const Vec<CPL> v0 = vadd(vload<CPL>(xr), vload<CPL>(csd + batch[node] * C + c));
      vstore(X0e + xblk(L, 0, 0, so) * C, vmul(v0, vload<CPL>(rade + radblk(L, 0, 0, so) * C)));
      gather_fwd_block<L, CPL, 1>(xr, wl, we, rade, X0e, X1e, X2e, so);
      gather_fwd_block<L, CPL, 2>(xr, wl, we, rade, X0e, X1e, X2e, so);
      if constexpr (L >= 3) gather_fwd_block<L, CPL, 3>(xr, wl, we, rade, X0e, X1e, X2e, so);
      if constexpr (L >= 4) gather_fwd_block<L, CPL, 4>(xr, wl, we, rade, X0e, X1e, X2e, so);
    }
  }
}

// Node-centric form (used when the caller passes both CSRs): one node per 128-thread
// workgroup, wave 0 walks the node's receiver segment (the receiver-side blocks of those
// edges), wave 1 its sender segment (the sender-side blocks), so every node row is read once
// per side instead of once per edge.  At lmax 4 a row is 12.8 KB and the edge-parallel form
// fetched 1.85x its algorithmic reads at bcc Fe (rows evicted between the edges that reuse
// them).  The row (csd added on l = 0) is kept in LDS; both waves load half of it.
template <int CPL, int L>
__global__ __launch_bounds__(128) void gather_fwd_node_lmax_kernel(
    const float* __restrict__ x, const float* __restrict__ wig, const float* __restrict__ ext,
    const float* __restrict__ rad, const float* __restrict__ csd, const int64_t* __restrict__ batch,
    const int32_t* __restrict__ rptr, const int32_t* __restrict__ ridx, const int32_t* __restrict__ sptr,
    const int32_t* __restrict__ sidx, float* __restrict__ X0, float* __restrict__ X1, float* __restrict__ X2) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  __shared__ __attribute__((aligned(16))) float s_v[K * C];
  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform();
  const int64_t n = (int64_t)blockIdx.x;
  const int c = lane * CPL;
  const float* xn = x + n * K * C + c;
  for (int k = wave; k < K; k += 2) {
    Vec<CPL> r = vload<CPL>(xn + k * C);
    if (k == 0) r = vadd(r, vload<CPL>(csd + batch[n] * C + c));
    vstore(s_v + k * C + c, r);
  }
  __syncthreads();
  const int so = wave == 0 ? 1 : 0;
  const int32_t* ptr = so ? rptr : sptr;
  const int32_t* idx = so ? ridx : sidx;
  const int32_t k0 = ptr[n], k1 = ptr[n + 1];
  const float* sv = s_v + c;
  for (int32_t k = k0; k < k1; ++k) {
    const int64_t e = idx[k];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* rade = rad + e * wrad(L) * C + c;
    float* X0e = X0 + e * wx0(L) * C + c;
    float* X1e = X1 + e * wx1(L) * C + c;
    float* X2e = X2 + e * wx2(L) * C + c;
    vstore_nt(X0e + xblk(L, 0, 0, so) * C, vmul(vload<CPL>(sv), vload_nt<CPL>(rade + radblk(L, 0, 0, so) * C)));
    gather_fwd_block<L, CPL, 1, true>(sv, wl, we, rade, X0e, X1e, X2e, so);
    gather_fwd_block<L, CPL, 2, true>(sv, wl, we, rade, X0e, X1e, X2e, so);
    if constexpr (L >= 3) gather_fwd_block<L, CPL, 3, true>(sv, wl, we, rade, X0e, X1e, X2e, so);
    if constexpr (L >= 4) gather_fwd_block<L, CPL, 4, true>(sv, wl, we, rade, X0e, X1e, X2e, so);
  }
}

// ---------------------------------------------------------------------------------------
// Gather backward (node-centric)
// ---------------------------------------------------------------------------------------

// reduce n <= 64 per-lane partial sums over the wave and store lane k's total to out[k]
// (added to out[k] when accumulating)
template <int n>
__device__ __forceinline__ void reduce_store(float (&part)[n], float* out, int lane, bool accumulate) {
  constexpr int V = n <= 16 ? 16 : n <= 32 ? 32 : 64;
  float p[V];
#pragma unroll
  for (int k = 0; k < V; ++k) p[k] = k < n ? part[k] : 0.0f;
  const float tot = wave_multi_sum<V>(p, lane);
  if (lane < n) out[lane] = accumulate ? out[lane] + tot : tot;
}

template <int L, int CPL, int l>
__device__ __forceinline__ void gather_bwd_block(const float* sv, const float* wl, const float* we,
                                                 const float* gX0e, const float* gX1e, const float* gX2e,
                                                 const float* rade, float* grade, Vec<CPL> (&acc)[ncoef(L)],
                                                 float* gw_l, int so, int c, int lane, bool accw) {
  constexpr int C = 64 * CPL;
  constexpr int nk = 2 * l + 1, mm = mmx(l), nr = 2 * mm + 1;
  Vec<CPL> v[nk];
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) v[l + mp] = vload<CPL>(sv + (l * l + l + mp) * C + c);
  Vec<CPL> grv[nr];
#pragma unroll
  for (int am = 0; am <= mm; ++am) {
    // the edge streams (rad, g_X, g_rad) are touched once: nontemporal
    const Vec<CPL> r = vload_nt<CPL>(rade + radblk(L, l, am, so) * C);
    Vec<CPL> gr = vzero<CPL>();
#pragma unroll
    for (int s = 0; s < (am == 0 ? 1 : 2); ++s) {
      const int m = s == 0 ? am : -am;
      const Vec<CPL> g = vload_nt<CPL>(xslot<L, CPL>(const_cast<float*>(gX0e), const_cast<float*>(gX1e),
                                                     const_cast<float*>(gX2e), l, m, so));
      Vec<CPL> rv = vzero<CPL>();
#pragma unroll
      for (int mp = -l; mp <= l; ++mp)
#pragma unroll
        for (int q = 0; q < CPL; ++q) rv[q] += dwig<l>(wl, we, m, mp) * v[l + mp][q];
#pragma unroll
      for (int q = 0; q < CPL; ++q) gr[q] += g[q] * rv[q];
      grv[mm + m] = vmul(g, r);
    }
    vstore_nt(grade + radblk(L, l, am, so) * C, gr);
  }
  // node gradient: acc[l, mp] += sum_m D[m][mp] grv[m]
#pragma unroll
  for (int mp = -l; mp <= l; ++mp)
#pragma unroll
    for (int m = -mm; m <= mm; ++m)
#pragma unroll
      for (int q = 0; q < CPL; ++q) acc[l * l + l + mp][q] += dwig<l>(wl, we, m, mp) * grv[mm + m][q];
  // g_wigner rows kept for this degree: dL/dD[m][mp] = sum_c grv[m] v[mp]
  float part[nr * nk];
#pragma unroll
  for (int m = 0; m < nr; ++m)
#pragma unroll
    for (int mp = 0; mp < nk; ++mp) part[m * nk + mp] = vdot(grv[m], v[mp]);
  static_assert(nr * nk <= 64, "one multi-value reduction per degree");
  reduce_store<nr * nk>(part, gw_l, lane, accw);
}

template <int CPL, int L>
__device__ __forceinline__ void gather_bwd_segment(const float* __restrict__ gX0, const float* __restrict__ gX1,
                                                   const float* __restrict__ gX2, const float* __restrict__ wig,
                                                   const float* __restrict__ ext, const float* __restrict__ rad,
                                                   const int32_t* __restrict__ ptr, const int32_t* __restrict__ idx,
                                                   int64_t n, int so, const float* sv, Vec<CPL> (&acc)[ncoef(L)],
                                                   float* __restrict__ g_rad, float* __restrict__ gw,
                                                   float* __restrict__ gext, int c, int lane, bool accw) {
  constexpr int C = 64 * CPL, EW = extw(L);
  const int32_t k0 = ptr[n], k1 = ptr[n + 1];
  for (int32_t k = k0; k < k1; ++k) {
    const int64_t e = idx[k];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* gX0e = gX0 + e * wx0(L) * C + c;
    const float* gX1e = gX1 + e * wx1(L) * C + c;
    const float* gX2e = gX2 + e * wx2(L) * C + c;
    const float* rade = rad + e * wrad(L) * C + c;
    float* grade = g_rad + e * wrad(L) * C + c;
    {
      const Vec<CPL> g = vload_nt<CPL>(gX0e + xblk(L, 0, 0, so) * C);
      const Vec<CPL> r = vload_nt<CPL>(rade + radblk(L, 0, 0, so) * C);
      vstore_nt(grade + radblk(L, 0, 0, so) * C, vmul(g, vload<CPL>(sv + c)));
#pragma unroll
      for (int q = 0; q < CPL; ++q) acc[0][q] += g[q] * r[q];
    }
    gather_bwd_block<L, CPL, 1>(sv, wl, we, gX0e, gX1e, gX2e, rade, grade, acc, gw + e * 34, so, c, lane, accw);
    gather_bwd_block<L, CPL, 2>(sv, wl, we, gX0e, gX1e, gX2e, rade, grade, acc, gw + e * 34 + 9, so, c, lane, accw);
    if constexpr (L >= 3)
      gather_bwd_block<L, CPL, 3>(sv, wl, we, gX0e, gX1e, gX2e, rade, grade, acc, gext + e * EW, so, c, lane, accw);
    if constexpr (L >= 4)
      gather_bwd_block<L, CPL, 4>(sv, wl, we, gX0e, gX1e, gX2e, rade, grade, acc, gext + e * EW + 35, so, c, lane,
                                  accw);
  }
}

// One node per 128-thread workgroup: wave 0 walks the receiver segment, wave 1 the sender
// segment; each wave keeps its own LDS copy of the node row (csd added on l = 0), the two
// node-gradient partials meet in LDS and g_x[n] is written once.
template <int CPL, int L>
__global__ __launch_bounds__(128) void gather_bwd_lmax_kernel(
    const float* __restrict__ gX0, const float* __restrict__ gX1, const float* __restrict__ gX2,
    const float* __restrict__ x, const float* __restrict__ wig, const float* __restrict__ ext,
    const float* __restrict__ rad, const float* __restrict__ csd, const int64_t* __restrict__ batch,
    const int32_t* __restrict__ rptr, const int32_t* __restrict__ ridx, const int32_t* __restrict__ sptr,
    const int32_t* __restrict__ sidx, float* __restrict__ g_x, float* __restrict__ gw_recv,
    float* __restrict__ gext_recv, float* __restrict__ gw_send, float* __restrict__ gext_send,
    float* __restrict__ g_rad, int64_t N, int32_t acc_flags) {
  constexpr int C = 64 * CPL, K = ncoef(L);
  __shared__ __attribute__((aligned(16))) float s_v[2][K * C];
  __shared__ __attribute__((aligned(16))) float s_send[K * C];
  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform();
  const int64_t n = (int64_t)blockIdx.x;
  const int c = lane * CPL;
  Vec<CPL> acc[K];
#pragma unroll
  for (int k = 0; k < K; ++k) acc[k] = vzero<CPL>();
  float* sv = s_v[wave];
  const float* xn = x + n * K * C + c;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Vec<CPL> r = vload<CPL>(xn + k * C);
    if (k == 0) r = vadd(r, vload<CPL>(csd + batch[n] * C + c));
    vstore(sv + k * C + c, r);
  }
  if (wave == 0) {
    // the receiver half goes into the caller's g_wigner / g_wig_ext (added to their contents
    // when accumulating: only this wave writes an edge's entries there), the sender half into
    // the workspace, added afterwards
    gather_bwd_segment<CPL, L>(gX0, gX1, gX2, wig, ext, rad, rptr, ridx, n, 1, sv, acc, g_rad, gw_recv, gext_recv, c,
                               lane, (acc_flags & 1) != 0);
  } else {
    gather_bwd_segment<CPL, L>(gX0, gX1, gX2, wig, ext, rad, sptr, sidx, n, 0, sv, acc, g_rad, gw_send, gext_send, c,
                               lane, false);
#pragma unroll
    for (int k = 0; k < K; ++k) vstore(&s_send[k * C + c], acc[k]);
  }
  __syncthreads();
  if (wave == 0) {
    float* gx = g_x + n * K * C + c;
#pragma unroll
    for (int k = 0; k < K; ++k) vstore(gx + k * C, vadd(acc[k], vload<CPL>(&s_send[k * C + c])));
  }
}

__global__ __launch_bounds__(256) void add_rows_kernel(float* __restrict__ a, const float* __restrict__ b, int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
    a[k] += b[k];
}

// ---------------------------------------------------------------------------------------
// Rotate-scatter forward / backward
// ---------------------------------------------------------------------------------------

template <int L, int CPL, int l>
__device__ __forceinline__ void scatter_fwd_block(const float* wl, const float* we, float en, const float* Z0e,
                                                  const float* Z1e, const float* Z2e, double (&acc)[ncoef(L)][CPL]) {
  constexpr int mm = mmx(l);
  Vec<CPL> z[2 * mm + 1];
#pragma unroll
  for (int m = -mm; m <= mm; ++m) z[mm + m] = vload<CPL>(zslot<L, CPL>(Z0e, Z1e, Z2e, l, m));
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) {
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      float s = 0.0f;
#pragma unroll
      for (int m = -mm; m <= mm; ++m) s += dwig<l>(wl, we, m, mp) * z[mm + m][q];
      acc[l * l + l + mp][q] += (double)(s * en);
    }
  }
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void scatter_fwd_lmax_kernel(
    const int32_t* __restrict__ rptr, const int32_t* __restrict__ col, const float* __restrict__ Z0,
    const float* __restrict__ Z1, const float* __restrict__ Z2, const float* __restrict__ wig,
    const float* __restrict__ ext, const float* __restrict__ env, const float* __restrict__ x_res,
    float* __restrict__ x_out, int64_t N) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_uniform();
  if (n >= N) return;
  double acc[K][CPL];
  const float* xr = x_res + n * K * C + c;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const Vec<CPL> t = vload<CPL>(xr + k * C);
#pragma unroll
    for (int q = 0; q < CPL; ++q) acc[k][q] = (double)t[q];
  }
  for (int32_t k = rptr[n]; k < rptr[n + 1]; ++k) {
    const int64_t e = col[k];
    const float en = env[e];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* Z0e = Z0 + e * (L + 1) * C + c;
    const float* Z1e = Z1 + e * 2 * L * C + c;
    const float* Z2e = Z2 + e * 2 * (L - 1) * C + c;
    const Vec<CPL> z0 = vload<CPL>(Z0e);
#pragma unroll
    for (int q = 0; q < CPL; ++q) acc[0][q] += (double)(z0[q] * en);
    scatter_fwd_block<L, CPL, 1>(wl, we, en, Z0e, Z1e, Z2e, acc);
    scatter_fwd_block<L, CPL, 2>(wl, we, en, Z0e, Z1e, Z2e, acc);
    if constexpr (L >= 3) scatter_fwd_block<L, CPL, 3>(wl, we, en, Z0e, Z1e, Z2e, acc);
    if constexpr (L >= 4) scatter_fwd_block<L, CPL, 4>(wl, we, en, Z0e, Z1e, Z2e, acc);
  }
  float* xo = x_out + n * K * C + c;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Vec<CPL> t;
#pragma unroll
    for (int q = 0; q < CPL; ++q) t[q] = (float)acc[k][q];
    vstore(xo + k * C, t);
  }
}

// one degree of the scatter backward: g_Z slots, this degree's g_wigner rows and its share
// of g_env (returned per lane, before the wave reduction)
template <int L, int CPL, int l>
__device__ __forceinline__ float scatter_bwd_block(const float* wl, const float* we, float en, const float* gn,
                                                   const float* Z0e, const float* Z1e, const float* Z2e, float* gZ0e,
                                                   float* gZ1e, float* gZ2e, float* gw_l, int lane, bool accw) {
  constexpr int C = 64 * CPL;
  constexpr int nk = 2 * l + 1, mm = mmx(l), nr = 2 * mm + 1;
  Vec<CPL> g[nk], z[nr];
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) g[l + mp] = vload<CPL>(gn + (l * l + l + mp) * C);
#pragma unroll
  for (int m = -mm; m <= mm; ++m) z[mm + m] = vload<CPL>(zslot<L, CPL>(Z0e, Z1e, Z2e, l, m));
  float ge = 0.0f;
#pragma unroll
  for (int m = -mm; m <= mm; ++m) {
    Vec<CPL> gz = vzero<CPL>();
#pragma unroll
    for (int mp = -l; mp <= l; ++mp)
#pragma unroll
      for (int q = 0; q < CPL; ++q) gz[q] += (g[l + mp][q] * en) * dwig<l>(wl, we, m, mp);
    vstore(const_cast<float*>(zslot<L, CPL>(gZ0e, gZ1e, gZ2e, l, m)), gz);
    // g_env: sum_c sum_mp g[mp] D[m][mp] z[m] = sum_c (D g)[m] z[m]
    Vec<CPL> dg = vzero<CPL>();
#pragma unroll
    for (int mp = -l; mp <= l; ++mp)
#pragma unroll
      for (int q = 0; q < CPL; ++q) dg[q] += dwig<l>(wl, we, m, mp) * g[l + mp][q];
    ge += vdot(dg, z[mm + m]);
  }
  float part[nr * nk];
#pragma unroll
  for (int m = 0; m < nr; ++m)
#pragma unroll
    for (int mp = 0; mp < nk; ++mp) part[m * nk + mp] = vdot(z[m], g[mp]) * en;
  reduce_store<nr * nk>(part, gw_l, lane, accw);
  return ge;
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void scatter_bwd_lmax_kernel(
    const float* __restrict__ g_out, const int64_t* __restrict__ idx_j, const float* __restrict__ Z0,
    const float* __restrict__ Z1, const float* __restrict__ Z2, const float* __restrict__ wig,
    const float* __restrict__ ext, const float* __restrict__ env, float* __restrict__ gZ0, float* __restrict__ gZ1,
    float* __restrict__ gZ2, float* __restrict__ g_wig, float* __restrict__ g_ext, float* __restrict__ g_env,
    int64_t E, int32_t acc) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  const bool accw = (acc & 1) != 0, acce = (acc & 2) != 0;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_uniform(); e < e1; e += (blockDim.x >> 6)) {
    const float en = env[e];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* gn = g_out + idx_j[e] * K * C + c;
    const float* Z0e = Z0 + e * (L + 1) * C + c;
    const float* Z1e = Z1 + e * 2 * L * C + c;
    const float* Z2e = Z2 + e * 2 * (L - 1) * C + c;
    float* gZ0e = gZ0 + e * (L + 1) * C + c;
    float* gZ1e = gZ1 + e * 2 * L * C + c;
    float* gZ2e = gZ2 + e * 2 * (L - 1) * C + c;
    const Vec<CPL> g0 = vload<CPL>(gn), z0 = vload<CPL>(Z0e);
    vstore(gZ0e, vscale(g0, en));
    float ge = vdot(g0, z0);
    ge += scatter_bwd_block<L, CPL, 1>(wl, we, en, gn, Z0e, Z1e, Z2e, gZ0e, gZ1e, gZ2e, g_wig + e * 34, lane, accw);
    ge += scatter_bwd_block<L, CPL, 2>(wl, we, en, gn, Z0e, Z1e, Z2e, gZ0e, gZ1e, gZ2e, g_wig + e * 34 + 9, lane,
                                       accw);
    if constexpr (L >= 3)
      ge += scatter_bwd_block<L, CPL, 3>(wl, we, en, gn, Z0e, Z1e, Z2e, gZ0e, gZ1e, gZ2e, g_ext + e * EW, lane, accw);
    if constexpr (L >= 4)
      ge += scatter_bwd_block<L, CPL, 4>(wl, we, en, gn, Z0e, Z1e, Z2e, gZ0e, gZ1e, gZ2e, g_ext + e * EW + 35, lane,
                                         accw);
    ge = wave_sum(ge);
    if (lane == 0) g_env[e] = acce ? g_env[e] + ge : ge;
  }
}

// ---------------------------------------------------------------------------------------
// Edge-degree embedding (init scatter) forward / backward
// ---------------------------------------------------------------------------------------

template <int L, int CPL, int l>
__device__ __forceinline__ void init_fwd_block(const float* wl, const float* we, float en, const float* rp,
                                               double (&acc)[ncoef(L)][CPL]) {
  constexpr int C = 64 * CPL;
  const Vec<CPL> r = vload<CPL>(rp + l * C);
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) {
    const float w = dwig<l>(wl, we, 0, mp);
#pragma unroll
    for (int q = 0; q < CPL; ++q) acc[l * l + l + mp][q] += (double)(r[q] * w * en);
  }
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void init_scatter_fwd_lmax_kernel(
    const int32_t* __restrict__ rptr, const int32_t* __restrict__ col, const float* __restrict__ rad,
    const float* __restrict__ wig, const float* __restrict__ ext, const float* __restrict__ env,
    const int64_t* __restrict__ Z, const int64_t* __restrict__ batch, const float* __restrict__ W_sphere,
    const float* __restrict__ csd, float* __restrict__ x_out, int64_t N) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_uniform();
  if (n >= N) return;
  double acc[K][CPL], base[CPL];
  {
    const Vec<CPL> ws = vload<CPL>(W_sphere + Z[n] * C + c);
    const Vec<CPL> cs = vload<CPL>(csd + batch[n] * C + c);
#pragma unroll
    for (int q = 0; q < CPL; ++q) base[q] = (double)(ws[q] + cs[q]);
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
      for (int q = 0; q < CPL; ++q) acc[k][q] = 0.0;
  }
  for (int32_t k = rptr[n]; k < rptr[n + 1]; ++k) {
    const int64_t e = col[k];
    const float en = env[e];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* rp = rad + e * (L + 1) * C + c;
    const Vec<CPL> r0 = vload<CPL>(rp);
#pragma unroll
    for (int q = 0; q < CPL; ++q) acc[0][q] += (double)(r0[q] * en);
    init_fwd_block<L, CPL, 1>(wl, we, en, rp, acc);
    init_fwd_block<L, CPL, 2>(wl, we, en, rp, acc);
    if constexpr (L >= 3) init_fwd_block<L, CPL, 3>(wl, we, en, rp, acc);
    if constexpr (L >= 4) init_fwd_block<L, CPL, 4>(wl, we, en, rp, acc);
  }
  // messages summed in fp64, divided by the rescale factor 5 once per node
  float* xo = x_out + n * K * C + c;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Vec<CPL> t;
#pragma unroll
    for (int q = 0; q < CPL; ++q) t[q] = (float)(k == 0 ? base[q] + acc[0][q] / 5.0 : acc[k][q] / 5.0);
    vstore(xo + k * C, t);
  }
}

// p = sum_mp g[mp] D[0][mp] (this degree's m = 0 projection); writes g_rad block l and the
// per-lane partials of the m = 0 row of g_wigner (2l + 1 values at part[off..])
template <int L, int CPL, int l>
__device__ __forceinline__ float init_bwd_block(const float* wl, const float* we, float en, const float* gn,
                                                const float* rp, float* grp, float* part) {
  constexpr int C = 64 * CPL;
  Vec<CPL> g[2 * l + 1];
#pragma unroll
  for (int mp = -l; mp <= l; ++mp) g[l + mp] = vscale(vload<CPL>(gn + (l * l + l + mp) * C), 1.0f / 5.0f);
  const Vec<CPL> r = vload<CPL>(rp + l * C);
  Vec<CPL> p = vzero<CPL>();
#pragma unroll
  for (int mp = -l; mp <= l; ++mp)
#pragma unroll
    for (int q = 0; q < CPL; ++q) p[q] += g[l + mp][q] * dwig<l>(wl, we, 0, mp);
  vstore(grp + l * C, vscale(p, en));
#pragma unroll
  for (int mp = 0; mp < 2 * l + 1; ++mp) part[mp] = vdot(g[mp], r);
  return vdot(p, r);
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void init_scatter_bwd_lmax_kernel(
    const float* __restrict__ g_out, const int64_t* __restrict__ idx_j, const float* __restrict__ rad,
    const float* __restrict__ wig, const float* __restrict__ ext, const float* __restrict__ env,
    float* __restrict__ g_rad, float* __restrict__ g_wig, float* __restrict__ g_ext, float* __restrict__ g_env,
    int64_t E, int32_t acc) {
  constexpr int C = 64 * CPL, K = ncoef(L), EW = extw(L);
  const bool accw = (acc & 1) != 0, acce = (acc & 2) != 0;
  // m = 0 row partials of degrees 1..L, then the g_env partial: 3 + 5 + 7 + 9 + 1 <= 32
  constexpr int NP = (L + 1) * (L + 1) - 1 + 1;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_uniform(); e < e1; e += (blockDim.x >> 6)) {
    const float en = env[e];
    const float* wl = wig + e * 34;
    const float* we = ext + e * EW;
    const float* gn = g_out + idx_j[e] * K * C + c;
    const float* rp = rad + e * (L + 1) * C + c;
    float* grp = g_rad + e * (L + 1) * C + c;
    float part[NP];
    const Vec<CPL> g0 = vscale(vload<CPL>(gn), 1.0f / 5.0f);
    vstore(grp, vscale(g0, en));
    float ge = vdot(g0, vload<CPL>(rp));
    ge += init_bwd_block<L, CPL, 1>(wl, we, en, gn, rp, grp, part + 0);
    ge += init_bwd_block<L, CPL, 2>(wl, we, en, gn, rp, grp, part + 3);
    if constexpr (L >= 3) ge += init_bwd_block<L, CPL, 3>(wl, we, en, gn, rp, grp, part + 8);
    if constexpr (L >= 4) ge += init_bwd_block<L, CPL, 4>(wl, we, en, gn, rp, grp, part + 15);
    part[NP - 1] = ge;
    float p32[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) p32[k] = k < NP ? part[k] : 0.0f;
    const float tot = wave_multi_sum<32>(p32, lane);
    // spread: lane t of the m = 0 row of degree l sits at value index (l^2 - 1) + t; the
    // wigner entry index is widx(l, 0, t - l).  Every lane takes part in the shuffles.
    float* gw = g_wig + e * 34;
    float* gx = g_ext + e * EW;
#pragma unroll
    for (int l = 1; l <= L; ++l) {
      const int nk = 2 * l + 1;
      const int src = (l * l - 1) + (lane < nk ? lane : 0);
      const float v = __shfl(tot, src, 64) * en;
      if (lane < nk) {
        const int w = widx(l, 0, lane - l);
        float* o = l <= 2 ? gw + w : gx + w;
        *o = accw ? *o + v : v;
      }
    }
    const float get = __shfl(tot, NP - 1, 64);
    if (lane == 0) g_env[e] = acce ? g_env[e] + get : get;
    // entries the forward does not read are zero (left as they are when accumulating)
    if (accw) continue;
    for (int k = lane; k < 34; k += 64) {
      const bool row0 = (k >= 3 && k < 6) || (k >= 19 && k < 24);
      if (!row0) gw[k] = 0.0f;
    }
    for (int k = lane; k < EW; k += 64) {
      const bool row0 = (k >= 14 && k < 21) || (k >= 53 && k < 62);
      if (!row0) gx[k] = 0.0f;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Gate forward / backward (reference-extended column order)
// ---------------------------------------------------------------------------------------

template <int L>
__global__ __launch_bounds__(256) void gating_fwd_lmax_kernel(const float* __restrict__ Y0,
                                                              const float* __restrict__ Y1,
                                                              const float* __restrict__ Y2, float* __restrict__ Z0,
                                                              float* __restrict__ Z1, float* __restrict__ Z2,
                                                              int64_t total, int32_t C4) {
  const int64_t C = 4 * (int64_t)C4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = t / C4;
    const int64_t c = 4 * (t - e * C4);
    const float* y0 = Y0 + e * (2 * L + 1) * C + c;
    const float* y1 = Y1 + e * 2 * L * C + c;
    const float* y2 = Y2 + e * 2 * (L - 1) * C + c;
    float* z0 = Z0 + e * (L + 1) * C + c;
    float* z1 = Z1 + e * 2 * L * C + c;
    float* z2 = Z2 + e * 2 * (L - 1) * C + c;
    const float4 l0 = ld4(y0 + L * C);
    st4(z0, l0 * make_float4(sigmoidf_(l0.x), sigmoidf_(l0.y), sigmoidf_(l0.z), sigmoidf_(l0.w)));
#pragma unroll
    for (int l = 1; l <= L; ++l) {
      const float4 a = ld4(y0 + (l - 1) * C);
      const float4 s = make_float4(sigmoidf_(a.x), sigmoidf_(a.y), sigmoidf_(a.z), sigmoidf_(a.w));
      st4(z0 + l * C, ld4(y0 + (L + l) * C) * s);
      st4(z1 + (l - 1) * C, ld4(y1 + (l - 1) * C) * s);
      st4(z1 + (L + l - 1) * C, ld4(y1 + (L + l - 1) * C) * s);
      if (l >= 2) {
        st4(z2 + (l - 2) * C, ld4(y2 + (l - 2) * C) * s);
        st4(z2 + (L - 1 + l - 2) * C, ld4(y2 + (L - 1 + l - 2) * C) * s);
      }
    }
  }
}

template <int L>
__global__ __launch_bounds__(256) void gating_bwd_lmax_kernel(
    const float* __restrict__ gZ0, const float* __restrict__ gZ1, const float* __restrict__ gZ2,
    const float* __restrict__ Y0, const float* __restrict__ Y1, const float* __restrict__ Y2,
    float* __restrict__ gY0, float* __restrict__ gY1, float* __restrict__ gY2, int64_t total, int32_t C4) {
  const int64_t C = 4 * (int64_t)C4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = t / C4;
    const int64_t c = 4 * (t - e * C4);
    const float* y0 = Y0 + e * (2 * L + 1) * C + c;
    const float* y1 = Y1 + e * 2 * L * C + c;
    const float* y2 = Y2 + e * 2 * (L - 1) * C + c;
    const float* g0 = gZ0 + e * (L + 1) * C + c;
    const float* g1 = gZ1 + e * 2 * L * C + c;
    const float* g2 = gZ2 + e * 2 * (L - 1) * C + c;
    float* o0 = gY0 + e * (2 * L + 1) * C + c;
    float* o1 = gY1 + e * 2 * L * C + c;
    float* o2 = gY2 + e * 2 * (L - 1) * C + c;
    {
      const float4 l0 = ld4(y0 + L * C), gl = ld4(g0);
      float4 o;
      float* op = &o.x;
      const float* lp = &l0.x;
      const float* gp = &gl.x;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float sl = sigmoidf_(lp[q]), dsl = sl * (1.0f - sl);
        op[q] = gp[q] * (sl + lp[q] * dsl);
      }
      st4(o0 + L * C, o);
    }
#pragma unroll
    for (int l = 1; l <= L; ++l) {
      const float4 a = ld4(y0 + (l - 1) * C);
      const float4 yl = ld4(y0 + (L + l) * C), gl = ld4(g0 + l * C);
      const float4 r = ld4(y1 + (l - 1) * C), gr = ld4(g1 + (l - 1) * C);
      const float4 im = ld4(y1 + (L + l - 1) * C), gi = ld4(g1 + (L + l - 1) * C);
      float4 r2 = make_float4(0.f, 0.f, 0.f, 0.f), gr2 = r2, i2 = r2, gi2 = r2;
      if (l >= 2) {
        r2 = ld4(y2 + (l - 2) * C);
        gr2 = ld4(g2 + (l - 2) * C);
        i2 = ld4(y2 + (L - 1 + l - 2) * C);
        gi2 = ld4(g2 + (L - 1 + l - 2) * C);
      }
      float4 og, oy, orr, oi, or2, oi2;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float s = sigmoidf_((&a.x)[q]), ds = s * (1.0f - s);
        float acc = (&gl.x)[q] * (&yl.x)[q] + (&gr.x)[q] * (&r.x)[q] + (&gi.x)[q] * (&im.x)[q];
        if (l >= 2) acc = acc + (&gr2.x)[q] * (&r2.x)[q] + (&gi2.x)[q] * (&i2.x)[q];
        (&og.x)[q] = ds * acc;
        (&oy.x)[q] = (&gl.x)[q] * s;
        (&orr.x)[q] = (&gr.x)[q] * s;
        (&oi.x)[q] = (&gi.x)[q] * s;
        (&or2.x)[q] = (&gr2.x)[q] * s;
        (&oi2.x)[q] = (&gi2.x)[q] * s;
      }
      st4(o0 + (l - 1) * C, og);
      st4(o0 + (L + l) * C, oy);
      st4(o1 + (l - 1) * C, orr);
      st4(o1 + (L + l - 1) * C, oi);
      if (l >= 2) {
        st4(o2 + (l - 2) * C, or2);
        st4(o2 + (L - 1 + l - 2) * C, oi2);
      }
    }
  }
}

}  // namespace lm
}  // namespace fu

using namespace fu;
using namespace fu::lm;

// Instantiate f for CPL = C / 64 and lmax.
template <typename F>
static void with_c_lmax(int32_t C, int32_t lmax, F f) {
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using L2 = std::integral_constant<int, 2>;
  using L3 = std::integral_constant<int, 3>;
  using L4 = std::integral_constant<int, 4>;
  auto by_l = [&](auto cpl) {
    if (lmax == 2) f(cpl, L2{});
    else if (lmax == 3) f(cpl, L3{});
    else f(cpl, L4{});
  };
  if (C == 64) by_l(I1{});
  else if (C == 128) by_l(I2{});
  else by_l(I4{});
}

template <typename F>
static void with_lmax(int32_t lmax, F f) {
  if (lmax == 2) f(std::integral_constant<int, 2>{});
  else if (lmax == 3) f(std::integral_constant<int, 3>{});
  else f(std::integral_constant<int, 4>{});
}

static int check_cl(int32_t C, int32_t lmax, const char* who) {
  if (C != 64 && C != 128 && C != 256)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d unsupported (64, 128 or 256)", who, C);
  if (lmax < 2 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d unsupported (2, 3 or 4)", who, lmax);
  return FU_OK;
}

static bool ext_ok(const float* p, int32_t lmax) { return lmax == 2 || p != nullptr; }

extern "C" int fu_gather_fwd_lmax(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                                  const float* wig_ext, const float* rad, const float* csd_emb, const int64_t* batch,
                                  const int32_t* recv_ptr, const int32_t* recv_idx, const int32_t* send_ptr,
                                  const int32_t* send_idx, float* X_m0, float* X_m1, float* X_m2, int64_t E, int64_t N,
                                  int64_t S, int32_t C, int32_t lmax, void* stream) {
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_fwd_lmax: bad shape");
  int st = check_cl(C, lmax, "fu_gather_fwd_lmax");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!x || !idx_i || !idx_j || !wigner || !ext_ok(wig_ext, lmax) || !rad || !csd_emb || !batch || !X_m0 || !X_m1 ||
      !X_m2)
    return set_error(FU_ERR_NULL, "fu_gather_fwd_lmax: NULL argument");
  const void* al[] = {x, rad, csd_emb, X_m0, X_m1, X_m2};
  for (const void* p : al)
    if (!aligned16(p)) return set_error(FU_ERR_ALIGN, "fu_gather_fwd_lmax: feature arrays must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const bool csrs = recv_ptr && recv_idx && send_ptr && send_idx;
  if (!csrs && (recv_ptr || recv_idx || send_ptr || send_idx))
    return set_error(FU_ERR_NULL, "fu_gather_fwd_lmax: pass all four CSR arrays or none");
  if (csrs && N > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_gather_fwd_lmax: N too large");
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    if (csrs) {
      if (N > 0)
        hipLaunchKernelGGL((gather_fwd_node_lmax_kernel<P, L>), dim3((unsigned)N), dim3(128), 0, s, x, wigner, wig_ext,
                           rad, csd_emb, batch, recv_ptr, recv_idx, send_ptr, send_idx, X_m0, X_m1, X_m2);
    } else {
      hipLaunchKernelGGL((gather_fwd_lmax_kernel<P, L>), dim3(edge_grid(E)), dim3(256),
                         0, s, x, idx_i, idx_j, wigner, wig_ext, rad, csd_emb, batch, X_m0, X_m1, X_m2, E);
    }
  });
  return check_launch("fu_gather_fwd_lmax");
}

extern "C" int fu_gather_bwd_lmax(const float* g_X_m0, const float* g_X_m1, const float* g_X_m2, const float* x,
                                  const float* wigner, const float* wig_ext, const float* rad, const float* csd_emb,
                                  const int64_t* batch, const int32_t* recv_ptr, const int32_t* recv_idx,
                                  const int32_t* send_ptr, const int32_t* send_idx, float* g_x, float* g_wigner,
                                  float* g_wig_ext, float* g_rad, float* ws, int64_t E, int64_t N, int64_t S,
                                  int32_t C, int32_t lmax, int32_t accumulate, void* stream) {
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_bwd_lmax: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_gather_bwd_lmax: accumulate=%d (0..3)", accumulate);
  int st = check_cl(C, lmax, "fu_gather_bwd_lmax");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (N > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_gather_bwd_lmax: N too large");
  if (!x || !csd_emb || !batch || !recv_ptr || !send_ptr || !g_x)
    return set_error(FU_ERR_NULL, "fu_gather_bwd_lmax: NULL argument");
  if (E > 0 && (!g_X_m0 || !g_X_m1 || !g_X_m2 || !wigner || !ext_ok(wig_ext, lmax) || !rad || !recv_idx ||
                !send_idx || !g_wigner || !ext_ok(g_wig_ext, lmax) || !g_rad || !ws))
    return set_error(FU_ERR_NULL, "fu_gather_bwd_lmax: NULL argument");
  const int EW = extw(lmax);
  hipStream_t s = as_stream(stream);
  float* ws_w = ws;
  float* ws_x = ws + E * 34;
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    hipLaunchKernelGGL((gather_bwd_lmax_kernel<P, L>), dim3((unsigned)N), dim3(128), 0, s, g_X_m0, g_X_m1, g_X_m2, x,
                       wigner, wig_ext, rad, csd_emb, batch, recv_ptr, recv_idx, send_ptr, send_idx, g_x, g_wigner,
                       g_wig_ext, ws_w, ws_x, g_rad, N, accumulate);
  });
  st = check_launch("fu_gather_bwd_lmax");
  if (st != FU_OK || E == 0) return st;
  hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)std::min<int64_t>(cdiv(E * 34, 256), 65536)), dim3(256), 0, s,
                     g_wigner, ws_w, E * 34);
  if (EW > 0)
    hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)std::min<int64_t>(cdiv(E * EW, 256), 65536)), dim3(256), 0, s,
                       g_wig_ext, ws_x, E * EW);
  return check_launch("fu_gather_bwd_lmax(add)");
}

extern "C" int fu_scatter_fwd_lmax(const int32_t* row_ptr, const int32_t* col_idx, const float* Z_m0,
                                   const float* Z_m1, const float* Z_m2, const float* wigner, const float* wig_ext,
                                   const float* env, const float* x_res, float* x_out, int64_t N, int64_t E, int32_t C,
                                   int32_t lmax, void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_scatter_fwd_lmax: bad shape");
  int st = check_cl(C, lmax, "fu_scatter_fwd_lmax");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!row_ptr || !x_res || !x_out ||
      (E > 0 && (!col_idx || !Z_m0 || !Z_m1 || !Z_m2 || !wigner || !ext_ok(wig_ext, lmax) || !env)))
    return set_error(FU_ERR_NULL, "fu_scatter_fwd_lmax: NULL argument");
  hipStream_t s = as_stream(stream);
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    hipLaunchKernelGGL((scatter_fwd_lmax_kernel<P, L>), dim3(cdiv(N, 4)), dim3(256), 0, s, row_ptr, col_idx, Z_m0,
                       Z_m1, Z_m2, wigner, wig_ext, env, x_res, x_out, N);
  });
  return check_launch("fu_scatter_fwd_lmax");
}

extern "C" int fu_scatter_bwd_lmax(const float* g_out, const int64_t* idx_j, const float* Z_m0, const float* Z_m1,
                                   const float* Z_m2, const float* wigner, const float* wig_ext, const float* env,
                                   float* g_Z_m0, float* g_Z_m1, float* g_Z_m2, float* g_wigner, float* g_wig_ext,
                                   float* g_env, int64_t E, int64_t N, int32_t C, int32_t lmax, int32_t accumulate,
                                   void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_scatter_bwd_lmax: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_scatter_bwd_lmax: accumulate=%d (0..3)", accumulate);
  int st = check_cl(C, lmax, "fu_scatter_bwd_lmax");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!g_out || !idx_j || !Z_m0 || !Z_m1 || !Z_m2 || !wigner || !ext_ok(wig_ext, lmax) || !env || !g_Z_m0 ||
      !g_Z_m1 || !g_Z_m2 || !g_wigner || !ext_ok(g_wig_ext, lmax) || !g_env)
    return set_error(FU_ERR_NULL, "fu_scatter_bwd_lmax: NULL argument");
  hipStream_t s = as_stream(stream);
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    hipLaunchKernelGGL((scatter_bwd_lmax_kernel<P, L>), dim3(edge_grid(E)),
                       dim3(256), 0, s, g_out, idx_j, Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, g_Z_m0, g_Z_m1, g_Z_m2,
                       g_wigner, g_wig_ext, g_env, E, accumulate);
  });
  return check_launch("fu_scatter_bwd_lmax");
}

extern "C" int fu_init_scatter_fwd_lmax(const int32_t* row_ptr, const int32_t* col_idx, const float* rad,
                                        const float* wigner, const float* wig_ext, const float* env, const int64_t* Z,
                                        const int64_t* batch, const float* W_sphere, const float* csd_emb,
                                        float* x_out, int64_t N, int64_t E, int64_t num_z, int64_t S, int32_t C,
                                        int32_t lmax, void* stream) {
  if (N < 0 || E < 0 || num_z < 1 || S < 1) return set_error(FU_ERR_SHAPE, "fu_init_scatter_fwd_lmax: bad shape");
  int st = check_cl(C, lmax, "fu_init_scatter_fwd_lmax");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!row_ptr || !Z || !batch || !W_sphere || !csd_emb || !x_out ||
      (E > 0 && (!col_idx || !rad || !wigner || !ext_ok(wig_ext, lmax) || !env)))
    return set_error(FU_ERR_NULL, "fu_init_scatter_fwd_lmax: NULL argument");
  hipStream_t s = as_stream(stream);
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    hipLaunchKernelGGL((init_scatter_fwd_lmax_kernel<P, L>), dim3(cdiv(N, 4)), dim3(256), 0, s, row_ptr, col_idx, rad,
                       wigner, wig_ext, env, Z, batch, W_sphere, csd_emb, x_out, N);
  });
  return check_launch("fu_init_scatter_fwd_lmax");
}

extern "C" int fu_init_scatter_bwd_lmax(const float* g_out, const int64_t* idx_j, const float* rad,
                                        const float* wigner, const float* wig_ext, const float* env, float* g_rad,
                                        float* g_wigner, float* g_wig_ext, float* g_env, int64_t E, int64_t N,
                                        int32_t C, int32_t lmax, int32_t accumulate, void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_init_scatter_bwd_lmax: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_init_scatter_bwd_lmax: accumulate=%d (0..3)", accumulate);
  int st = check_cl(C, lmax, "fu_init_scatter_bwd_lmax");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!g_out || !idx_j || !rad || !wigner || !ext_ok(wig_ext, lmax) || !env || !g_rad || !g_wigner ||
      !ext_ok(g_wig_ext, lmax) || !g_env)
    return set_error(FU_ERR_NULL, "fu_init_scatter_bwd_lmax: NULL argument");
  hipStream_t s = as_stream(stream);
  with_c_lmax(C, lmax, [&](auto cpl, auto lv) {
    constexpr int P = decltype(cpl)::value, L = decltype(lv)::value;
    hipLaunchKernelGGL((init_scatter_bwd_lmax_kernel<P, L>), dim3(edge_grid(E)),
                       dim3(256), 0, s, g_out, idx_j, rad, wigner, wig_ext, env, g_rad, g_wigner, g_wig_ext, g_env, E,
                       accumulate);
  });
  return check_launch("fu_init_scatter_bwd_lmax");
}

static int gating_lmax_check(const void* const* ptrs, int n, int64_t E, int32_t C, int32_t lmax, const char* who) {
  if (E < 0 || C <= 0) return set_error(FU_ERR_SHAPE, "%s: bad shape E=%lld C=%d", who, (long long)E, C);
  if (C % 4 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 4", who, C);
  if (lmax < 2 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d unsupported (2, 3 or 4)", who, lmax);
  for (int k = 0; k < n && E > 0; ++k) {
    if (ptrs[k] == nullptr) return set_error(FU_ERR_NULL, "%s: pointer %d is NULL", who, k);
    if (!aligned16(ptrs[k])) return set_error(FU_ERR_ALIGN, "%s: pointer %d not 16-byte aligned", who, k);
  }
  return FU_OK;
}

extern "C" int fu_gating_fwd_lmax(const float* Y_m0, const float* Y_m1, const float* Y_m2, float* Z_m0, float* Z_m1,
                                  float* Z_m2, int64_t E, int32_t C, int32_t lmax, void* stream) {
  const void* ptrs[] = {Y_m0, Y_m1, Y_m2, Z_m0, Z_m1, Z_m2};
  int st = gating_lmax_check(ptrs, 6, E, C, lmax, "fu_gating_fwd_lmax");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  const int64_t total = E * (C / 4);
  const int64_t blocks = std::min<int64_t>(cdiv(total, 256), kMaxBlocks);
  with_lmax(lmax, [&](auto lv) {
    hipLaunchKernelGGL((gating_fwd_lmax_kernel<decltype(lv)::value>), dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), Y_m0, Y_m1, Y_m2, Z_m0, Z_m1, Z_m2, total, C / 4);
  });
  return check_launch("fu_gating_fwd_lmax");
}

extern "C" int fu_gating_bwd_lmax(const float* g_Z_m0, const float* g_Z_m1, const float* g_Z_m2, const float* Y_m0,
                                  const float* Y_m1, const float* Y_m2, float* g_Y_m0, float* g_Y_m1, float* g_Y_m2,
                                  int64_t E, int32_t C, int32_t lmax, void* stream) {
  const void* ptrs[] = {g_Z_m0, g_Z_m1, g_Z_m2, Y_m0, Y_m1, Y_m2, g_Y_m0, g_Y_m1, g_Y_m2};
  int st = gating_lmax_check(ptrs, 9, E, C, lmax, "fu_gating_bwd_lmax");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  const int64_t total = E * (C / 4);
  const int64_t blocks = std::min<int64_t>(cdiv(total, 256), kMaxBlocks);
  with_lmax(lmax, [&](auto lv) {
    hipLaunchKernelGGL((gating_bwd_lmax_kernel<decltype(lv)::value>), dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), g_Z_m0, g_Z_m1, g_Z_m2, Y_m0, Y_m1, Y_m2, g_Y_m0, g_Y_m1, g_Y_m2, total,
                       C / 4);
  });
  return check_launch("fu_gating_bwd_lmax");
}
