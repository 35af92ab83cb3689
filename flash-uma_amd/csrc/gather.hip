// Gather-rotate of sender/receiver SH rows into the edge frame (ops/gather.py:34-154) and
// its backward pass (ops/gather.py:160-405) without atomics.
//
// Forward: one wave64 per edge, lanes across channels (CPL = C/64 per lane); each workgroup
// takes a contiguous edge range, XCD-aware (block_edge_range).  The edge's indices and its 34
// Wigner scalars are wave-uniform (scalar loads); every node row, radial row and output slot
// is one coalesced row access.  At C = 128 a wave takes two edges, 32 lanes of 4 channels
// each (gather_fwd_pair_kernel).
//
// Backward: node-centric.  A 128-thread workgroup owns one node: one wave walks the node's
// receiver segment (edges e with idx_j[e] = n, receiver CSR) and the other its sender
// segment (idx_i[e] = n, sender CSR).  Each wave recomputes the rotated own row,
// writes its half of g_rad, accumulates D^T g into the node gradient in CSR order, and
// reduces its half of g_wigner across lanes.  The two node partials are added through LDS
// (receiver part + sender part) and g_x[n] is written once: deterministic, no atomics.
#include "edge_layout.h"
#include "fu_vec.h"

namespace fu {

template <int CPL>
struct Rows9 {
  Vec<CPL> r[9];
};

// rv = diag(1, D1, D2) v with wigner scalars w (row-major L=1 then L=2 block).
template <int CPL>
__device__ __forceinline__ void rotate9(const float* w, const Rows9<CPL>& v, Rows9<CPL>& out) {
  out.r[0] = v.r[0];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
      out.r[1 + a][q] = w[3 * a + 0] * v.r[1][q] + w[3 * a + 1] * v.r[2][q] + w[3 * a + 2] * v.r[3][q];
  }
#pragma unroll
  for (int a = 0; a < 5; ++a) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
      out.r[4 + a][q] = w[9 + 5 * a + 0] * v.r[4][q] + w[9 + 5 * a + 1] * v.r[5][q] + w[9 + 5 * a + 2] * v.r[6][q] +
                        w[9 + 5 * a + 3] * v.r[7][q] + w[9 + 5 * a + 4] * v.r[8][q];
  }
}

// out += diag(1, D1, D2)^T g
template <int CPL>
__device__ __forceinline__ void add_rotate9_t(const float* w, const Rows9<CPL>& g, Rows9<CPL>& out) {
#pragma unroll
  for (int q = 0; q < CPL; ++q) out.r[0][q] += g.r[0][q];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
      out.r[1 + b][q] += w[0 + b] * g.r[1][q] + w[3 + b] * g.r[2][q] + w[6 + b] * g.r[3][q];
  }
#pragma unroll
  for (int b = 0; b < 5; ++b) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
      out.r[4 + b][q] += w[9 + b] * g.r[4][q] + w[14 + b] * g.r[5][q] + w[19 + b] * g.r[6][q] +
                         w[24 + b] * g.r[7][q] + w[29 + b] * g.r[8][q];
  }
}

__device__ __forceinline__ int wave_id_uniform() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// M0 false: the m = 0 slots are neither computed nor stored (X0 unused), nor are their radial
// blocks read: conv1 m = 0 gathers its operand itself (fu_gather_linear_gate).
template <int CPL, int L, bool M0 = true>
__global__ __launch_bounds__(256) void gather_fwd_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j,
    const float* __restrict__ wig, const float* __restrict__ rad, const float* __restrict__ csd,
    const int64_t* __restrict__ batch, float* __restrict__ X0, float* __restrict__ X1,
    float* __restrict__ X2, int64_t E) {
  constexpr int C = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_id_uniform(); e < e1; e += (blockDim.x >> 6)) {
    const int64_t i = idx_i[e], j = idx_j[e];
    float w[34];
#pragma unroll
    for (int k = 0; k < 34; ++k) w[k] = wig[e * 34 + k];
    Rows9<CPL> vs, vt, rs, rt;
    const float* xs = x + i * 9 * C + c;
    const float* xt = x + j * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      vs.r[k] = vload<CPL>(xs + k * C);
      vt.r[k] = vload<CPL>(xt + k * C);
    }
    vs.r[0] = vadd(vs.r[0], vload<CPL>(csd + batch[i] * C + c));
    vt.r[0] = vadd(vt.r[0], vload<CPL>(csd + batch[j] * C + c));
    rotate9(w, vs, rs);
    rotate9(w, vt, rt);
    // radial block k (reference numbering: even = sender, odd = receiver)
    const float* rr = rad + e * 12 * C + c;
    Vec<CPL> r[12];
#pragma unroll
    for (int k = M0 ? 0 : 6; k < 12; ++k) r[k] = vload_nt<CPL>(rr + slot_rad<L>(k & 1, k >> 1) * C);
    float* o0 = X0 + e * 6 * C + c;
    float* o1 = X1 + e * 8 * C + c;
    float* o2 = X2 + e * 4 * C + c;
    // m0 slots: rotated coefficient k0, k2, k6; m1: k3, k7 (R) and k1, k5 (I); m2: k8 (R), k4 (I)
    constexpr int K0[3] = {0, 2, 6}, K1[4] = {3, 7, 1, 5}, K2[2] = {8, 4};
    if constexpr (M0) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        vstore_nt(o0 + slot_m0<L>(0, q) * C, vmul(rs.r[K0[q]], r[2 * q]));
        vstore_nt(o0 + slot_m0<L>(1, q) * C, vmul(rt.r[K0[q]], r[2 * q + 1]));
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vstore_nt(o1 + slot_m1<L>(0, q) * C, vmul(rs.r[K1[q]], r[6 + 2 * (q & 1)]));
      vstore_nt(o1 + slot_m1<L>(1, q) * C, vmul(rt.r[K1[q]], r[7 + 2 * (q & 1)]));
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      vstore_nt(o2 + slot_m2<L>(0, q) * C, vmul(rs.r[K2[q]], r[10]));
      vstore_nt(o2 + slot_m2<L>(1, q) * C, vmul(rt.r[K2[q]], r[11]));
    }
  }
}

// C = 128 with two edges per wave: lanes 0-31 take edge e, lanes 32-63 edge e + 1, four
// channels per lane, so every access is 16 bytes per lane (against 8 with one edge per wave:
// 748-752 against 772-776 us at bcc Fe, bitwise equal outputs).  The Wigner scalars are then
// per-lane loads (two edges per wave), which the L1 serves.
template <int L, bool M0 = true>
__global__ __launch_bounds__(256) void gather_fwd_pair_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j,
    const float* __restrict__ wig, const float* __restrict__ rad, const float* __restrict__ csd,
    const int64_t* __restrict__ batch, float* __restrict__ X0, float* __restrict__ X1,
    float* __restrict__ X2, int64_t E) {
  constexpr int CPL = 4, C = 128;
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int c = (lane & 31) * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  const int nw = blockDim.x >> 6;
  for (int64_t eb = e0 + 2 * wave_id_uniform(); eb < e1; eb += 2 * nw) {
    // the second half of a wave at the range's odd end recomputes edge eb and stores nothing
    const bool live = eb + half < e1;
    const int64_t e = live ? eb + half : eb;
    const int64_t i = idx_i[e], j = idx_j[e];
    float w[34];
#pragma unroll
    for (int k = 0; k < 34; ++k) w[k] = wig[e * 34 + k];
    Rows9<CPL> vs, vt, rs, rt;
    const float* xs = x + i * 9 * C + c;
    const float* xt = x + j * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      vs.r[k] = vload<CPL>(xs + k * C);
      vt.r[k] = vload<CPL>(xt + k * C);
    }
    vs.r[0] = vadd(vs.r[0], vload<CPL>(csd + batch[i] * C + c));
    vt.r[0] = vadd(vt.r[0], vload<CPL>(csd + batch[j] * C + c));
    rotate9(w, vs, rs);
    rotate9(w, vt, rt);
    const float* rr = rad + e * 12 * C + c;
    Vec<CPL> r[12];
#pragma unroll
    for (int k = M0 ? 0 : 6; k < 12; ++k) r[k] = vload_nt<CPL>(rr + slot_rad<L>(k & 1, k >> 1) * C);
    if (!live) continue;
    float* o0 = X0 + e * 6 * C + c;
    float* o1 = X1 + e * 8 * C + c;
    float* o2 = X2 + e * 4 * C + c;
    constexpr int K0[3] = {0, 2, 6}, K1[4] = {3, 7, 1, 5}, K2[2] = {8, 4};
    if constexpr (M0) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        vstore_nt(o0 + slot_m0<L>(0, q) * C, vmul(rs.r[K0[q]], r[2 * q]));
        vstore_nt(o0 + slot_m0<L>(1, q) * C, vmul(rt.r[K0[q]], r[2 * q + 1]));
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vstore_nt(o1 + slot_m1<L>(0, q) * C, vmul(rs.r[K1[q]], r[6 + 2 * (q & 1)]));
      vstore_nt(o1 + slot_m1<L>(1, q) * C, vmul(rt.r[K1[q]], r[7 + 2 * (q & 1)]));
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      vstore_nt(o2 + slot_m2<L>(0, q) * C, vmul(rs.r[K2[q]], r[10]));
      vstore_nt(o2 + slot_m2<L>(1, q) * C, vmul(rt.r[K2[q]], r[11]));
    }
  }
}

// Per-edge data of one side of the gather backward (receiver side: so = 1, sender: so = 0).
// The Wigner scalars arrive as one vector load (lane q < 34 holds scalar q) so that every
// load of an edge is counted by vmcnt and the next edge's loads stay in flight while this
// edge is processed; they are broadcast with readlane when used.
template <int CPL>
struct SideEdge {
  float wl;
  Vec<CPL> g[9];   // this side's g_X slots: m0 a/b/c, m1 a/b/c/d, m2 a/b
  Vec<CPL> r[6];   // this side's radial blocks so, 2+so, ..., 10+so
};

__device__ __forceinline__ float read_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int CPL, int L>
__device__ __forceinline__ void side_load(const float* __restrict__ gX0, const float* __restrict__ gX1,
                                          const float* __restrict__ gX2, const float* __restrict__ wig,
                                          const float* __restrict__ rad, int64_t e, int so, int c, int lane,
                                          SideEdge<CPL>& d) {
  constexpr int C = 64 * CPL;
  d.wl = lane < 34 ? wig[e * 34 + lane] : 0.0f;
  const float* g0 = gX0 + e * 6 * C + c;
  const float* g1 = gX1 + e * 8 * C + c;
  const float* g2 = gX2 + e * 4 * C + c;
#pragma unroll
  for (int q = 0; q < 3; ++q) d.g[q] = vload_nt<CPL>(g0 + slot_m0<L>(so, q) * C);
#pragma unroll
  for (int q = 0; q < 4; ++q) d.g[3 + q] = vload_nt<CPL>(g1 + slot_m1<L>(so, q) * C);
#pragma unroll
  for (int q = 0; q < 2; ++q) d.g[7 + q] = vload_nt<CPL>(g2 + slot_m2<L>(so, q) * C);
  const float* rp = rad + e * 12 * C + c;
#pragma unroll
  for (int q = 0; q < 6; ++q) d.r[q] = vload_nt<CPL>(rp + slot_rad<L>(so, q) * C);
}

// v (the node's own row, csd added) is read from the wave's LDS copy, so that it holds no
// VGPRs across the loop; the registers go to the edges in flight instead.
template <int CPL>
__device__ __forceinline__ Vec<CPL> lds_row(const float* sv, int k, int c) {
  return vload<CPL>(sv + k * (64 * CPL) + c);
}

template <int CPL, int L>
__device__ __forceinline__ void side_apply(const SideEdge<CPL>& d, int64_t e, int so, int c, const float* sv,
                                           Rows9<CPL>& acc, float* __restrict__ g_rad, float* __restrict__ gw_out,
                                           int lane, bool accw) {
  constexpr int C = 64 * CPL;
  float w[34];
#pragma unroll
  for (int q = 0; q < 34; ++q) w[q] = read_lane(d.wl, q);
  {
    Rows9<CPL> v, rv;
#pragma unroll
    for (int k = 0; k < 9; ++k) v.r[k] = lds_row<CPL>(sv, k, c);
    rotate9(w, v, rv);
    // this side's radial gradients (reference blocks so, 2+so, ..., 10+so)
    float* gr = g_rad + e * 12 * C + c;
    vstore_nt(gr + slot_rad<L>(so, 0) * C, vmul(d.g[0], rv.r[0]));
    vstore_nt(gr + slot_rad<L>(so, 1) * C, vmul(d.g[1], rv.r[2]));
    vstore_nt(gr + slot_rad<L>(so, 2) * C, vmul(d.g[2], rv.r[6]));
    vstore_nt(gr + slot_rad<L>(so, 3) * C, vadd(vmul(d.g[3], rv.r[3]), vmul(d.g[5], rv.r[1])));
    vstore_nt(gr + slot_rad<L>(so, 4) * C, vadd(vmul(d.g[4], rv.r[7]), vmul(d.g[6], rv.r[5])));
    vstore_nt(gr + slot_rad<L>(so, 5) * C, vadd(vmul(d.g[7], rv.r[8]), vmul(d.g[8], rv.r[4])));
  }
  // gradient w.r.t. the rotated coefficients of this node's row
  Rows9<CPL> grv;
  grv.r[0] = vmul(d.g[0], d.r[0]);
  grv.r[2] = vmul(d.g[1], d.r[1]);
  grv.r[6] = vmul(d.g[2], d.r[2]);
  grv.r[3] = vmul(d.g[3], d.r[3]);
  grv.r[7] = vmul(d.g[4], d.r[4]);
  grv.r[1] = vmul(d.g[5], d.r[3]);
  grv.r[5] = vmul(d.g[6], d.r[4]);
  grv.r[8] = vmul(d.g[7], d.r[5]);
  grv.r[4] = vmul(d.g[8], d.r[5]);
  add_rotate9_t(w, grv, acc);
  // this side's g_wigner: dL/dD1[a][b] = sum_c grv[1+a] v[1+b], dL/dD2[a][b] = sum_c grv[4+a] v[4+b],
  // reduced in two batches (entries 0..23 as 32 values, 24..33 as 16) to bound live registers
  {
    float part[32];
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const Vec<CPL> vb = lds_row<CPL>(sv, 1 + b, c);
#pragma unroll
      for (int a = 0; a < 3; ++a) part[3 * a + b] = vdot(grv.r[1 + a], vb);
    }
#pragma unroll
    for (int b = 0; b < 5; ++b) {
      const Vec<CPL> vb = lds_row<CPL>(sv, 4 + b, c);
#pragma unroll
      for (int a = 0; a < 3; ++a) part[9 + 5 * a + b] = vdot(grv.r[4 + a], vb);
    }
#pragma unroll
    for (int q = 24; q < 32; ++q) part[q] = 0.0f;
    const float tot = wave_multi_sum<32>(part, lane);
    if (lane < 24) gw_out[e * 34 + lane] = accw ? gw_out[e * 34 + lane] + tot : tot;
  }
  {
    float part[16];
#pragma unroll
    for (int b = 0; b < 5; ++b) {
      const Vec<CPL> vb = lds_row<CPL>(sv, 4 + b, c);
#pragma unroll
      for (int a = 3; a < 5; ++a) part[5 * (a - 3) + b] = vdot(grv.r[4 + a], vb);
    }
#pragma unroll
    for (int q = 10; q < 16; ++q) part[q] = 0.0f;
    const float tot = wave_multi_sum<16>(part, lane);
    if (lane < 10) gw_out[e * 34 + 24 + lane] = accw ? gw_out[e * 34 + 24 + lane] + tot : tot;
  }
}

// One side of one node's gather backward: walk the node's CSR segment in order.  The
// segment's edge ids are fetched 64 at a time into one VGPR (lane t holds the t-th id) and
// broadcast with readlane; the loads of edge t+1 are issued before edge t is processed.
template <int CPL, int L>
__device__ __forceinline__ void gather_bwd_side(const float* __restrict__ gX0, const float* __restrict__ gX1,
                                                const float* __restrict__ gX2, const float* __restrict__ wig,
                                                const float* __restrict__ rad, const int32_t* __restrict__ ptr,
                                                const int32_t* __restrict__ idx, int64_t n, int so, const float* sv,
                                                Rows9<CPL>& acc, float* __restrict__ g_rad,
                                                float* __restrict__ gw_out, int lane, bool accw) {
  const int c = lane * CPL;
  const int32_t k0 = ptr[n], k1 = ptr[n + 1];
  for (int32_t base = k0; base < k1; base += 64) {
    const int cnt = (int)std::min<int32_t>(64, k1 - base);
    const int32_t ids = lane < cnt ? idx[base + lane] : 0;
    SideEdge<CPL> d0, d1;
    int64_t e0 = __builtin_amdgcn_readlane(ids, 0);
    side_load<CPL, L>(gX0, gX1, gX2, wig, rad, e0, so, c, lane, d0);
    int t = 0;
    // sched_barrier(0) keeps the scheduler from sinking the next edge's loads into the
    // current edge's arithmetic, which would shrink the prefetch distance below one edge.
    for (; t + 2 <= cnt; t += 2) {
      const int64_t e1 = __builtin_amdgcn_readlane(ids, t + 1);
      side_load<CPL, L>(gX0, gX1, gX2, wig, rad, e1, so, c, lane, d1);
      __builtin_amdgcn_sched_barrier(0);
      side_apply<CPL, L>(d0, e0, so, c, sv, acc, g_rad, gw_out, lane, accw);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 2 < cnt) {
        e0 = __builtin_amdgcn_readlane(ids, t + 2);
        side_load<CPL, L>(gX0, gX1, gX2, wig, rad, e0, so, c, lane, d0);
      }
      __builtin_amdgcn_sched_barrier(0);
      side_apply<CPL, L>(d1, e1, so, c, sv, acc, g_rad, gw_out, lane, accw);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (t < cnt) side_apply<CPL, L>(d0, e0, so, c, sv, acc, g_rad, gw_out, lane, accw);
  }
}

// One node per 128-thread workgroup (wave 0: receiver segment, wave 1: sender segment); at
// least 3 waves per SIMD, since the loop is bound by the number of edge loads in flight.  At
// C = 256 two edges in flight need more than the 170 registers of 3 waves per SIMD (449
// spilled to scratch) or the 256 of 2 (116): one wave per SIMD keeps them in registers and
// accumulation registers (2.26x faster at 245,760 edges: 5,160 -> 2,285 us).
template <int CPL, int L>
__global__ __launch_bounds__(128, CPL >= 4 ? 1 : 3) void gather_bwd_kernel(
    const float* __restrict__ gX0, const float* __restrict__ gX1, const float* __restrict__ gX2,
    const float* __restrict__ x, const float* __restrict__ wig, const float* __restrict__ rad,
    const float* __restrict__ csd, const int64_t* __restrict__ batch, const int32_t* __restrict__ rptr,
    const int32_t* __restrict__ ridx, const int32_t* __restrict__ sptr, const int32_t* __restrict__ sidx,
    float* __restrict__ g_x, float* __restrict__ g_wig, float* __restrict__ g_rad, float* __restrict__ ws,
    int64_t N, int32_t acc_flags) {
  constexpr int C = 64 * CPL;
  __shared__ __attribute__((aligned(16))) float s_send[1][9 * C];
  __shared__ __attribute__((aligned(16))) float s_v[2][9 * C];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id_uniform();
  const int node_local = 0;
  const int side = wave;  // 0: receiver segment, 1: sender segment
  const int64_t n = (int64_t)blockIdx.x;
  const int c = lane * CPL;
  Rows9<CPL> acc;
#pragma unroll
  for (int k = 0; k < 9; ++k) acc.r[k] = vzero<CPL>();
  if (n < N) {
    // the node's own row (csd added on l = 0) in this wave's LDS slot; each lane reads back
    // only the channels it wrote, so no barrier is needed
    float* sv = s_v[wave];
    const float* xn = x + n * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      Vec<CPL> r = vload<CPL>(xn + k * C);
      if (k == 0) r = vadd(r, vload<CPL>(csd + batch[n] * C + c));
      vstore(sv + k * C + c, r);
    }
    if (side == 0) {
      // receiver half into g_wigner (added to its contents when accumulating: only this wave
      // writes an edge's entries there); sender half into the workspace, added afterwards
      gather_bwd_side<CPL, L>(gX0, gX1, gX2, wig, rad, rptr, ridx, n, 1, sv, acc, g_rad, g_wig, lane,
                              (acc_flags & 1) != 0);
    } else {
      gather_bwd_side<CPL, L>(gX0, gX1, gX2, wig, rad, sptr, sidx, n, 0, sv, acc, g_rad, ws, lane, false);
#pragma unroll
      for (int k = 0; k < 9; ++k) vstore(&s_send[node_local][k * C + c], acc.r[k]);
    }
  }
  __syncthreads();
  if (n < N && side == 0) {
    float* gx = g_x + n * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) vstore(gx + k * C, vadd(acc.r[k], vload<CPL>(&s_send[node_local][k * C + c])));
  }
}

__global__ __launch_bounds__(256) void add_inplace_kernel(float* __restrict__ a, const float* __restrict__ b,
                                                          int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
    a[k] += b[k];
}

template <int CPL, int L>
static void launch_gather_fwd(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                              const float* rad, const float* csd, const int64_t* batch, float* X0, float* X1,
                              float* X2, int64_t E, hipStream_t st) {
  if constexpr (CPL == 2) {
    if (X0)
      hipLaunchKernelGGL((gather_fwd_pair_kernel<L>), dim3(edge_grid(E)), dim3(256), 0, st, x, idx_i, idx_j, wigner,
                         rad, csd, batch, X0, X1, X2, E);
    else
      hipLaunchKernelGGL((gather_fwd_pair_kernel<L, false>), dim3(edge_grid(E)), dim3(256), 0, st, x, idx_i, idx_j,
                         wigner, rad, csd, batch, X0, X1, X2, E);
  } else if (X0) {
    hipLaunchKernelGGL((gather_fwd_kernel<CPL, L>), dim3(edge_grid(E)), dim3(256), 0, st, x, idx_i, idx_j, wigner,
                       rad, csd, batch, X0, X1, X2, E);
  } else {
    hipLaunchKernelGGL((gather_fwd_kernel<CPL, L, false>), dim3(edge_grid(E)), dim3(256), 0, st, x, idx_i, idx_j,
                       wigner, rad, csd, batch, X0, X1, X2, E);
  }
}

template <int CPL, int L>
static void launch_gather_bwd(const float* gX0, const float* gX1, const float* gX2, const float* x,
                              const float* wigner, const float* rad, const float* csd, const int64_t* batch,
                              const int32_t* rptr, const int32_t* ridx, const int32_t* sptr, const int32_t* sidx,
                              float* g_x, float* g_wig, float* g_rad, float* ws, int64_t N, int32_t acc,
                              hipStream_t st) {
  hipLaunchKernelGGL((gather_bwd_kernel<CPL, L>), dim3((unsigned)N), dim3(128), 0, st, gX0, gX1, gX2, x, wigner, rad, csd,
                     batch, rptr, ridx, sptr, sidx, g_x, g_wig, g_rad, ws, N, acc);
}

}  // namespace fu

using namespace fu;

// Instantiate f for CPL = C / 64 and the slot layout.
template <typename F>
static void with_c_layout(int32_t C, int32_t layout, F f) {
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using L0 = std::integral_constant<int, 0>;
  using L1 = std::integral_constant<int, 1>;
  if (C == 64) layout ? f(I1{}, L1{}) : f(I1{}, L0{});
  else if (C == 128) layout ? f(I2{}, L1{}) : f(I2{}, L0{});
  else layout ? f(I4{}, L1{}) : f(I4{}, L0{});
}

static int check_c(int32_t C, const char* who) {
  if (C != 64 && C != 128 && C != 256)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d unsupported (64, 128 or 256)", who, C);
  return FU_OK;
}

extern "C" int fu_gather_fwd(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                             const float* rad, const float* csd_emb, const int64_t* batch, float* X_m0, float* X_m1,
                             float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C, int32_t layout,
                             void* stream) {
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_fwd: bad shape");
  if (layout != 0 && layout != 1) return set_error(FU_ERR_UNSUPPORTED, "fu_gather_fwd: layout %d", layout);
  int st = check_c(C, "fu_gather_fwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  // X_m0 may be NULL: the m = 0 part is then skipped (its GEMM gathers it, fu_gather_linear_gate)
  if (!x || !idx_i || !idx_j || !wigner || !rad || !csd_emb || !batch || !X_m1 || !X_m2)
    return set_error(FU_ERR_NULL, "fu_gather_fwd: NULL argument");
  const void* al[] = {x, rad, csd_emb, X_m0 ? X_m0 : X_m1, X_m1, X_m2};
  for (const void* p : al)
    if (!aligned16(p)) return set_error(FU_ERR_ALIGN, "fu_gather_fwd: feature arrays must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  with_c_layout(C, layout, [&](auto cpl, auto lay) {
    launch_gather_fwd<decltype(cpl)::value, decltype(lay)::value>(x, idx_i, idx_j, wigner, rad, csd_emb, batch, X_m0,
                                                                  X_m1, X_m2, E, s);
  });
  return check_launch("fu_gather_fwd");
}

extern "C" int fu_gather_bwd(const float* g_X_m0, const float* g_X_m1, const float* g_X_m2, const float* x,
                             const int64_t* idx_i, const int64_t* idx_j, const float* wigner, const float* rad,
                             const float* csd_emb, const int64_t* batch, const int32_t* recv_ptr,
                             const int32_t* recv_idx, const int32_t* send_ptr, const int32_t* send_idx, float* g_x,
                             float* g_wigner, float* g_rad, float* g_wig_ws, int64_t E, int64_t N, int64_t S,
                             int32_t C, int32_t layout, int32_t accumulate, void* stream) {
  (void)idx_i;
  (void)idx_j;
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_bwd: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_gather_bwd: accumulate=%d (0..3)", accumulate);
  if (layout != 0 && layout != 1) return set_error(FU_ERR_UNSUPPORTED, "fu_gather_bwd: layout %d", layout);
  int st = check_c(C, "fu_gather_bwd");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (N > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_gather_bwd: N too large");
  if (!x || !csd_emb || !batch || !recv_ptr || !send_ptr || !g_x)
    return set_error(FU_ERR_NULL, "fu_gather_bwd: NULL argument");
  if (E > 0 && (!g_X_m0 || !g_X_m1 || !g_X_m2 || !wigner || !rad || !recv_idx || !send_idx || !g_wigner || !g_rad ||
                !g_wig_ws))
    return set_error(FU_ERR_NULL, "fu_gather_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  with_c_layout(C, layout, [&](auto cpl, auto lay) {
    launch_gather_bwd<decltype(cpl)::value, decltype(lay)::value>(g_X_m0, g_X_m1, g_X_m2, x, wigner, rad, csd_emb,
                                                                  batch, recv_ptr, recv_idx, send_ptr, send_idx, g_x,
                                                                  g_wigner, g_rad, g_wig_ws, N, accumulate, s);
  });
  st = check_launch("fu_gather_bwd");
  if (st != FU_OK || E == 0) return st;
  const int64_t tot = E * 34;
  hipLaunchKernelGGL(add_inplace_kernel, dim3((unsigned)std::min<int64_t>(cdiv(tot, 256), 65536)), dim3(256), 0, s,
                     g_wigner, g_wig_ws, tot);
  return check_launch("fu_gather_bwd(add)");
}
