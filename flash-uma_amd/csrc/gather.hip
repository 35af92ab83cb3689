// Gather-rotate of sender/receiver SH rows into the edge frame (ops/gather.py:34-154) and
// its backward pass (ops/gather.py:160-405) without atomics.
//
// Forward: one wave64 per edge, lanes across channels (CPL = C/64 per lane).  The edge's
// indices and its 34 Wigner scalars are wave-uniform (scalar loads); every node row, radial
// row and output slot is one coalesced row access.
//
// Backward: node-centric.  A 256-thread workgroup owns two nodes; for each node one wave
// walks the node's receiver segment (edges e with idx_j[e] = n, receiver CSR) and one wave
// its sender segment (idx_i[e] = n, sender CSR).  Each wave recomputes the rotated own row,
// writes its half of g_rad, accumulates D^T g into the node gradient in CSR order, and
// reduces its half of g_wigner across lanes.  The two node partials are added through LDS
// (receiver part + sender part) and g_x[n] is written once: deterministic, no atomics.
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

template <int CPL>
__global__ __launch_bounds__(256) void gather_fwd_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ idx_i, const int64_t* __restrict__ idx_j,
    const float* __restrict__ wig, const float* __restrict__ rad, const float* __restrict__ csd,
    const int64_t* __restrict__ batch, float* __restrict__ X0, float* __restrict__ X1,
    float* __restrict__ X2, int64_t E) {
  constexpr int C = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t e = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_uniform(); e < E; e += waves) {
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
    for (int k = 0; k < 12; ++k) r[k] = vload<CPL>(rr + k * C);
    float* o0 = X0 + e * 6 * C + c;
    float* o1 = X1 + e * 8 * C + c;
    float* o2 = X2 + e * 4 * C + c;
    vstore(o0 + 0 * C, vmul(rs.r[0], r[0]));
    vstore(o0 + 1 * C, vmul(rt.r[0], r[1]));
    vstore(o0 + 2 * C, vmul(rs.r[2], r[2]));
    vstore(o0 + 3 * C, vmul(rt.r[2], r[3]));
    vstore(o0 + 4 * C, vmul(rs.r[6], r[4]));
    vstore(o0 + 5 * C, vmul(rt.r[6], r[5]));
    vstore(o1 + 0 * C, vmul(rs.r[3], r[6]));
    vstore(o1 + 1 * C, vmul(rt.r[3], r[7]));
    vstore(o1 + 2 * C, vmul(rs.r[7], r[8]));
    vstore(o1 + 3 * C, vmul(rt.r[7], r[9]));
    vstore(o1 + 4 * C, vmul(rs.r[1], r[6]));
    vstore(o1 + 5 * C, vmul(rt.r[1], r[7]));
    vstore(o1 + 6 * C, vmul(rs.r[5], r[8]));
    vstore(o1 + 7 * C, vmul(rt.r[5], r[9]));
    vstore(o2 + 0 * C, vmul(rs.r[8], r[10]));
    vstore(o2 + 1 * C, vmul(rt.r[8], r[11]));
    vstore(o2 + 2 * C, vmul(rs.r[4], r[10]));
    vstore(o2 + 3 * C, vmul(rt.r[4], r[11]));
  }
}

// Per-edge data of one side of the gather backward (receiver side: so = 1, sender: so = 0).
template <int CPL>
struct SideEdge {
  float w[34];
  Vec<CPL> g[9];   // this side's g_X slots: m0 a/b/c, m1 a/b/c/d, m2 a/b
  Vec<CPL> r[6];   // this side's radial blocks so, 2+so, ..., 10+so
};

template <int CPL>
__device__ __forceinline__ void side_load(const float* __restrict__ gX0, const float* __restrict__ gX1,
                                          const float* __restrict__ gX2, const float* __restrict__ wig,
                                          const float* __restrict__ rad, int64_t e, int so, int c, SideEdge<CPL>& d) {
  constexpr int C = 64 * CPL;
#pragma unroll
  for (int q = 0; q < 34; ++q) d.w[q] = wig[e * 34 + q];
  const float* g0 = gX0 + e * 6 * C + so * C + c;
  const float* g1 = gX1 + e * 8 * C + so * C + c;
  const float* g2 = gX2 + e * 4 * C + so * C + c;
  d.g[0] = vload<CPL>(g0); d.g[1] = vload<CPL>(g0 + 2 * C); d.g[2] = vload<CPL>(g0 + 4 * C);
  d.g[3] = vload<CPL>(g1); d.g[4] = vload<CPL>(g1 + 2 * C); d.g[5] = vload<CPL>(g1 + 4 * C);
  d.g[6] = vload<CPL>(g1 + 6 * C);
  d.g[7] = vload<CPL>(g2); d.g[8] = vload<CPL>(g2 + 2 * C);
  const float* rp = rad + e * 12 * C + so * C + c;
#pragma unroll
  for (int q = 0; q < 6; ++q) d.r[q] = vload<CPL>(rp + 2 * q * C);
}

template <int CPL>
__device__ __forceinline__ void side_apply(const SideEdge<CPL>& d, int64_t e, int so, int c, const Rows9<CPL>& v,
                                           Rows9<CPL>& acc, float* __restrict__ g_rad, float* __restrict__ gw_out,
                                           int lane) {
  constexpr int C = 64 * CPL;
  Rows9<CPL> rv;
  rotate9(d.w, v, rv);
  // this side's radial gradients (blocks so, 2+so, ..., 10+so)
  float* gr = g_rad + e * 12 * C + so * C + c;
  vstore(gr + 0 * C, vmul(d.g[0], rv.r[0]));
  vstore(gr + 2 * C, vmul(d.g[1], rv.r[2]));
  vstore(gr + 4 * C, vmul(d.g[2], rv.r[6]));
  vstore(gr + 6 * C, vadd(vmul(d.g[3], rv.r[3]), vmul(d.g[5], rv.r[1])));
  vstore(gr + 8 * C, vadd(vmul(d.g[4], rv.r[7]), vmul(d.g[6], rv.r[5])));
  vstore(gr + 10 * C, vadd(vmul(d.g[7], rv.r[8]), vmul(d.g[8], rv.r[4])));
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
  add_rotate9_t(d.w, grv, acc);
  // this side's g_wigner: dL/dD1[a][b] = sum_c grv[1+a] v[1+b], dL/dD2[a][b] = sum_c grv[4+a] v[4+b]
  float part[64];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) part[3 * a + b] = vdot(grv.r[1 + a], v.r[1 + b]);
#pragma unroll
  for (int a = 0; a < 5; ++a)
#pragma unroll
    for (int b = 0; b < 5; ++b) part[9 + 5 * a + b] = vdot(grv.r[4 + a], v.r[4 + b]);
#pragma unroll
  for (int q = 34; q < 64; ++q) part[q] = 0.0f;
  const float tot = wave_multi_sum<64>(part, lane);
  if (lane < 34) gw_out[e * 34 + lane] = tot;
}

// One side of one node's gather backward: walk the node's CSR segment in order, two edges
// per iteration so that their loads overlap.
template <int CPL>
__device__ __forceinline__ void gather_bwd_side(const float* __restrict__ gX0, const float* __restrict__ gX1,
                                                const float* __restrict__ gX2, const float* __restrict__ wig,
                                                const float* __restrict__ rad, const int32_t* __restrict__ ptr,
                                                const int32_t* __restrict__ idx, int64_t n, int so,
                                                const Rows9<CPL>& v, Rows9<CPL>& acc, float* __restrict__ g_rad,
                                                float* __restrict__ gw_out, int lane) {
  const int c = lane * CPL;
  const int32_t k0 = ptr[n], k1 = ptr[n + 1];
  int32_t k = k0;
  for (; k + 1 < k1; k += 2) {
    const int64_t ea = idx[k], eb = idx[k + 1];
    SideEdge<CPL> da, db;
    side_load<CPL>(gX0, gX1, gX2, wig, rad, ea, so, c, da);
    side_load<CPL>(gX0, gX1, gX2, wig, rad, eb, so, c, db);
    side_apply<CPL>(da, ea, so, c, v, acc, g_rad, gw_out, lane);
    side_apply<CPL>(db, eb, so, c, v, acc, g_rad, gw_out, lane);
  }
  if (k < k1) {
    const int64_t e = idx[k];
    SideEdge<CPL> d;
    side_load<CPL>(gX0, gX1, gX2, wig, rad, e, so, c, d);
    side_apply<CPL>(d, e, so, c, v, acc, g_rad, gw_out, lane);
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void gather_bwd_kernel(
    const float* __restrict__ gX0, const float* __restrict__ gX1, const float* __restrict__ gX2,
    const float* __restrict__ x, const float* __restrict__ wig, const float* __restrict__ rad,
    const float* __restrict__ csd, const int64_t* __restrict__ batch, const int32_t* __restrict__ rptr,
    const int32_t* __restrict__ ridx, const int32_t* __restrict__ sptr, const int32_t* __restrict__ sidx,
    float* __restrict__ g_x, float* __restrict__ g_wig, float* __restrict__ g_rad, float* __restrict__ ws,
    int64_t N) {
  constexpr int C = 64 * CPL;
  __shared__ __attribute__((aligned(16))) float s_send[2][9 * C];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id_uniform();
  const int node_local = wave >> 1;
  const int side = wave & 1;  // 0: receiver segment, 1: sender segment
  const int64_t n = (int64_t)blockIdx.x * 2 + node_local;
  const int c = lane * CPL;
  Rows9<CPL> acc;
#pragma unroll
  for (int k = 0; k < 9; ++k) acc.r[k] = vzero<CPL>();
  if (n < N) {
    Rows9<CPL> v;
    const float* xn = x + n * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) v.r[k] = vload<CPL>(xn + k * C);
    v.r[0] = vadd(v.r[0], vload<CPL>(csd + batch[n] * C + c));
    if (side == 0) {
      gather_bwd_side<CPL>(gX0, gX1, gX2, wig, rad, rptr, ridx, n, 1, v, acc, g_rad, g_wig, lane);
    } else {
      gather_bwd_side<CPL>(gX0, gX1, gX2, wig, rad, sptr, sidx, n, 0, v, acc, g_rad, ws, lane);
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

template <int CPL>
static void launch_gather_fwd(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                              const float* rad, const float* csd, const int64_t* batch, float* X0, float* X1,
                              float* X2, int64_t E, hipStream_t st) {
  hipLaunchKernelGGL(gather_fwd_kernel<CPL>, dim3((unsigned)std::min<int64_t>(cdiv(E, 4), 8192)), dim3(256), 0, st, x, idx_i, idx_j, wigner, rad,
                     csd, batch, X0, X1, X2, E);
}

template <int CPL>
static void launch_gather_bwd(const float* gX0, const float* gX1, const float* gX2, const float* x,
                              const float* wigner, const float* rad, const float* csd, const int64_t* batch,
                              const int32_t* rptr, const int32_t* ridx, const int32_t* sptr, const int32_t* sidx,
                              float* g_x, float* g_wig, float* g_rad, float* ws, int64_t N, hipStream_t st) {
  hipLaunchKernelGGL(gather_bwd_kernel<CPL>, dim3(cdiv(N, 2)), dim3(256), 0, st, gX0, gX1, gX2, x, wigner, rad, csd,
                     batch, rptr, ridx, sptr, sidx, g_x, g_wig, g_rad, ws, N);
}

}  // namespace fu

using namespace fu;

static int check_c(int32_t C, const char* who) {
  if (C != 64 && C != 128 && C != 256)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d unsupported (64, 128 or 256)", who, C);
  return FU_OK;
}

extern "C" int fu_gather_fwd(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                             const float* rad, const float* csd_emb, const int64_t* batch, float* X_m0, float* X_m1,
                             float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C, void* stream) {
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_fwd: bad shape");
  int st = check_c(C, "fu_gather_fwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!x || !idx_i || !idx_j || !wigner || !rad || !csd_emb || !batch || !X_m0 || !X_m1 || !X_m2)
    return set_error(FU_ERR_NULL, "fu_gather_fwd: NULL argument");
  const void* al[] = {x, rad, csd_emb, X_m0, X_m1, X_m2};
  for (const void* p : al)
    if (!aligned16(p)) return set_error(FU_ERR_ALIGN, "fu_gather_fwd: feature arrays must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  if (C == 64) launch_gather_fwd<1>(x, idx_i, idx_j, wigner, rad, csd_emb, batch, X_m0, X_m1, X_m2, E, s);
  else if (C == 128) launch_gather_fwd<2>(x, idx_i, idx_j, wigner, rad, csd_emb, batch, X_m0, X_m1, X_m2, E, s);
  else launch_gather_fwd<4>(x, idx_i, idx_j, wigner, rad, csd_emb, batch, X_m0, X_m1, X_m2, E, s);
  return check_launch("fu_gather_fwd");
}

extern "C" int fu_gather_bwd(const float* g_X_m0, const float* g_X_m1, const float* g_X_m2, const float* x,
                             const int64_t* idx_i, const int64_t* idx_j, const float* wigner, const float* rad,
                             const float* csd_emb, const int64_t* batch, const int32_t* recv_ptr,
                             const int32_t* recv_idx, const int32_t* send_ptr, const int32_t* send_idx, float* g_x,
                             float* g_wigner, float* g_rad, float* g_wig_ws, int64_t E, int64_t N, int64_t S,
                             int32_t C, void* stream) {
  (void)idx_i;
  (void)idx_j;
  if (E < 0 || N < 0 || S < 1) return set_error(FU_ERR_SHAPE, "fu_gather_bwd: bad shape");
  int st = check_c(C, "fu_gather_bwd");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!x || !csd_emb || !batch || !recv_ptr || !send_ptr || !g_x)
    return set_error(FU_ERR_NULL, "fu_gather_bwd: NULL argument");
  if (E > 0 && (!g_X_m0 || !g_X_m1 || !g_X_m2 || !wigner || !rad || !recv_idx || !send_idx || !g_wigner || !g_rad ||
                !g_wig_ws))
    return set_error(FU_ERR_NULL, "fu_gather_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  if (C == 64)
    launch_gather_bwd<1>(g_X_m0, g_X_m1, g_X_m2, x, wigner, rad, csd_emb, batch, recv_ptr, recv_idx, send_ptr,
                         send_idx, g_x, g_wigner, g_rad, g_wig_ws, N, s);
  else if (C == 128)
    launch_gather_bwd<2>(g_X_m0, g_X_m1, g_X_m2, x, wigner, rad, csd_emb, batch, recv_ptr, recv_idx, send_ptr,
                         send_idx, g_x, g_wigner, g_rad, g_wig_ws, N, s);
  else
    launch_gather_bwd<4>(g_X_m0, g_X_m1, g_X_m2, x, wigner, rad, csd_emb, batch, recv_ptr, recv_idx, send_ptr,
                         send_idx, g_x, g_wigner, g_rad, g_wig_ws, N, s);
  st = check_launch("fu_gather_bwd");
  if (st != FU_OK || E == 0) return st;
  const int64_t tot = E * 34;
  hipLaunchKernelGGL(add_inplace_kernel, dim3((unsigned)std::min<int64_t>(cdiv(tot, 256), 65536)), dim3(256), 0, s,
                     g_wigner, g_wig_ws, tot);
  return check_launch("fu_gather_bwd(add)");
}
