// Inverse rotation + envelope + deterministic FP64 CSR segment sum onto receivers
// (ops/scatter.py:45-140), the edge-degree embedding scatter (ops/scatter.py:360-423) and
// both backward passes (ops/scatter.py:146-292, 426-481).
//
// Forward kernels: one wave64 per receiver node, lanes across channels; the node's CSR
// segment is walked in order and every edge message (computed in fp32 exactly as the
// reference forms it) is accumulated into fp64 registers, then rounded once to fp32.
// Backward kernels: one wave64 per edge, contiguous XCD-aware edge range per workgroup
// (block_edge_range); the per-edge channel reductions for g_wigner and g_env use one
// multi-value wave reduction.
#include "fu_vec.h"

namespace fu {

__device__ __forceinline__ int wave_id_u() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Rotated-frame values zr[0..8] of one edge from the three Zout m-blocks:
// Z_m0 = [k0, k2, k6], Z_m1 = [k3, k7, k1, k5], Z_m2 = [k8, k4].
// The conv2 outputs are read once by each scatter pass, so they carry the nontemporal hint
// (scatter forward 231 -> 215 us at bcc Fe).
template <int CPL>
__device__ __forceinline__ void load_zr(const float* Z0, const float* Z1, const float* Z2, int64_t e, int c,
                                        Vec<CPL> (&zr)[9]) {
  constexpr int C = 64 * CPL;
  const float* z0 = Z0 + e * 3 * C + c;
  const float* z1 = Z1 + e * 4 * C + c;
  const float* z2 = Z2 + e * 2 * C + c;
  zr[0] = vload_nt<CPL>(z0);
  zr[2] = vload_nt<CPL>(z0 + C);
  zr[6] = vload_nt<CPL>(z0 + 2 * C);
  zr[3] = vload_nt<CPL>(z1);
  zr[7] = vload_nt<CPL>(z1 + C);
  zr[1] = vload_nt<CPL>(z1 + 2 * C);
  zr[5] = vload_nt<CPL>(z1 + 3 * C);
  zr[8] = vload_nt<CPL>(z2);
  zr[4] = vload_nt<CPL>(z2 + C);
}

template <int CPL>
__global__ __launch_bounds__(256) void scatter_fwd_kernel(const int32_t* __restrict__ rptr,
                                                          const int32_t* __restrict__ col,
                                                          const float* __restrict__ Z0, const float* __restrict__ Z1,
                                                          const float* __restrict__ Z2, const float* __restrict__ wig,
                                                          const float* __restrict__ env,
                                                          const float* __restrict__ x_res, float* __restrict__ x_out,
                                                          int64_t N) {
  constexpr int C = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_u();
  if (n >= N) return;
  double acc[9][CPL];
  const float* xr = x_res + n * 9 * C + c;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    const Vec<CPL> t = vload<CPL>(xr + k * C);
#pragma unroll
    for (int q = 0; q < CPL; ++q) acc[k][q] = (double)t[q];
  }
  const int32_t k0 = rptr[n], k1 = rptr[n + 1];
  // one edge's message env * D^T zr, accumulated into the fp64 registers
  auto accumulate = [&](const float* w, float en, const Vec<CPL>(&zr)[9]) {
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      acc[0][q] += (double)(zr[0][q] * en);
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const float m = w[3 + b] * zr[2][q] + w[0 + b] * zr[1][q] + w[6 + b] * zr[3][q];
        acc[1 + b][q] += (double)(m * en);
      }
#pragma unroll
      for (int b = 0; b < 5; ++b) {
        const float m = w[19 + b] * zr[6][q] + w[14 + b] * zr[5][q] + w[24 + b] * zr[7][q] + w[9 + b] * zr[4][q] +
                        w[29 + b] * zr[8][q];
        acc[4 + b][q] += (double)(m * en);
      }
    }
  };
  int32_t k = k0;
  // summed in CSR order; the next edge's loads are issued before the current edge is summed
  // (two register sets, sched_barrier keeping the scheduler from sinking them: 214.6 ->
  // 211.2 us at bcc Fe against two edges loaded together and then summed)
  if (k < k1) {
    float wa[34], wb[34];
    float ena, enb;
    Vec<CPL> za[9], zb[9];
    auto load = [&](int64_t e, float (&w)[34], float& en, Vec<CPL> (&z)[9]) {
#pragma unroll
      for (int q = 0; q < 34; ++q) w[q] = wig[e * 34 + q];
      en = env[e];
      load_zr<CPL>(Z0, Z1, Z2, e, c, z);
    };
    load(col[k], wa, ena, za);
    for (; k + 2 <= k1; k += 2) {
      load(col[k + 1], wb, enb, zb);
      __builtin_amdgcn_sched_barrier(0);
      accumulate(wa, ena, za);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 2 < k1) load(col[k + 2], wa, ena, za);
      __builtin_amdgcn_sched_barrier(0);
      accumulate(wb, enb, zb);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (k < k1) accumulate(wa, ena, za);
  }
  float* xo = x_out + n * 9 * C + c;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    Vec<CPL> t;
#pragma unroll
    for (int q = 0; q < CPL; ++q) t[q] = (float)acc[k][q];
    vstore(xo + k * C, t);
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void scatter_bwd_kernel(const float* __restrict__ g_out,
                                                          const int64_t* __restrict__ idx_j,
                                                          const float* __restrict__ Z0, const float* __restrict__ Z1,
                                                          const float* __restrict__ Z2, const float* __restrict__ wig,
                                                          const float* __restrict__ env, float* __restrict__ gZ0,
                                                          float* __restrict__ gZ1, float* __restrict__ gZ2,
                                                          float* __restrict__ g_wig, float* __restrict__ g_env,
                                                          int64_t E, int32_t acc) {
  constexpr int C = 64 * CPL;
  const bool accw = (acc & 1) != 0, acce = (acc & 2) != 0;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_id_u(); e < e1; e += (blockDim.x >> 6)) {
    const int64_t j = idx_j[e];
    float w[34];
#pragma unroll
    for (int q = 0; q < 34; ++q) w[q] = wig[e * 34 + q];
    const float en = env[e];
    Vec<CPL> g[9], zr[9];
    const float* go = g_out + j * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) g[k] = vload<CPL>(go + k * C);
    load_zr<CPL>(Z0, Z1, Z2, e, c, zr);
    // g_zr = env * D g (rotated-frame gradient of this edge's message)
    Vec<CPL> gz[9];
    gz[0] = vscale(g[0], en);
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int q = 0; q < CPL; ++q)
        gz[1 + a][q] = (g[1][q] * en) * w[3 * a + 0] + (g[2][q] * en) * w[3 * a + 1] + (g[3][q] * en) * w[3 * a + 2];
#pragma unroll
    for (int a = 0; a < 5; ++a)
#pragma unroll
      for (int q = 0; q < CPL; ++q)
        gz[4 + a][q] = (g[4][q] * en) * w[9 + 5 * a + 0] + (g[5][q] * en) * w[9 + 5 * a + 1] +
                       (g[6][q] * en) * w[9 + 5 * a + 2] + (g[7][q] * en) * w[9 + 5 * a + 3] +
                       (g[8][q] * en) * w[9 + 5 * a + 4];
    float* o0 = gZ0 + e * 3 * C + c;
    float* o1 = gZ1 + e * 4 * C + c;
    float* o2 = gZ2 + e * 2 * C + c;
    vstore_nt(o0, gz[0]);
    vstore_nt(o0 + C, gz[2]);
    vstore_nt(o0 + 2 * C, gz[6]);
    vstore_nt(o1, gz[3]);
    vstore_nt(o1 + C, gz[7]);
    vstore_nt(o1 + 2 * C, gz[1]);
    vstore_nt(o1 + 3 * C, gz[5]);
    vstore_nt(o2, gz[8]);
    vstore_nt(o2 + C, gz[4]);
    // channel reductions: dL/dD1[a][b] = env sum_c zr[1+a] g[1+b], dL/dD2 likewise, and
    // dL/denv = sum_c sum_k g[k] (D^T zr)[k]
    float part[64];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) part[3 * a + b] = vdot(zr[1 + a], g[1 + b]);
#pragma unroll
    for (int a = 0; a < 5; ++a)
#pragma unroll
      for (int b = 0; b < 5; ++b) part[9 + 5 * a + b] = vdot(zr[4 + a], g[4 + b]);
    float ge = vdot(g[0], zr[0]);
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
#pragma unroll
      for (int b = 0; b < 3; ++b)
        ge += g[1 + b][q] * (w[3 + b] * zr[2][q] + w[0 + b] * zr[1][q] + w[6 + b] * zr[3][q]);
#pragma unroll
      for (int b = 0; b < 5; ++b)
        ge += g[4 + b][q] * (w[19 + b] * zr[6][q] + w[14 + b] * zr[5][q] + w[24 + b] * zr[7][q] +
                             w[9 + b] * zr[4][q] + w[29 + b] * zr[8][q]);
    }
    part[34] = ge;
#pragma unroll
    for (int q = 35; q < 64; ++q) part[q] = 0.0f;
    const float tot = wave_multi_sum<64>(part, lane);
    if (lane < 34) g_wig[e * 34 + lane] = accw ? g_wig[e * 34 + lane] + tot * en : tot * en;
    if (lane == 34) g_env[e] = acce ? g_env[e] + tot : tot;
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void init_scatter_fwd_kernel(
    const int32_t* __restrict__ rptr, const int32_t* __restrict__ col, const float* __restrict__ rad,
    const float* __restrict__ wig, const float* __restrict__ env, const int64_t* __restrict__ Z,
    const int64_t* __restrict__ batch, const float* __restrict__ W_sphere, const float* __restrict__ csd,
    float* __restrict__ x_out, int64_t N) {
  constexpr int C = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_u();
  if (n >= N) return;
  double acc[9][CPL], base[CPL];
  {
    const Vec<CPL> ws = vload<CPL>(W_sphere + Z[n] * C + c);
    const Vec<CPL> cs = vload<CPL>(csd + batch[n] * C + c);
#pragma unroll
    for (int q = 0; q < CPL; ++q) base[q] = (double)(ws[q] + cs[q]);
#pragma unroll
    for (int k = 0; k < 9; ++k)
#pragma unroll
      for (int q = 0; q < CPL; ++q) acc[k][q] = 0.0;
  }
  // The receiver's edges in CSR order; the next edge's loads are issued before the current
  // edge is accumulated (two register sets, sched_barrier keeping the scheduler from sinking
  // them), since one edge's arithmetic is short next to its load latency.
  struct EdgeData {
    float en, w1[3], w2[5];
    Vec<CPL> r[3];
  };
  auto load = [&](int32_t k, EdgeData& d) {
    const int64_t e = col[k];
    d.en = env[e];
#pragma unroll
    for (int b = 0; b < 3; ++b) d.w1[b] = wig[e * 34 + 3 + b];   // L=1 row 1
#pragma unroll
    for (int b = 0; b < 5; ++b) d.w2[b] = wig[e * 34 + 19 + b];  // L=2 row 2
    const float* rp = rad + e * 3 * C + c;
#pragma unroll
    for (int t = 0; t < 3; ++t) d.r[t] = vload_nt<CPL>(rp + t * C);
  };
  // messages summed in fp64 and divided by the rescale factor 5 once per node (the reference
  // divides each message, ops/scatter.py:409-411; same value to fp32 rounding)
  auto add = [&](const EdgeData& d) {
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      acc[0][q] += (double)(d.r[0][q] * d.en);
#pragma unroll
      for (int b = 0; b < 3; ++b) acc[1 + b][q] += (double)(d.r[1][q] * d.w1[b] * d.en);
#pragma unroll
      for (int b = 0; b < 5; ++b) acc[4 + b][q] += (double)(d.r[2][q] * d.w2[b] * d.en);
    }
  };
  const int32_t k0 = rptr[n], k1 = rptr[n + 1];
  if (k0 < k1) {
    EdgeData d0, d1;
    load(k0, d0);
    int32_t k = k0;
    for (; k + 2 <= k1; k += 2) {
      load(k + 1, d1);
      __builtin_amdgcn_sched_barrier(0);
      add(d0);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 2 < k1) load(k + 2, d0);
      __builtin_amdgcn_sched_barrier(0);
      add(d1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (k < k1) add(d0);
  }
  float* xo = x_out + n * 9 * C + c;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    Vec<CPL> t;
#pragma unroll
    for (int q = 0; q < CPL; ++q) t[q] = (float)(k == 0 ? base[q] + acc[0][q] / 5.0 : acc[k][q] / 5.0);
    vstore(xo + k * C, t);
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void init_scatter_bwd_kernel(const float* __restrict__ g_out,
                                                               const int64_t* __restrict__ idx_j,
                                                               const float* __restrict__ rad,
                                                               const float* __restrict__ wig,
                                                               const float* __restrict__ env, float* __restrict__ g_rad,
                                                               float* __restrict__ g_wig, float* __restrict__ g_env,
                                                               int64_t E, int32_t acc) {
  constexpr int C = 64 * CPL;
  const bool accw = (acc & 1) != 0, acce = (acc & 2) != 0;
  const int lane = threadIdx.x & 63;
  const int c = lane * CPL;
  int64_t e0, e1;
  block_edge_range(E, e0, e1);
  for (int64_t e = e0 + wave_id_u(); e < e1; e += (blockDim.x >> 6)) {
    const int64_t j = idx_j[e];
    const float en = env[e];
    float w1[3], w2[5];
#pragma unroll
    for (int b = 0; b < 3; ++b) w1[b] = wig[e * 34 + 3 + b];
#pragma unroll
    for (int b = 0; b < 5; ++b) w2[b] = wig[e * 34 + 19 + b];
    Vec<CPL> g[9];
    const float* go = g_out + j * 9 * C + c;
#pragma unroll
    for (int k = 0; k < 9; ++k) g[k] = vscale(vload<CPL>(go + k * C), 1.0f / 5.0f);
    const float* rp = rad + e * 3 * C + c;
    const Vec<CPL> r0 = vload_nt<CPL>(rp), r1 = vload_nt<CPL>(rp + C), r2 = vload_nt<CPL>(rp + 2 * C);
    Vec<CPL> p1, p2;  // projections of g onto the L=1 row 1 and L=2 row 2
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      p1[q] = g[1][q] * w1[0] + g[2][q] * w1[1] + g[3][q] * w1[2];
      p2[q] = g[4][q] * w2[0] + g[5][q] * w2[1] + g[6][q] * w2[2] + g[7][q] * w2[3] + g[8][q] * w2[4];
    }
    float* gr = g_rad + e * 3 * C + c;
    vstore_nt(gr, vscale(g[0], en));
    vstore_nt(gr + C, vscale(p1, en));
    vstore_nt(gr + 2 * C, vscale(p2, en));
    float part[16];
#pragma unroll
    for (int b = 0; b < 3; ++b) part[b] = vdot(g[1 + b], r1);
#pragma unroll
    for (int b = 0; b < 5; ++b) part[3 + b] = vdot(g[4 + b], r2);
    part[8] = vdot(g[0], r0) + vdot(p1, r1) + vdot(p2, r2);
#pragma unroll
    for (int q = 9; q < 16; ++q) part[q] = 0.0f;
    const float tot = wave_multi_sum<16>(part, lane);
    // g_wigner row: only L1 row 1 (3..5) and L2 row 2 (19..23) are read by the forward
    // lane l holds the total of value l mod 16; gather the 8 wigner totals to lanes 3..5
    // and 19..23 with every lane active in the shuffles
    const bool in1 = lane >= 3 && lane < 6, in2 = lane >= 19 && lane < 24;
    const int src = in1 ? lane - 3 : (in2 ? lane - 16 : 0);
    const float sh = __shfl(tot, src, 64);
    const float outv = (in1 || in2) ? sh : 0.0f;
    const float ge = __shfl(tot, 8, 64);
    if (lane < 34) g_wig[e * 34 + lane] = accw ? g_wig[e * 34 + lane] + outv * en : outv * en;
    if (lane == 0) g_env[e] = acce ? g_env[e] + ge : ge;
  }
}

template <int CPL>
static void launch_scatter_fwd(const int32_t* rptr, const int32_t* col, const float* Z0, const float* Z1,
                               const float* Z2, const float* wig, const float* env, const float* x_res, float* x_out,
                               int64_t N, hipStream_t st) {
  hipLaunchKernelGGL(scatter_fwd_kernel<CPL>, dim3(cdiv(N, 4)), dim3(256), 0, st, rptr, col, Z0, Z1, Z2, wig, env,
                     x_res, x_out, N);
}

template <int CPL>
static void launch_scatter_bwd(const float* g_out, const int64_t* idx_j, const float* Z0, const float* Z1,
                               const float* Z2, const float* wig, const float* env, float* gZ0, float* gZ1, float* gZ2,
                               float* g_wig, float* g_env, int64_t E, int32_t acc, hipStream_t st) {
  hipLaunchKernelGGL(scatter_bwd_kernel<CPL>, dim3(edge_grid(E)), dim3(256), 0, st, g_out, idx_j, Z0, Z1, Z2, wig,
                     env, gZ0, gZ1, gZ2, g_wig, g_env, E, acc);
}

}  // namespace fu

using namespace fu;

static int check_c_s(int32_t C, const char* who) {
  if (C != 64 && C != 128 && C != 256)
    return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d unsupported (64, 128 or 256)", who, C);
  return FU_OK;
}

extern "C" int fu_scatter_fwd(const int32_t* row_ptr, const int32_t* col_idx, const float* Z_m0, const float* Z_m1,
                              const float* Z_m2, const float* wigner, const float* env, const float* x_res,
                              float* x_out, int64_t N, int64_t E, int32_t C, void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_scatter_fwd: bad shape");
  int st = check_c_s(C, "fu_scatter_fwd");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!row_ptr || !x_res || !x_out || (E > 0 && (!col_idx || !Z_m0 || !Z_m1 || !Z_m2 || !wigner || !env)))
    return set_error(FU_ERR_NULL, "fu_scatter_fwd: NULL argument");
  hipStream_t s = as_stream(stream);
  if (C == 64) launch_scatter_fwd<1>(row_ptr, col_idx, Z_m0, Z_m1, Z_m2, wigner, env, x_res, x_out, N, s);
  else if (C == 128) launch_scatter_fwd<2>(row_ptr, col_idx, Z_m0, Z_m1, Z_m2, wigner, env, x_res, x_out, N, s);
  else launch_scatter_fwd<4>(row_ptr, col_idx, Z_m0, Z_m1, Z_m2, wigner, env, x_res, x_out, N, s);
  return check_launch("fu_scatter_fwd");
}

extern "C" int fu_scatter_bwd(const float* g_out, const int64_t* idx_j, const float* Z_m0, const float* Z_m1,
                              const float* Z_m2, const float* wigner, const float* env, float* g_Z_m0, float* g_Z_m1,
                              float* g_Z_m2, float* g_wigner, float* g_env, int64_t E, int64_t N, int32_t C,
                              int32_t accumulate, void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_scatter_bwd: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_scatter_bwd: accumulate=%d (0..3)", accumulate);
  int st = check_c_s(C, "fu_scatter_bwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!g_out || !idx_j || !Z_m0 || !Z_m1 || !Z_m2 || !wigner || !env || !g_Z_m0 || !g_Z_m1 || !g_Z_m2 || !g_wigner ||
      !g_env)
    return set_error(FU_ERR_NULL, "fu_scatter_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  if (C == 64)
    launch_scatter_bwd<1>(g_out, idx_j, Z_m0, Z_m1, Z_m2, wigner, env, g_Z_m0, g_Z_m1, g_Z_m2, g_wigner, g_env, E,
                          accumulate, s);
  else if (C == 128)
    launch_scatter_bwd<2>(g_out, idx_j, Z_m0, Z_m1, Z_m2, wigner, env, g_Z_m0, g_Z_m1, g_Z_m2, g_wigner, g_env, E,
                          accumulate, s);
  else
    launch_scatter_bwd<4>(g_out, idx_j, Z_m0, Z_m1, Z_m2, wigner, env, g_Z_m0, g_Z_m1, g_Z_m2, g_wigner, g_env, E,
                          accumulate, s);
  return check_launch("fu_scatter_bwd");
}

extern "C" int fu_init_scatter_fwd(const int32_t* row_ptr, const int32_t* col_idx, const float* rad,
                                   const float* wigner, const float* env, const int64_t* Z, const int64_t* batch,
                                   const float* W_sphere, const float* csd_emb, float* x_out, int64_t N, int64_t E,
                                   int64_t num_z, int64_t S, int32_t C, void* stream) {
  if (N < 0 || E < 0 || num_z < 1 || S < 1) return set_error(FU_ERR_SHAPE, "fu_init_scatter_fwd: bad shape");
  int st = check_c_s(C, "fu_init_scatter_fwd");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!row_ptr || !Z || !batch || !W_sphere || !csd_emb || !x_out || (E > 0 && (!col_idx || !rad || !wigner || !env)))
    return set_error(FU_ERR_NULL, "fu_init_scatter_fwd: NULL argument");
  hipStream_t s = as_stream(stream);
  const dim3 grid(cdiv(N, 4));
  if (C == 64)
    hipLaunchKernelGGL(init_scatter_fwd_kernel<1>, grid, dim3(256), 0, s, row_ptr, col_idx, rad, wigner, env, Z, batch,
                       W_sphere, csd_emb, x_out, N);
  else if (C == 128)
    hipLaunchKernelGGL(init_scatter_fwd_kernel<2>, grid, dim3(256), 0, s, row_ptr, col_idx, rad, wigner, env, Z, batch,
                       W_sphere, csd_emb, x_out, N);
  else
    hipLaunchKernelGGL(init_scatter_fwd_kernel<4>, grid, dim3(256), 0, s, row_ptr, col_idx, rad, wigner, env, Z, batch,
                       W_sphere, csd_emb, x_out, N);
  return check_launch("fu_init_scatter_fwd");
}

extern "C" int fu_init_scatter_bwd(const float* g_out, const int64_t* idx_j, const float* rad, const float* wigner,
                                   const float* env, float* g_rad, float* g_wigner, float* g_env, int64_t E, int64_t N,
                                   int32_t C, int32_t accumulate, void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_init_scatter_bwd: bad shape");
  if (accumulate < 0 || accumulate > 3)
    return set_error(FU_ERR_UNSUPPORTED, "fu_init_scatter_bwd: accumulate=%d (0..3)", accumulate);
  int st = check_c_s(C, "fu_init_scatter_bwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  if (!g_out || !idx_j || !rad || !wigner || !env || !g_rad || !g_wigner || !g_env)
    return set_error(FU_ERR_NULL, "fu_init_scatter_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  const dim3 grid(edge_grid(E));
  if (C == 64)
    hipLaunchKernelGGL(init_scatter_bwd_kernel<1>, grid, dim3(256), 0, s, g_out, idx_j, rad, wigner, env, g_rad,
                       g_wigner, g_env, E, accumulate);
  else if (C == 128)
    hipLaunchKernelGGL(init_scatter_bwd_kernel<2>, grid, dim3(256), 0, s, g_out, idx_j, rad, wigner, env, g_rad,
                       g_wigner, g_env, E, accumulate);
  else
    hipLaunchKernelGGL(init_scatter_bwd_kernel<4>, grid, dim3(256), 0, s, g_out, idx_j, rad, wigner, env, g_rad,
                       g_wigner, g_env, E, accumulate);
  return check_launch("fu_init_scatter_bwd");
}
