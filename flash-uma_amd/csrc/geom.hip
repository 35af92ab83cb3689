// Per-edge geometry: edge vector, envelope, Gaussian basis, element embeddings and the
// quaternion edge frame with its L=1 and L=2 Wigner blocks (ops/geom.py:36-214), and the
// vector-Jacobian product back to the edge vector (ops/geom.py:220-493) with a
// deterministic CSR reduction onto atoms in place of the reference's atomics.
//
// Frame: the reference's two-chart quaternion blend (ops/geom.py:106-131) gives q; the L=1
// block is the rotation matrix R(q) (ops/geom.py:137-139).  The L=2 block is evaluated as
// the l=2 representation induced by R on symmetric traceless tensors,
//     D2[a][b] = <B_a, R B_b R^T>,
// with the orthonormal basis B = {xz, xy, (2y^2-x^2-z^2)/sqrt3, yz, z^2-x^2} (each /sqrt2 in
// the off-diagonal/diagonal sense).  This equals the reference's quartic polynomials
// (ops/geom.py:154-178) identically in q and needs only products of R entries; its VJP is
// dL/dR = 2 sum_ab gD2[a][b] B_a R B_b.
//
// Layout: one thread per edge for the scalar geometry; the (E, 34) Wigner rows, env and the
// x_edge_raw rows of a 128-edge block are staged through LDS and written cooperatively so
// every global store is coalesced.
#include "fu_common.h"

namespace fu {

constexpr int GEOM_BLOCK = 128;
constexpr float kEps = 1e-7f;
constexpr float kInvSqrt2 = 0.70710678118654752f;
constexpr float kInvSqrt6 = 0.40824829046386302f;
constexpr float kSqrt2 = 1.41421356237309505f;

struct Frame {
  // quaternion pipeline intermediates kept for the backward pass
  float ex, ey, ez;
  float n1, q1w, q1x, q1z;   // chart 1 (unflipped, normalised)
  float n2, q2w, q2x, q2y;   // chart 2 (normalised)
  float t, num, den, s;
  bool flip;
  float ne, qw, qx, qy, qz;  // blended, normalised quaternion
};

__device__ __forceinline__ void frame_from_dir(float ex, float ey, float ez, Frame& f) {
  f.ex = ex; f.ey = ey; f.ez = ez;
  f.n1 = sqrtf((1.0f + ey) * (1.0f + ey) + ez * ez + ex * ex + kEps);
  f.q1w = (1.0f + ey) / f.n1; f.q1x = -ez / f.n1; f.q1z = ex / f.n1;
  f.n2 = sqrtf(ez * ez + (1.0f - ey) * (1.0f - ey) + ex * ex + kEps);
  f.q2w = -ez / f.n2; f.q2x = (1.0f - ey) / f.n2; f.q2y = ex / f.n2;
  f.t = fminf(fmaxf((ey + 0.9f) / 1.8f, 0.0f), 1.0f);
  f.num = 2.0f * f.t - 1.0f;
  f.den = fmaxf(f.t * (1.0f - f.t), kEps);
  float s = sigmoidf_(f.num / f.den);
  if (f.t < kEps) s = 0.0f;
  if (f.t > 1.0f - kEps) s = 1.0f;
  f.s = s;
  f.flip = (f.q1w * f.q2w + f.q1x * f.q2x) < 0.0f;
  const float sg = f.flip ? -1.0f : 1.0f;
  const float uw = (1.0f - s) * f.q2w + s * (sg * f.q1w);
  const float ux = (1.0f - s) * f.q2x + s * (sg * f.q1x);
  const float uy = (1.0f - s) * f.q2y;
  const float uz = s * (sg * f.q1z);
  f.ne = sqrtf(uw * uw + ux * ux + uy * uy + uz * uz + kEps);
  f.qw = uw / f.ne; f.qx = ux / f.ne; f.qy = uy / f.ne; f.qz = uz / f.ne;
}

__device__ __forceinline__ void rot_from_quat(float w, float x, float y, float z, float R[3][3]) {
  R[0][0] = 1.0f - 2.0f * (y * y + z * z); R[0][1] = 2.0f * (x * y - w * z); R[0][2] = 2.0f * (x * z + w * y);
  R[1][0] = 2.0f * (x * y + w * z); R[1][1] = 1.0f - 2.0f * (x * x + z * z); R[1][2] = 2.0f * (y * z - w * x);
  R[2][0] = 2.0f * (x * z - w * y); R[2][1] = 2.0f * (y * z + w * x); R[2][2] = 1.0f - 2.0f * (x * x + y * y);
}

// M = R B_b R^T for basis element b, returned as its 6 independent entries
// (xx, yy, zz, xy, xz, yz).
__device__ __forceinline__ void conj_basis(const float R[3][3], int b, float m[6]) {
  // r_i^T B_b r_j for (i, j) in {(0,0),(1,1),(2,2),(0,1),(0,2),(1,2)}
  const int I[6] = {0, 1, 2, 0, 0, 1};
  const int J[6] = {0, 1, 2, 1, 2, 2};
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const float* ri = R[I[k]];
    const float* rj = R[J[k]];
    float v;
    switch (b) {
      case 0: v = (ri[0] * rj[2] + ri[2] * rj[0]) * kInvSqrt2; break;
      case 1: v = (ri[0] * rj[1] + ri[1] * rj[0]) * kInvSqrt2; break;
      case 2: v = (2.0f * ri[1] * rj[1] - ri[0] * rj[0] - ri[2] * rj[2]) * kInvSqrt6; break;
      case 3: v = (ri[1] * rj[2] + ri[2] * rj[1]) * kInvSqrt2; break;
      default: v = (ri[2] * rj[2] - ri[0] * rj[0]) * kInvSqrt2; break;
    }
    m[k] = v;
  }
}

// <B_a, M> for a symmetric M given by its 6 entries.
__device__ __forceinline__ float basis_dot(int a, const float m[6]) {
  switch (a) {
    case 0: return kSqrt2 * m[4];
    case 1: return kSqrt2 * m[3];
    case 2: return (2.0f * m[1] - m[0] - m[2]) * kInvSqrt6;
    case 3: return kSqrt2 * m[5];
    default: return (m[2] - m[0]) * kInvSqrt2;
  }
}

__device__ __forceinline__ void wigner_from_rot(const float R[3][3], float w[34]) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) w[3 * i + j] = R[i][j];
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    float m[6];
    conj_basis(R, b, m);
#pragma unroll
    for (int a = 0; a < 5; ++a) w[9 + 5 * a + b] = basis_dot(a, m);
  }
}

// Symmetric 3x3 basis matrix B_a as a dense array.
__device__ __forceinline__ void basis_dense(int a, float B[3][3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) B[i][j] = 0.0f;
  switch (a) {
    case 0: B[0][2] = B[2][0] = kInvSqrt2; break;
    case 1: B[0][1] = B[1][0] = kInvSqrt2; break;
    case 2: B[0][0] = -kInvSqrt6; B[1][1] = 2.0f * kInvSqrt6; B[2][2] = -kInvSqrt6; break;
    case 3: B[1][2] = B[2][1] = kInvSqrt2; break;
    default: B[0][0] = -kInvSqrt2; B[2][2] = kInvSqrt2; break;
  }
}

__device__ __forceinline__ float envelope(float dist, float cutoff) {
  const float u = dist / cutoff;
  const float u2 = u * u;
  const float u5 = u2 * u2 * u;
  const float env = 1.0f + u5 * (-21.0f + u * (35.0f - 15.0f * u));
  return u < 1.0f ? env : 0.0f;
}

__global__ __launch_bounds__(GEOM_BLOCK) void geom_fwd_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ Z, const int64_t* __restrict__ idx_i,
    const int64_t* __restrict__ idx_j, const float* __restrict__ shifts,
    const float* __restrict__ W_src, const float* __restrict__ W_tgt,
    const float* __restrict__ offset_g, float* __restrict__ x_edge, int64_t ld_xe,
    float* __restrict__ wig, float* __restrict__ env_out, int64_t E, int32_t B, int32_t C,
    float cutoff, float coeff_g) {
  __shared__ float s_wig[GEOM_BLOCK * 34];
  __shared__ float s_dist[GEOM_BLOCK];
  __shared__ int64_t s_zi[GEOM_BLOCK], s_zj[GEOM_BLOCK];

  const int64_t e0 = (int64_t)blockIdx.x * GEOM_BLOCK;
  const int nloc = (int)min<int64_t>(GEOM_BLOCK, E - e0);
  const int t = threadIdx.x;

  if (t < nloc) {
    const int64_t e = e0 + t;
    const int64_t i = idx_i[e], j = idx_j[e];
    const float dx = pos[3 * i + 0] - pos[3 * j + 0] + shifts[3 * e + 0];
    const float dy = pos[3 * i + 1] - pos[3 * j + 1] + shifts[3 * e + 1];
    const float dz = pos[3 * i + 2] - pos[3 * j + 2] + shifts[3 * e + 2];
    const float dist = sqrtf(dx * dx + dy * dy + dz * dz);
    const float dsafe = fmaxf(dist, kEps);
    env_out[e] = envelope(dist, cutoff);
    s_dist[t] = dist;
    if (W_src != nullptr) {
      s_zi[t] = Z[i];
      s_zj[t] = Z[j];
    }
    Frame f;
    frame_from_dir(dx / dsafe, dy / dsafe, dz / dsafe, f);
    float R[3][3];
    rot_from_quat(f.qw, f.qx, f.qy, f.qz, R);
    float w[34];
    wigner_from_rot(R, w);
#pragma unroll
    for (int k = 0; k < 34; ++k) s_wig[t * 34 + k] = w[k];
  }
  __syncthreads();

  // coalesced copy of the block's contiguous Wigner rows
  float* wdst = wig + e0 * 34;
  for (int k = t; k < nloc * 34; k += GEOM_BLOCK) wdst[k] = s_wig[k];

  // x_edge_raw rows: [Gaussians (B) | W_src[Z_i] (C) | W_tgt[Z_j] (C)]
  const int width = (W_src != nullptr) ? B + 2 * C : B;
  const int64_t total = (int64_t)nloc * width;
  for (int64_t k = t; k < total; k += GEOM_BLOCK) {
    const int el = (int)(k / width);
    const int col = (int)(k - (int64_t)el * width);
    float v;
    if (col < B) {
      const float diff = s_dist[el] - offset_g[col];
      v = expf(coeff_g * diff * diff);
    } else if (col < B + C) {
      v = W_src[s_zi[el] * C + (col - B)];
    } else {
      v = W_tgt[s_zj[el] * C + (col - B - C)];
    }
    x_edge[(e0 + el) * ld_xe + col] = v;
  }
}

__global__ __launch_bounds__(GEOM_BLOCK) void geom_bwd_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ idx_i,
    const int64_t* __restrict__ idx_j, const float* __restrict__ shifts,
    const float* __restrict__ offset_g, const float* __restrict__ g_xe, int64_t ld_gxe,
    const float* __restrict__ g_wig, const float* __restrict__ g_env, float* __restrict__ g_d,
    int64_t E, int32_t B, float cutoff, float coeff_g) {
  extern __shared__ float s_dyn[];
  float* s_gw = s_dyn;                          // [GEOM_BLOCK][34]
  const int64_t e0 = (int64_t)blockIdx.x * GEOM_BLOCK;
  const int nloc = (int)min<int64_t>(GEOM_BLOCK, E - e0);
  const int t = threadIdx.x;

  // cooperative, coalesced staging of the block's g_wigner rows.  The Gaussian gradients are
  // read by each thread from its own row below: a wave's 64 rows are 64 whole cache-line pairs,
  // and staging them too (33 KB per block) limited the kernel to 3 blocks per CU (167-172
  // against 99-101 us at bcc Fe).
  if (g_wig != nullptr) {
    const float* src = g_wig + e0 * 34;
    for (int k = t; k < nloc * 34; k += GEOM_BLOCK) s_gw[k] = src[k];
  }
  __syncthreads();
  if (t >= nloc) return;

  const int64_t e = e0 + t;
  const int64_t i = idx_i[e], j = idx_j[e];
  const float dx = pos[3 * i + 0] - pos[3 * j + 0] + shifts[3 * e + 0];
  const float dy = pos[3 * i + 1] - pos[3 * j + 1] + shifts[3 * e + 1];
  const float dz = pos[3 * i + 2] - pos[3 * j + 2] + shifts[3 * e + 2];
  const float dist = sqrtf(dx * dx + dy * dy + dz * dz);
  const float dsafe = fmaxf(dist, kEps);
  Frame f;
  frame_from_dir(dx / dsafe, dy / dsafe, dz / dsafe, f);

  float gex = 0.0f, gey = 0.0f, gez = 0.0f;
  if (g_wig != nullptr) {
    const float* gw = s_gw + t * 34;
    float R[3][3];
    rot_from_quat(f.qw, f.qx, f.qy, f.qz, R);
    // dL/dR = g_D1 + 2 sum_a B_a R S_a,  S_a = sum_b gD2[a][b] B_b
    float G[3][3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
      for (int c = 0; c < 3; ++c) G[r][c] = gw[3 * r + c];
#pragma unroll
    for (int a = 0; a < 5; ++a) {
      float S[3][3] = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
#pragma unroll
      for (int b = 0; b < 5; ++b) {
        float Bb[3][3];
        basis_dense(b, Bb);
        const float g = gw[9 + 5 * a + b];
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
          for (int c = 0; c < 3; ++c) S[r][c] += g * Bb[r][c];
      }
      float RS[3][3];
#pragma unroll
      for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) RS[r][c] = R[r][0] * S[0][c] + R[r][1] * S[1][c] + R[r][2] * S[2][c];
      float Ba[3][3];
      basis_dense(a, Ba);
#pragma unroll
      for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c)
          G[r][c] += 2.0f * (Ba[r][0] * RS[0][c] + Ba[r][1] * RS[1][c] + Ba[r][2] * RS[2][c]);
    }
    // dL/dq through R(q) (ops/geom.py:313-316 for the L=1 part)
    const float w = f.qw, x = f.qx, y = f.qy, z = f.qz;
    const float gqw = 2.0f * x * (G[2][1] - G[1][2]) + 2.0f * y * (G[0][2] - G[2][0]) + 2.0f * z * (G[1][0] - G[0][1]);
    const float gqx = 2.0f * w * (G[2][1] - G[1][2]) + 2.0f * y * (G[0][1] + G[1][0]) + 2.0f * z * (G[0][2] + G[2][0]) -
                      4.0f * x * (G[1][1] + G[2][2]);
    const float gqy = 2.0f * w * (G[0][2] - G[2][0]) + 2.0f * x * (G[0][1] + G[1][0]) + 2.0f * z * (G[1][2] + G[2][1]) -
                      4.0f * y * (G[0][0] + G[2][2]);
    const float gqz = 2.0f * w * (G[1][0] - G[0][1]) + 2.0f * x * (G[0][2] + G[2][0]) + 2.0f * y * (G[1][2] + G[2][1]) -
                      4.0f * z * (G[0][0] + G[1][1]);
    // normalisation q = u / |u|_eps (ops/geom.py:415-419)
    const float proj = gqw * w + gqx * x + gqy * y + gqz * z;
    const float guw = (gqw - w * proj) / f.ne, gux = (gqx - x * proj) / f.ne;
    const float guy = (gqy - y * proj) / f.ne, guz = (gqz - z * proj) / f.ne;
    // blend u = (1-s) q2 + s q1f (ops/geom.py:421-428)
    const float sg = f.flip ? -1.0f : 1.0f;
    const float q1wf = sg * f.q1w, q1xf = sg * f.q1x, q1zf = sg * f.q1z;
    const float s = f.s;
    const float g_s = guw * (q1wf - f.q2w) + gux * (q1xf - f.q2x) + guy * (0.0f - f.q2y) + guz * q1zf;
    const float g1w = sg * guw * s, g1x = sg * gux * s, g1z = sg * guz * s;
    const float g2w = guw * (1.0f - s), g2x = gux * (1.0f - s), g2y = guy * (1.0f - s);
    // blend weight s(t) (ops/geom.py:430-437)
    const float ds_darg = s * (1.0f - s);
    const float dt_den = (f.t * (1.0f - f.t) <= kEps) ? 0.0f : 1.0f - 2.0f * f.t;
    const float darg_dt = (2.0f * f.den - f.num * dt_den) / (f.den * f.den);
    const bool valid = (f.t > kEps) && (f.t < 1.0f - kEps);
    const float gey_s = valid ? g_s * ds_darg * darg_dt * (1.0f / 1.8f) : 0.0f;
    // chart 1: (w, x, z) = (1+ey, -ez, ex) / n1 (ops/geom.py:439-442)
    const float p1 = g1w * f.q1w + g1x * f.q1x + g1z * f.q1z;
    const float gv1w = (g1w - f.q1w * p1) / f.n1, gv1x = (g1x - f.q1x * p1) / f.n1;
    const float gv1z = (g1z - f.q1z * p1) / f.n1;
    // chart 2: (w, x, y) = (-ez, 1-ey, ex) / n2 (ops/geom.py:444-447)
    const float p2 = g2w * f.q2w + g2x * f.q2x + g2y * f.q2y;
    const float gv2w = (g2w - f.q2w * p2) / f.n2, gv2x = (g2x - f.q2x * p2) / f.n2;
    const float gv2y = (g2y - f.q2y * p2) / f.n2;
    gex = gv1z + gv2y;
    gey = gv1w - gv2x + gey_s;
    gez = -gv1x - gv2w;
  }

  // radial terms: Gaussians and envelope (ops/geom.py:453-471)
  float g_dist = 0.0f;
  if (g_xe != nullptr) {
    const float* gg = g_xe + e * ld_gxe;
    for (int b = 0; b < B; ++b) {
      const float diff = dist - offset_g[b];
      const float gauss = expf(coeff_g * diff * diff);
      g_dist += gg[b] * (2.0f * coeff_g * diff * gauss);
    }
  }
  if (g_env != nullptr) {
    const float u = dist / cutoff;
    const float u4 = u * u * u * u;
    const float denv = u4 * (-105.0f + u * (210.0f - 105.0f * u));
    if (u < 1.0f) g_dist += g_env[e] * denv / cutoff;
  }
  const float ex = f.ex, ey = f.ey, ez = f.ez;
  const float pe = gex * ex + gey * ey + gez * ez;
  g_d[3 * e + 0] = (gex - ex * pe) / dsafe + g_dist * ex;
  g_d[3 * e + 1] = (gey - ey * pe) / dsafe + g_dist * ey;
  g_d[3 * e + 2] = (gez - ez * pe) / dsafe + g_dist * ez;
}

// g_pos[n] = sum over send(n) of g_d - sum over recv(n) of g_d, fp64.  One wave per node:
// lane t takes the segments' entries t, t + 64, ... in CSR order, then a fixed butterfly sums
// the lanes, so the result is the same on every run.  (One thread per node walked ~60 entries
// serially on 8,192 threads: 38 us at bcc Fe.)
__global__ __launch_bounds__(256) void edge_vec_reduce_kernel(const float* __restrict__ g_d,
                                                              const int32_t* __restrict__ rptr,
                                                              const int32_t* __restrict__ ridx,
                                                              const int32_t* __restrict__ sptr,
                                                              const int32_t* __restrict__ sidx,
                                                              float* __restrict__ g_pos, int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;   // wave-uniform
  double ax = 0.0, ay = 0.0, az = 0.0;
  for (int32_t k = sptr[n] + lane; k < sptr[n + 1]; k += 64) {
    const int64_t e = sidx[k];
    ax += (double)g_d[3 * e + 0];
    ay += (double)g_d[3 * e + 1];
    az += (double)g_d[3 * e + 2];
  }
  for (int32_t k = rptr[n] + lane; k < rptr[n + 1]; k += 64) {
    const int64_t e = ridx[k];
    ax -= (double)g_d[3 * e + 0];
    ay -= (double)g_d[3 * e + 1];
    az -= (double)g_d[3 * e + 2];
  }
  ax = wave_sum_d(ax);
  ay = wave_sum_d(ay);
  az = wave_sum_d(az);
  if (lane == 0) {
    g_pos[3 * n + 0] = (float)ax;
    g_pos[3 * n + 1] = (float)ay;
    g_pos[3 * n + 2] = (float)az;
  }
}

}  // namespace fu

using namespace fu;

extern "C" int fu_geom_fwd(const float* pos, const int64_t* Z, const int64_t* idx_i, const int64_t* idx_j,
                           const float* shifts, const float* W_src, const float* W_tgt, const float* offset_g,
                           float* x_edge_raw, int64_t ld_xe, float* wigner, float* env, int64_t E, int64_t N,
                           int32_t B, int32_t C, float cutoff, float coeff_g, void* stream) {
  if (E < 0 || N < 0 || B <= 0 || C < 0) return set_error(FU_ERR_SHAPE, "fu_geom_fwd: bad shape");
  if ((W_src == nullptr) != (W_tgt == nullptr))
    return set_error(FU_ERR_NULL, "fu_geom_fwd: W_src and W_tgt must both be given or both NULL");
  const int width = W_src ? B + 2 * C : B;
  if (ld_xe < width) return set_error(FU_ERR_SHAPE, "fu_geom_fwd: ld_xe=%lld < row width %d", (long long)ld_xe, width);
  if (!(cutoff > 0.0f)) return set_error(FU_ERR_SHAPE, "fu_geom_fwd: cutoff must be > 0");
  if (E == 0) return FU_OK;
  if (!pos || !idx_i || !idx_j || !shifts || !offset_g || !x_edge_raw || !wigner || !env || (W_src && !Z))
    return set_error(FU_ERR_NULL, "fu_geom_fwd: NULL argument");
  hipLaunchKernelGGL(geom_fwd_kernel, dim3(cdiv(E, GEOM_BLOCK)), dim3(GEOM_BLOCK), 0, as_stream(stream), pos, Z,
                     idx_i, idx_j, shifts, W_src, W_tgt, offset_g, x_edge_raw, ld_xe, wigner, env, E, B, C, cutoff,
                     coeff_g);
  return check_launch("fu_geom_fwd");
}

extern "C" int fu_geom_bwd(const float* pos, const int64_t* idx_i, const int64_t* idx_j, const float* shifts,
                           const float* offset_g, const float* g_x_edge_raw, int64_t ld_gxe, const float* g_wigner,
                           const float* g_env, float* g_d, int64_t E, int64_t N, int32_t B, float cutoff,
                           float coeff_g, void* stream) {
  if (E < 0 || N < 0 || B <= 0 || B > 256) return set_error(FU_ERR_SHAPE, "fu_geom_bwd: bad shape (B must be 1..256)");
  if (g_x_edge_raw && ld_gxe < B) return set_error(FU_ERR_SHAPE, "fu_geom_bwd: ld_gxe < B");
  if (E == 0) return FU_OK;
  if (!pos || !idx_i || !idx_j || !shifts || !offset_g || !g_d) return set_error(FU_ERR_NULL, "fu_geom_bwd: NULL argument");
  const size_t lds = sizeof(float) * GEOM_BLOCK * 34;
  hipLaunchKernelGGL(geom_bwd_kernel, dim3(cdiv(E, GEOM_BLOCK)), dim3(GEOM_BLOCK), lds, as_stream(stream), pos, idx_i,
                     idx_j, shifts, offset_g, g_x_edge_raw, ld_gxe, g_wigner, g_env, g_d, E, B, cutoff, coeff_g);
  return check_launch("fu_geom_bwd");
}

extern "C" int fu_edge_vec_reduce(const float* g_d, const int32_t* recv_ptr, const int32_t* recv_idx,
                                  const int32_t* send_ptr, const int32_t* send_idx, float* g_pos, int64_t N, int64_t E,
                                  void* stream) {
  if (N < 0 || E < 0) return set_error(FU_ERR_SHAPE, "fu_edge_vec_reduce: bad shape");
  if (!recv_ptr || !send_ptr || !g_pos || (E > 0 && (!g_d || !recv_idx || !send_idx)))
    return set_error(FU_ERR_NULL, "fu_edge_vec_reduce: NULL argument");
  if (N == 0) return FU_OK;
  hipLaunchKernelGGL(edge_vec_reduce_kernel, dim3(cdiv(N, 4)), dim3(256), 0, as_stream(stream), g_d, recv_ptr,
                     recv_idx, send_ptr, send_idx, g_pos, N);
  return check_launch("fu_edge_vec_reduce");
}
