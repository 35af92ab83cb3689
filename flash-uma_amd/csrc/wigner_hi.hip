// Wigner blocks of degree 3 and 4 for lmax > 2 (the reference stops at lmax = 2: its 34 scalars
// are the L=1 and L=2 blocks, ops/geom.py:137-178, and wrapper.py:105-118 rejects larger lmax).
//
// The edge frame keeps the orders |m| <= 2 only, so per edge only rows m = -2..2 of D^3 (5 x 7)
// and D^4 (5 x 9) are needed; they are derived from the reference's blocks by the recursion
// D^l = U_l^T (D^(l-1) (x) D^1) U_l with the constant couplings of wigner_tables.h (D^3 in
// full, since D^4 needs every row of it).  One thread per edge; the couplings are sparse and
// every zero term is removed at compile time (loops unrolled over constant tables).
//
// Backward: the vector-Jacobian product through the same recursion, returning the
// contributions to dL/dD^1 and dL/dD^2 (the 34 reference scalars), which the geometry
// backward then carries to the edge vector.
#include "fu_common.h"
#include "wigner_tables.h"

namespace fu {

template <int l>
__device__ __forceinline__ constexpr float coupling(int r, int b) {
  if constexpr (l == 3) return kU3[r][b];
  else return kU4[r][b];
}

// true when column b of U_l has a nonzero entry in row block k (rows 3k .. 3k+2)
template <int l>
__device__ __forceinline__ constexpr bool block_used(int k, int b) {
  return coupling<l>(3 * k, b) != 0.0f || coupling<l>(3 * k + 1, b) != 0.0f || coupling<l>(3 * k + 2, b) != 0.0f;
}

// T[k][j] = sum_p R[j][p] U_l[3k + p][b] for one column b
template <int l>
__device__ __forceinline__ void rec_t(const float (&R)[3][3], int b, float (&T)[2 * l - 1][3]) {
#pragma unroll
  for (int k = 0; k < 2 * l - 1; ++k) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      float t = 0.0f;
#pragma unroll
      for (int p = 0; p < 3; ++p)
        if (coupling<l>(3 * k + p, b) != 0.0f) t += R[j][p] * coupling<l>(3 * k + p, b);
      T[k][j] = t;
    }
  }
}

// out[a][b] = D^l[R0 + a][b] for a < NR
template <int l, int R0, int NR>
__device__ __forceinline__ void rec_fwd(const float (&D)[2 * l - 1][2 * l - 1], const float (&R)[3][3],
                                        float (&out)[NR][2 * l + 1]) {
  constexpr int nl = 2 * l - 1, nh = 2 * l + 1;
#pragma unroll
  for (int b = 0; b < nh; ++b) {
    float T[nl][3];
    rec_t<l>(R, b, T);
#pragma unroll
    for (int a = 0; a < NR; ++a) out[a][b] = 0.0f;
#pragma unroll
    for (int i = 0; i < nl; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        bool needed = false;
#pragma unroll
        for (int a = 0; a < NR; ++a) needed = needed || coupling<l>(3 * i + j, R0 + a) != 0.0f;
        if (!needed) continue;
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < nl; ++k)
          if (block_used<l>(k, b)) m += D[i][k] * T[k][j];
#pragma unroll
        for (int a = 0; a < NR; ++a)
          if (coupling<l>(3 * i + j, R0 + a) != 0.0f) out[a][b] += coupling<l>(3 * i + j, R0 + a) * m;
      }
    }
  }
}

// VJP of rec_fwd: G = dL/dout (NR x nh) -> gD += dL/dD^(l-1), gR += dL/dR
template <int l, int R0, int NR>
__device__ __forceinline__ void rec_bwd(const float (&D)[2 * l - 1][2 * l - 1], const float (&R)[3][3],
                                        const float (&G)[NR][2 * l + 1], float (&gD)[2 * l - 1][2 * l - 1],
                                        float (&gR)[3][3]) {
  constexpr int nl = 2 * l - 1, nh = 2 * l + 1;
#pragma unroll
  for (int b = 0; b < nh; ++b) {
    float T[nl][3], gT[nl][3];
    rec_t<l>(R, b, T);
#pragma unroll
    for (int k = 0; k < nl; ++k)
#pragma unroll
      for (int j = 0; j < 3; ++j) gT[k][j] = 0.0f;
#pragma unroll
    for (int i = 0; i < nl; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        bool needed = false;
#pragma unroll
        for (int a = 0; a < NR; ++a) needed = needed || coupling<l>(3 * i + j, R0 + a) != 0.0f;
        if (!needed) continue;
        float gm = 0.0f;
#pragma unroll
        for (int a = 0; a < NR; ++a)
          if (coupling<l>(3 * i + j, R0 + a) != 0.0f) gm += coupling<l>(3 * i + j, R0 + a) * G[a][b];
#pragma unroll
        for (int k = 0; k < nl; ++k) {
          if (!block_used<l>(k, b)) continue;
          gD[i][k] += gm * T[k][j];
          gT[k][j] += D[i][k] * gm;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < nl; ++k) {
      if (!block_used<l>(k, b)) continue;
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          if (coupling<l>(3 * k + p, b) != 0.0f) gR[j][p] += gT[k][j] * coupling<l>(3 * k + p, b);
    }
  }
}

__device__ __forceinline__ void load_low(const float* __restrict__ w, float (&R)[3][3], float (&D2)[5][5]) {
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) R[a][b] = w[3 * a + b];
#pragma unroll
  for (int a = 0; a < 5; ++a)
#pragma unroll
    for (int b = 0; b < 5; ++b) D2[a][b] = w[9 + 5 * a + b];
}

constexpr int ext_width(int lmax) { return lmax >= 4 ? 80 : lmax == 3 ? 35 : 0; }

template <int LMAX>
__global__ __launch_bounds__(128) void wigner_ext_fwd_kernel(const float* __restrict__ wig, float* __restrict__ ext,
                                                              int64_t E) {
  constexpr int W = ext_width(LMAX);
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float R[3][3], D2[5][5];
  load_low(wig + e * 34, R, D2);
  float D3[7][7];
  rec_fwd<3, 0, 7>(D2, R, D3);
  float* o = ext + e * W;
#pragma unroll
  for (int a = 0; a < 5; ++a)
#pragma unroll
    for (int b = 0; b < 7; ++b) o[7 * a + b] = D3[1 + a][b];
  if constexpr (LMAX >= 4) {
    float D4[5][9];
    rec_fwd<4, 2, 5>(D3, R, D4);
#pragma unroll
    for (int a = 0; a < 5; ++a)
#pragma unroll
      for (int b = 0; b < 9; ++b) o[35 + 9 * a + b] = D4[a][b];
  }
}

template <int LMAX>
__global__ __launch_bounds__(128) void wigner_ext_bwd_kernel(const float* __restrict__ wig,
                                                              const float* __restrict__ g_ext,
                                                              float* __restrict__ g_wig, int64_t E) {
  constexpr int W = ext_width(LMAX);
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float R[3][3], D2[5][5];
  load_low(wig + e * 34, R, D2);
  const float* g = g_ext + e * W;
  float gR[3][3], gD2[5][5], G3[7][7];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) gR[a][b] = 0.0f;
#pragma unroll
  for (int a = 0; a < 5; ++a)
#pragma unroll
    for (int b = 0; b < 5; ++b) gD2[a][b] = 0.0f;
#pragma unroll
  for (int a = 0; a < 7; ++a)
#pragma unroll
    for (int b = 0; b < 7; ++b) G3[a][b] = (a >= 1 && a <= 5) ? g[7 * (a - 1) + b] : 0.0f;
  if constexpr (LMAX >= 4) {
    float D3[7][7], G4[5][9];
    rec_fwd<3, 0, 7>(D2, R, D3);
#pragma unroll
    for (int a = 0; a < 5; ++a)
#pragma unroll
      for (int b = 0; b < 9; ++b) G4[a][b] = g[35 + 9 * a + b];
    rec_bwd<4, 2, 5>(D3, R, G4, G3, gR);
  }
  rec_bwd<3, 0, 7>(D2, R, G3, gD2, gR);
  float* o = g_wig + e * 34;
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) o[3 * a + b] = gR[a][b];
#pragma unroll
  for (int a = 0; a < 5; ++a)
#pragma unroll
    for (int b = 0; b < 5; ++b) o[9 + 5 * a + b] = gD2[a][b];
}

}  // namespace fu

using namespace fu;

extern "C" int fu_wigner_ext_width(int32_t lmax) {
  return (lmax >= 2 && lmax <= 4) ? ext_width(lmax) : -1;
}

extern "C" int fu_wigner_ext_fwd(const float* wigner, float* wig_ext, int64_t E, int32_t lmax, void* stream) {
  if (E < 0) return set_error(FU_ERR_SHAPE, "fu_wigner_ext_fwd: bad shape");
  if (lmax < 3 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "fu_wigner_ext_fwd: lmax=%d (3 or 4)", lmax);
  if (E == 0) return FU_OK;
  if (!wigner || !wig_ext) return set_error(FU_ERR_NULL, "fu_wigner_ext_fwd: NULL argument");
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)cdiv(E, 128));
  if (lmax == 3) hipLaunchKernelGGL(wigner_ext_fwd_kernel<3>, grid, dim3(128), 0, s, wigner, wig_ext, E);
  else hipLaunchKernelGGL(wigner_ext_fwd_kernel<4>, grid, dim3(128), 0, s, wigner, wig_ext, E);
  return check_launch("fu_wigner_ext_fwd");
}

extern "C" int fu_wigner_ext_bwd(const float* wigner, const float* g_wig_ext, float* g_wigner, int64_t E,
                                 int32_t lmax, void* stream) {
  if (E < 0) return set_error(FU_ERR_SHAPE, "fu_wigner_ext_bwd: bad shape");
  if (lmax < 3 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "fu_wigner_ext_bwd: lmax=%d (3 or 4)", lmax);
  if (E == 0) return FU_OK;
  if (!wigner || !g_wig_ext || !g_wigner) return set_error(FU_ERR_NULL, "fu_wigner_ext_bwd: NULL argument");
  if (E > (int64_t)0xffffffff * 128) return set_error(FU_ERR_SHAPE, "fu_wigner_ext_bwd: E too large");
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)cdiv(E, 128));
  if (lmax == 3) hipLaunchKernelGGL(wigner_ext_bwd_kernel<3>, grid, dim3(128), 0, s, wigner, g_wig_ext, g_wigner, E);
  else hipLaunchKernelGGL(wigner_ext_bwd_kernel<4>, grid, dim3(128), 0, s, wigner, g_wig_ext, g_wigner, E);
  return check_launch("fu_wigner_ext_bwd");
}
