// Row LayerNorm (biased variance) + affine + SiLU and its input gradient
// (ops/ln_silu.py:29-123), for the radial-MLP hidden rows (D = edge channels).
//
// LPR = D/4 lanes own one row (4 consecutive floats per lane, one float4 access), so a
// wave64 covers 64/LPR rows; row statistics are butterfly sums within the LPR-lane group.
#include "fu_common.h"

namespace fu {

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int LPR>
__global__ __launch_bounds__(256) void ln_silu_fwd_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float* __restrict__ out,
                                                          float* __restrict__ mean_out, float* __restrict__ rstd_out,
                                                          int64_t M, float eps) {
  constexpr int D = 4 * LPR;
  constexpr int RPB = 256 / LPR;  // rows per block
  const int sub = threadIdx.x % LPR;
  const int64_t rows_step = (int64_t)gridDim.x * RPB;
  const float4 g = ld4(gamma + 4 * sub), b = ld4(beta + 4 * sub);
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < M; row += rows_step) {
    const float4 v = ld4(x + row * D + 4 * sub);
    const float mean = group_sum<LPR>(v.x + v.y + v.z + v.w) / D;
    const float4 xc = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
    const float var = group_sum<LPR>(xc.x * xc.x + xc.y * xc.y + xc.z * xc.z + xc.w * xc.w) / D;
    const float rstd = 1.0f / sqrtf(var + eps);
    float4 y;
    y.x = xc.x * rstd * g.x + b.x;
    y.y = xc.y * rstd * g.y + b.y;
    y.z = xc.z * rstd * g.z + b.z;
    y.w = xc.w * rstd * g.w + b.w;
    st4(out + row * D + 4 * sub,
        make_float4(y.x * sigmoidf_(y.x), y.y * sigmoidf_(y.y), y.z * sigmoidf_(y.z), y.w * sigmoidf_(y.w)));
    if (sub == 0) {
      mean_out[row] = mean;
      rstd_out[row] = rstd;
    }
  }
}

__device__ __forceinline__ float dsilu(float y) {
  const float s = sigmoidf_(y);
  return s + y * s * (1.0f - s);
}

template <int LPR>
__global__ __launch_bounds__(256) void ln_silu_bwd_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta,
                                                          const float* __restrict__ mean_in,
                                                          const float* __restrict__ rstd_in,
                                                          const float* __restrict__ g_out, float* __restrict__ g_x,
                                                          int64_t M) {
  constexpr int D = 4 * LPR;
  constexpr int RPB = 256 / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t rows_step = (int64_t)gridDim.x * RPB;
  const float4 g = ld4(gamma + 4 * sub), b = ld4(beta + 4 * sub);
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < M; row += rows_step) {
    const float4 v = ld4(x + row * D + 4 * sub);
    const float4 go = ld4(g_out + row * D + 4 * sub);
    const float mean = mean_in[row], rstd = rstd_in[row];
    const float xh[4] = {(v.x - mean) * rstd, (v.y - mean) * rstd, (v.z - mean) * rstd, (v.w - mean) * rstd};
    const float gg[4] = {g.x, g.y, g.z, g.w}, bb[4] = {b.x, b.y, b.z, b.w}, gov[4] = {go.x, go.y, go.z, go.w};
    float gxh[4];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float y = xh[k] * gg[k] + bb[k];
      gxh[k] = gov[k] * dsilu(y) * gg[k];
      s1 += gxh[k];
      s2 += gxh[k] * xh[k];
    }
    s1 = group_sum<LPR>(s1);
    s2 = group_sum<LPR>(s2);
    float4 o;
    o.x = rstd * (gxh[0] - (s1 + xh[0] * s2) / D);
    o.y = rstd * (gxh[1] - (s1 + xh[1] * s2) / D);
    o.z = rstd * (gxh[2] - (s1 + xh[2] * s2) / D);
    o.w = rstd * (gxh[3] - (s1 + xh[3] * s2) / D);
    st4(g_x + row * D + 4 * sub, o);
  }
}

}  // namespace fu

using namespace fu;

extern "C" int fu_ln_silu_fwd(const float* x, const float* gamma, const float* beta, float* out, float* mean,
                              float* rstd, int64_t M, int32_t D, float eps, void* stream) {
  if (M < 0) return set_error(FU_ERR_SHAPE, "fu_ln_silu_fwd: bad shape");
  if (D != 64 && D != 128 && D != 256) return set_error(FU_ERR_UNSUPPORTED, "fu_ln_silu_fwd: D=%d unsupported", D);
  if (M == 0) return FU_OK;
  if (!x || !gamma || !beta || !out || !mean || !rstd) return set_error(FU_ERR_NULL, "fu_ln_silu_fwd: NULL argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(gamma) || !aligned16(beta))
    return set_error(FU_ERR_ALIGN, "fu_ln_silu_fwd: rows must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int rpb = 256 / (D / 4);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(M, rpb), 65536);
  if (D == 64) hipLaunchKernelGGL(ln_silu_fwd_kernel<16>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, out, mean, rstd, M, eps);
  else if (D == 128) hipLaunchKernelGGL(ln_silu_fwd_kernel<32>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, out, mean, rstd, M, eps);
  else hipLaunchKernelGGL(ln_silu_fwd_kernel<64>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, out, mean, rstd, M, eps);
  return check_launch("fu_ln_silu_fwd");
}

extern "C" int fu_ln_silu_bwd(const float* x, const float* gamma, const float* beta, const float* mean,
                              const float* rstd, const float* g_out, float* g_x, int64_t M, int32_t D, void* stream) {
  if (M < 0) return set_error(FU_ERR_SHAPE, "fu_ln_silu_bwd: bad shape");
  if (D != 64 && D != 128 && D != 256) return set_error(FU_ERR_UNSUPPORTED, "fu_ln_silu_bwd: D=%d unsupported", D);
  if (M == 0) return FU_OK;
  if (!x || !gamma || !beta || !mean || !rstd || !g_out || !g_x) return set_error(FU_ERR_NULL, "fu_ln_silu_bwd: NULL argument");
  if (!aligned16(x) || !aligned16(g_out) || !aligned16(g_x) || !aligned16(gamma) || !aligned16(beta))
    return set_error(FU_ERR_ALIGN, "fu_ln_silu_bwd: rows must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int rpb = 256 / (D / 4);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(M, rpb), 65536);
  if (D == 64) hipLaunchKernelGGL(ln_silu_bwd_kernel<16>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, mean, rstd, g_out, g_x, M);
  else if (D == 128) hipLaunchKernelGGL(ln_silu_bwd_kernel<32>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, mean, rstd, g_out, g_x, M);
  else hipLaunchKernelGGL(ln_silu_bwd_kernel<64>, dim3(blocks), dim3(256), 0, s, x, gamma, beta, mean, rstd, g_out, g_x, M);
  return check_launch("fu_ln_silu_bwd");
}
