// Row LayerNorm (biased variance) + affine + SiLU and its input gradient
// (ops/ln_silu.py:29-123), for the radial-MLP hidden rows (D = edge channels).
//
// General ("grouped") form: a row of the input matrix holds G groups of D values; group g of
// row e is normalised on its own, with its own gamma/beta/bias, after adding optional
// per-element table rows tab_src[z[isrc[e]]] and tab_dst[z[idst[e]]] (z = atomic numbers,
// isrc/idst = edge endpoints).  This lets the first radial
// layer of all blocks run as one GEMM over the Gaussian basis while the element-embedding
// part of that layer (W1[:, B:] [W_src[Z_i]; W_tgt[Z_j]]) comes from precomputed tables.
//
// LPR = D/4 lanes own one (row, group) (4 consecutive floats per lane, one float4 access), so
// a wave64 covers 64/LPR of them; statistics are butterfly sums within the LPR-lane group.
#include "fu_common.h"

namespace fu {

struct LnArgs {
  const float* x; int64_t ldx;
  const float* tab_src; const float* tab_dst; int64_t ldt;
  const int64_t* z; const int64_t* isrc; const int64_t* idst;
  const float* bias; const float* gamma; const float* beta;
  int64_t M; int32_t G;
};

// Table rows of one input row (nullptr without tables).
struct RowTabs {
  const float* src;
  const float* dst;
};

__device__ __forceinline__ RowTabs row_tables(const LnArgs& a, int64_t row) {
  if (a.tab_src == nullptr) return {nullptr, nullptr};
  return {a.tab_src + a.z[a.isrc[row]] * a.ldt, a.tab_dst + a.z[a.idst[row]] * a.ldt};
}

// x + tables + bias for the 4 values of this lane in (row, group)
template <int D>
__device__ __forceinline__ float4 ln_input(const LnArgs& a, const RowTabs& t, int64_t row, int g, int sub) {
  const int col = g * D + 4 * sub;
  float4 v = ld4(a.x + row * a.ldx + col);
  if (t.src != nullptr) v = v + ld4(t.src + col) + ld4(t.dst + col);
  if (a.bias != nullptr) v = v + ld4(a.bias + col);
  return v;
}

// One (row, group) of the forward: LayerNorm statistics over the group's D values, affine, SiLU.
template <int LPR>
__device__ __forceinline__ void ln_fwd_item(const LnArgs& a, const RowTabs& t, int64_t row, int g, int sub,
                                            float* __restrict__ out, int64_t ldo, float* __restrict__ mean_out,
                                            float* __restrict__ rstd_out, float eps) {
  constexpr int D = 4 * LPR;
  const float4 v = ln_input<D>(a, t, row, g, sub);
  const float mean = group_sum<LPR>(v.x + v.y + v.z + v.w) / D;
  const float4 xc = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
  const float var = group_sum<LPR>(xc.x * xc.x + xc.y * xc.y + xc.z * xc.z + xc.w * xc.w) / D;
  const float rstd = 1.0f / sqrtf(var + eps);
  const float4 gm = ld4(a.gamma + g * D + 4 * sub), bt = ld4(a.beta + g * D + 4 * sub);
  float4 y;
  y.x = xc.x * rstd * gm.x + bt.x;
  y.y = xc.y * rstd * gm.y + bt.y;
  y.z = xc.z * rstd * gm.z + bt.z;
  y.w = xc.w * rstd * gm.w + bt.w;
  st4(out + row * ldo + g * D + 4 * sub,
      make_float4(y.x * sigmoidf_(y.x), y.y * sigmoidf_(y.y), y.z * sigmoidf_(y.z), y.w * sigmoidf_(y.w)));
  if (sub == 0) {
    mean_out[row * a.G + g] = mean;
    rstd_out[row * a.G + g] = rstd;
  }
}

// Rows are spread over LPR-lane groups (256 / LPR rows per block, grid-stride); each group
// walks the G column groups of its row, so the table rows are located once per row.
template <int LPR>
__global__ __launch_bounds__(256) void ln_silu_fwd_kernel(LnArgs a, float* __restrict__ out, int64_t ldo,
                                                          float* __restrict__ mean_out, float* __restrict__ rstd_out,
                                                          float eps) {
  constexpr int RPB = 256 / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t step = (int64_t)gridDim.x * RPB;
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < a.M; row += step) {
    const RowTabs t = row_tables(a, row);
    for (int g = 0; g < a.G; ++g) ln_fwd_item<LPR>(a, t, row, g, sub, out, ldo, mean_out, rstd_out, eps);
  }
}

__device__ __forceinline__ float dsilu(float y) {
  const float s = sigmoidf_(y);
  return s + y * s * (1.0f - s);
}

template <int LPR>
__device__ __forceinline__ void ln_bwd_item(const LnArgs& a, const RowTabs& t, int64_t row, int g, int sub,
                                            const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                                            const float* __restrict__ g_out, int64_t ldg, float* __restrict__ g_x,
                                            int64_t ldgx) {
  constexpr int D = 4 * LPR;
  const float4 v = ln_input<D>(a, t, row, g, sub);
  const float4 go = ld4(g_out + row * ldg + g * D + 4 * sub);
  const float4 gm = ld4(a.gamma + g * D + 4 * sub), bt = ld4(a.beta + g * D + 4 * sub);
  const float mean = mean_in[row * a.G + g], rstd = rstd_in[row * a.G + g];
  const float xh[4] = {(v.x - mean) * rstd, (v.y - mean) * rstd, (v.z - mean) * rstd, (v.w - mean) * rstd};
  const float gg[4] = {gm.x, gm.y, gm.z, gm.w}, bb[4] = {bt.x, bt.y, bt.z, bt.w}, gov[4] = {go.x, go.y, go.z, go.w};
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
  st4(g_x + row * ldgx + g * D + 4 * sub, o);
}

template <int LPR>
__global__ __launch_bounds__(256) void ln_silu_bwd_kernel(LnArgs a, const float* __restrict__ mean_in,
                                                          const float* __restrict__ rstd_in,
                                                          const float* __restrict__ g_out, int64_t ldg,
                                                          float* __restrict__ g_x, int64_t ldgx) {
  constexpr int RPB = 256 / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t step = (int64_t)gridDim.x * RPB;
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < a.M; row += step) {
    const RowTabs t = row_tables(a, row);
    for (int g = 0; g < a.G; ++g) ln_bwd_item<LPR>(a, t, row, g, sub, mean_in, rstd_in, g_out, ldg, g_x, ldgx);
  }
}

static unsigned ln_blocks(int64_t rows, int D) {
  const int rpb = 256 / (D / 4);
  return (unsigned)std::min<int64_t>(cdiv(rows, rpb), 65536);
}

static int ln_check(const LnArgs& a, int64_t ld_out, int32_t D, const char* who) {
  if (a.M < 0 || a.G < 1) return set_error(FU_ERR_SHAPE, "%s: bad shape", who);
  if (D != 64 && D != 128 && D != 256) return set_error(FU_ERR_UNSUPPORTED, "%s: D=%d unsupported", who, D);
  if (a.ldx < (int64_t)a.G * D || ld_out < (int64_t)a.G * D) return set_error(FU_ERR_SHAPE, "%s: row stride < G*D", who);
  if ((a.ldx | ld_out) % 4 != 0 || (a.tab_src && a.ldt % 4 != 0))
    return set_error(FU_ERR_ALIGN, "%s: row strides must be multiples of 4", who);
  if ((a.tab_src == nullptr) != (a.tab_dst == nullptr) || (a.tab_src && a.M > 0 && (!a.z || !a.isrc || !a.idst)))
    return set_error(FU_ERR_NULL, "%s: tables need both sides and their element ids", who);
  if (a.M > 0 && (!a.x || !a.gamma || !a.beta)) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  const void* al[] = {a.x, a.tab_src, a.tab_dst, a.bias, a.gamma, a.beta};
  for (const void* p : al)
    if (p && !aligned16(p)) return set_error(FU_ERR_ALIGN, "%s: arrays must be 16-byte aligned", who);
  return FU_OK;
}

template <typename F>
static void ln_dispatch(int32_t D, F f) {
  if (D == 64) f(std::integral_constant<int, 16>{});
  else if (D == 128) f(std::integral_constant<int, 32>{});
  else f(std::integral_constant<int, 64>{});
}

}  // namespace fu

using namespace fu;

extern "C" int fu_ln_silu_grouped_fwd(const float* x, int64_t ldx, const float* tab_src, const float* tab_dst,
                                      int64_t ldt, const int64_t* z, const int64_t* isrc, const int64_t* idst,
                                      const float* bias, const float* gamma, const float* beta, float* out, int64_t ldo, float* mean,
                                      float* rstd, int64_t M, int32_t G, int32_t D, float eps, void* stream) {
  LnArgs a{x, ldx, tab_src, tab_dst, ldt, z, isrc, idst, bias, gamma, beta, M, G};
  int st = ln_check(a, ldo, D, "fu_ln_silu_grouped_fwd");
  if (st != FU_OK) return st;
  if (M == 0) return FU_OK;
  if (!out || !mean || !rstd || !aligned16(out)) return set_error(FU_ERR_NULL, "fu_ln_silu_grouped_fwd: bad output");
  hipStream_t s = as_stream(stream);
  const unsigned blocks = ln_blocks(M, D);
  ln_dispatch(D, [&](auto lpr) {
    hipLaunchKernelGGL(ln_silu_fwd_kernel<decltype(lpr)::value>, dim3(blocks), dim3(256), 0, s, a, out, ldo, mean,
                       rstd, eps);
  });
  return check_launch("fu_ln_silu_grouped_fwd");
}

extern "C" int fu_ln_silu_grouped_bwd(const float* x, int64_t ldx, const float* tab_src, const float* tab_dst,
                                      int64_t ldt, const int64_t* z, const int64_t* isrc, const int64_t* idst,
                                      const float* bias, const float* gamma, const float* beta, const float* mean, const float* rstd,
                                      const float* g_out, int64_t ldg, float* g_x, int64_t ldgx, int64_t M, int32_t G,
                                      int32_t D, void* stream) {
  LnArgs a{x, ldx, tab_src, tab_dst, ldt, z, isrc, idst, bias, gamma, beta, M, G};
  int st = ln_check(a, ldgx, D, "fu_ln_silu_grouped_bwd");
  if (st != FU_OK) return st;
  if (M == 0) return FU_OK;
  if (!mean || !rstd || !g_out || !g_x || ldg < (int64_t)G * D || ldg % 4 != 0 || !aligned16(g_out) ||
      !aligned16(g_x))
    return set_error(FU_ERR_NULL, "fu_ln_silu_grouped_bwd: bad gradient arguments");
  hipStream_t s = as_stream(stream);
  const unsigned blocks = ln_blocks(M, D);
  ln_dispatch(D, [&](auto lpr) {
    hipLaunchKernelGGL(ln_silu_bwd_kernel<decltype(lpr)::value>, dim3(blocks), dim3(256), 0, s, a, mean, rstd, g_out,
                       ldg, g_x, ldgx);
  });
  return check_launch("fu_ln_silu_grouped_bwd");
}

extern "C" int fu_ln_silu_fwd(const float* x, const float* gamma, const float* beta, float* out, float* mean,
                              float* rstd, int64_t M, int32_t D, float eps, void* stream) {
  if (M < 0) return set_error(FU_ERR_SHAPE, "fu_ln_silu_fwd: bad shape");
  if (D != 64 && D != 128 && D != 256) return set_error(FU_ERR_UNSUPPORTED, "fu_ln_silu_fwd: D=%d unsupported", D);
  return fu_ln_silu_grouped_fwd(x, D, nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, gamma, beta, out, D, mean, rstd,
                                M, 1, D, eps, stream);
}

extern "C" int fu_ln_silu_bwd(const float* x, const float* gamma, const float* beta, const float* mean,
                              const float* rstd, const float* g_out, float* g_x, int64_t M, int32_t D, void* stream) {
  if (M < 0) return set_error(FU_ERR_SHAPE, "fu_ln_silu_bwd: bad shape");
  if (D != 64 && D != 128 && D != 256) return set_error(FU_ERR_UNSUPPORTED, "fu_ln_silu_bwd: D=%d unsupported", D);
  return fu_ln_silu_grouped_bwd(x, D, nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, gamma, beta, mean, rstd, g_out,
                                D, g_x, D, M, 1, D, stream);
}
