// Node-level kernels around the edge hot path: the equivariant RMS norm over SH
// coefficients and the gate activation of the atom-wise FFN (the FAIRChem modules the
// reference attaches as norm_1 / norm_2 / atom_wise / final_norm, model.py:145,157,218),
// row permutations of node and edge arrays (model.py:72-74,221) and the PBC shift product
// with its deterministic cell-gradient reduction (wrapper.py:193-194).
//
// Norm / gate: one wave64 per atom, lanes across channels, the (lmax + 1)^2 coefficient rows
// (lmax = 2, 3 or 4) in registers; row statistics are wave reductions.
#include "fu_vec.h"

namespace fu {

// degree l of SH coefficient k = l^2 + l + m
__device__ __forceinline__ constexpr int deg_of(int k) { return k < 1 ? 0 : k < 4 ? 1 : k < 9 ? 2 : k < 16 ? 3 : 4; }
// degree-balanced weight 1 / ((2l + 1)(lmax + 1))
template <int L>
__device__ __forceinline__ constexpr float bal_of(int l) { return 1.0f / (float)((2 * l + 1) * (L + 1)); }

__device__ __forceinline__ int wave_id_n() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// out = feat * (ms + eps)^-1/2 * w[deg] (+ b on l=0), feat = x with l=0 centred over channels,
// ms = mean_c sum_k feat_kc^2 / ((2 l_k + 1)(lmax + 1)).
template <int CPL, int L>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ b, float* __restrict__ out,
                                                           float* __restrict__ inv_rms, int64_t N, float eps) {
  constexpr int C = 64 * CPL, NK = (L + 1) * (L + 1);
  const int lane = threadIdx.x & 63, c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_n();
  if (n >= N) return;
  Vec<CPL> f[NK];
  const float* xn = x + n * NK * C + c;
#pragma unroll
  for (int k = 0; k < NK; ++k) f[k] = vload<CPL>(xn + k * C);
  float s0 = 0.0f;
#pragma unroll
  for (int q = 0; q < CPL; ++q) s0 += f[0][q];
  const float mean0 = wave_sum(s0) / C;
#pragma unroll
  for (int q = 0; q < CPL; ++q) f[0][q] -= mean0;
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NK; ++k) ss += bal_of<L>(deg_of(k)) * vdot(f[k], f[k]);
  const float ms = wave_sum(ss) / C;
  const float inv = 1.0f / sqrtf(ms + eps);
  if (lane == 0) inv_rms[n] = inv;
  float* on = out + n * NK * C + c;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const Vec<CPL> wk = vload<CPL>(w + deg_of(k) * C + c);
    Vec<CPL> o;
#pragma unroll
    for (int q = 0; q < CPL; ++q) o[q] = f[k][q] * (inv * wk[q]);
    if (k == 0) o = vadd(o, vload<CPL>(b + c));
    vstore(on + k * C, o);
  }
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ inv_rms,
                                                           const float* __restrict__ g_out,
                                                           const float* __restrict__ g_res, float* __restrict__ g_x,
                                                           int64_t N) {
  constexpr int C = 64 * CPL, NK = (L + 1) * (L + 1);
  const int lane = threadIdx.x & 63, c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_n();
  if (n >= N) return;
  Vec<CPL> f[NK], gw[NK];
  const float* xn = x + n * NK * C + c;
  const float* gn = g_out + n * NK * C + c;
#pragma unroll
  for (int k = 0; k < NK; ++k) f[k] = vload<CPL>(xn + k * C);
  float s0 = 0.0f;
#pragma unroll
  for (int q = 0; q < CPL; ++q) s0 += f[0][q];
  const float mean0 = wave_sum(s0) / C;
#pragma unroll
  for (int q = 0; q < CPL; ++q) f[0][q] -= mean0;
  const float inv = inv_rms[n];
  float s = 0.0f;  // sum_kc g_out w feat
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const Vec<CPL> wk = vload<CPL>(w + deg_of(k) * C + c);
    gw[k] = vmul(vload<CPL>(gn + k * C), wk);
    s += vdot(gw[k], f[k]);
  }
  s = wave_sum(s);
  // d out_kc / d feat_k'c' = inv w_kc delta - inv^3 bal_k' feat_k'c' w_kc feat_kc / C
  const float coef = inv * inv * inv * s / C;
  Vec<CPL> gf[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int q = 0; q < CPL; ++q) gf[k][q] = inv * gw[k][q] - coef * bal_of<L>(deg_of(k)) * f[k][q];
  float t0 = 0.0f;
#pragma unroll
  for (int q = 0; q < CPL; ++q) t0 += gf[0][q];
  const float mg0 = wave_sum(t0) / C;
#pragma unroll
  for (int q = 0; q < CPL; ++q) gf[0][q] -= mg0;
  float* go = g_x + n * NK * C + c;
  if (g_res) {  // the gradient of a residual branch that read the same x
    const float* gr = g_res + n * NK * C + c;
#pragma unroll
    for (int k = 0; k < NK; ++k) gf[k] = vadd(gf[k], vload<CPL>(gr + k * C));
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) vstore(go + k * C, gf[k]);
}

// Gate activation of the atom-wise FFN: gates = sigmoid(silu(pre)) per degree l >= 1 and
// channel; out_0 = silu(h_0), out_k = h_k * gate[l_k] for k >= 1.  pre is (N, lmax H), h and
// out are (N, (lmax + 1)^2, H).
template <int CPL, int L>
__global__ __launch_bounds__(256) void gate_fwd_kernel(const float* __restrict__ pre, const float* __restrict__ h,
                                                       float* __restrict__ out, int64_t N) {
  constexpr int H = 64 * CPL, NK = (L + 1) * (L + 1);
  const int lane = threadIdx.x & 63, c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_n();
  if (n >= N) return;
  Vec<CPL> gate[L];
#pragma unroll
  for (int l = 0; l < L; ++l) {
    const Vec<CPL> p = vload<CPL>(pre + n * L * H + l * H + c);
#pragma unroll
    for (int q = 0; q < CPL; ++q) gate[l][q] = sigmoidf_(p[q] * sigmoidf_(p[q]));
  }
  const float* hn = h + n * NK * H + c;
  float* on = out + n * NK * H + c;
  {
    const Vec<CPL> h0 = vload<CPL>(hn);
    Vec<CPL> o;
#pragma unroll
    for (int q = 0; q < CPL; ++q) o[q] = h0[q] * sigmoidf_(h0[q]);
    vstore(on, o);
  }
#pragma unroll
  for (int k = 1; k < NK; ++k) vstore(on + k * H, vmul(vload<CPL>(hn + k * H), gate[deg_of(k) - 1]));
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void gate_bwd_kernel(const float* __restrict__ pre, const float* __restrict__ h,
                                                       const float* __restrict__ g_out, float* __restrict__ g_pre,
                                                       float* __restrict__ g_h, int64_t N) {
  constexpr int H = 64 * CPL, NK = (L + 1) * (L + 1);
  const int lane = threadIdx.x & 63, c = lane * CPL;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id_n();
  if (n >= N) return;
  Vec<CPL> p[L], gate[L], ggate[L];
#pragma unroll
  for (int l = 0; l < L; ++l) {
    p[l] = vload<CPL>(pre + n * L * H + l * H + c);
#pragma unroll
    for (int q = 0; q < CPL; ++q) gate[l][q] = sigmoidf_(p[l][q] * sigmoidf_(p[l][q]));
    ggate[l] = vzero<CPL>();
  }
  const float* hn = h + n * NK * H + c;
  const float* gn = g_out + n * NK * H + c;
  float* ghn = g_h + n * NK * H + c;
  {
    const Vec<CPL> h0 = vload<CPL>(hn), g0 = vload<CPL>(gn);
    Vec<CPL> o;
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const float s = sigmoidf_(h0[q]);
      o[q] = g0[q] * (s + h0[q] * s * (1.0f - s));
    }
    vstore(ghn, o);
  }
#pragma unroll
  for (int k = 1; k < NK; ++k) {
    const int l = deg_of(k) - 1;
    const Vec<CPL> hk = vload<CPL>(hn + k * H), gk = vload<CPL>(gn + k * H);
    vstore(ghn + k * H, vmul(gk, gate[l]));
#pragma unroll
    for (int q = 0; q < CPL; ++q) ggate[l][q] += gk[q] * hk[q];
  }
#pragma unroll
  for (int l = 0; l < L; ++l) {
    Vec<CPL> o;
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const float sp = sigmoidf_(p[l][q]);
      const float du = sp + p[l][q] * sp * (1.0f - sp);  // d silu(pre) / d pre
      const float g = gate[l][q];
      o[q] = ggate[l][q] * g * (1.0f - g) * du;
    }
    vstore(g_pre + n * L * H + l * H + c, o);
  }
}

// dst[r, :] = src[idx[r], :] for rows of `width` floats.
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ src, const int64_t* __restrict__ idx,
                                                          float* __restrict__ dst, int64_t rows, int32_t width) {
  const int64_t total = rows * width;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / width;
    const int64_t k = t - r * width;
    dst[t] = src[idx[r] * width + k];
  }
}

// dst[idx[r], :] = src[r, :] (idx is a permutation: every destination row written once).
__global__ __launch_bounds__(256) void scatter_rows_kernel(const float* __restrict__ src,
                                                           const int64_t* __restrict__ idx, float* __restrict__ dst,
                                                           int64_t rows, int32_t width) {
  const int64_t total = rows * width;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / width;
    const int64_t k = t - r * width;
    dst[idx[r] * width + k] = src[t];
  }
}

// shifts[e] = offsets[perm[e]] @ cell (perm may be NULL: identity).
__global__ __launch_bounds__(256) void edge_shifts_kernel(const float* __restrict__ off, const float* __restrict__ cell,
                                                          const int64_t* __restrict__ perm, float* __restrict__ shifts,
                                                          int64_t E) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < E; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = perm ? perm[e] : e;
    const float o0 = off[3 * s], o1 = off[3 * s + 1], o2 = off[3 * s + 2];
#pragma unroll
    for (int d = 0; d < 3; ++d) shifts[3 * e + d] = o0 * cell[d] + o1 * cell[3 + d] + o2 * cell[6 + d];
  }
}

// out[a][b] = sum_e A[pa(e)][a] * B[e][b]: stage 1 — each workgroup reduces a contiguous
// slice in fp64 into partials[blockIdx][9]; stage 2 — one workgroup sums the partials in
// block order.  Deterministic for a fixed grid.
constexpr int OS_BLOCKS = 256;
__global__ __launch_bounds__(256) void outer_sum3_stage1(const float* __restrict__ A, const int64_t* __restrict__ pa,
                                                         const float* __restrict__ B, double* __restrict__ partial,
                                                         int64_t E) {
  __shared__ double red[9][256];
  const int64_t per = (E + gridDim.x - 1) / gridDim.x;
  const int64_t e0 = blockIdx.x * per, e1 = min(E, e0 + per);
  double acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
    const int64_t s = pa ? pa[e] : e;
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) acc[3 * a + b] += (double)A[3 * s + a] * (double)B[3 * e + b];
  }
#pragma unroll
  for (int k = 0; k < 9; ++k) red[k][threadIdx.x] = acc[k];
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s)
#pragma unroll
      for (int k = 0; k < 9; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x < 9) partial[blockIdx.x * 9 + threadIdx.x] = red[threadIdx.x][0];
}

// One wave: lane t sums the partials of blocks t, t + 64, ... in that order, then a fixed
// butterfly over the 64 lanes (the same order every call; nine serial sums over all blocks
// in one lane each took 44 us)
__global__ __launch_bounds__(64) void outer_sum3_stage2(const double* __restrict__ partial, int nblocks,
                                                        float* __restrict__ out) {
  const int t = threadIdx.x;
  double s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = t; b < nblocks; b += 64)
#pragma unroll
    for (int k = 0; k < 9; ++k) s[k] += partial[b * 9 + k];
#pragma unroll
  for (int k = 0; k < 9; ++k)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s[k] += __shfl_xor(s[k], off);
  if (t == 0)
#pragma unroll
    for (int k = 0; k < 9; ++k) out[k] = (float)s[k];
}

// Calls f(CPL, lmax) as integral constants; FU_ERR_UNSUPPORTED for other C.
template <typename F>
static int launch_cpl_l(int32_t C, int32_t lmax, F f) {
  auto by_l = [&](auto cpl) {
    if (lmax == 2) f(cpl, std::integral_constant<int, 2>{});
    else if (lmax == 3) f(cpl, std::integral_constant<int, 3>{});
    else f(cpl, std::integral_constant<int, 4>{});
  };
  if (C == 64) return by_l(std::integral_constant<int, 1>{}), FU_OK;
  if (C == 128) return by_l(std::integral_constant<int, 2>{}), FU_OK;
  if (C == 256) return by_l(std::integral_constant<int, 4>{}), FU_OK;
  return FU_ERR_UNSUPPORTED;
}

}  // namespace fu

using namespace fu;

#define FU_LMAX_CHECK(who)                                                                        \
  if (lmax < 2 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, who ": lmax=%d unsupported (2, 3 or 4)", lmax)

extern "C" int fu_rms_norm_sh_fwd(const float* x, const float* weight, const float* bias, float* out, float* inv_rms,
                                  int64_t N, int32_t C, int32_t lmax, float eps, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_rms_norm_sh_fwd: bad shape");
  FU_LMAX_CHECK("fu_rms_norm_sh_fwd");
  if (N == 0) return FU_OK;
  if (!x || !weight || !bias || !out || !inv_rms) return set_error(FU_ERR_NULL, "fu_rms_norm_sh_fwd: NULL argument");
  hipStream_t s = as_stream(stream);
  int st = launch_cpl_l(C, lmax, [&](auto cpl, auto lv) {
    hipLaunchKernelGGL((rms_norm_fwd_kernel<decltype(cpl)::value, decltype(lv)::value>), dim3(cdiv(N, 4)), dim3(256),
                       0, s, x, weight, bias, out, inv_rms, N, eps);
  });
  if (st != FU_OK) return set_error(st, "fu_rms_norm_sh_fwd: C=%d unsupported (64, 128 or 256)", C);
  return check_launch("fu_rms_norm_sh_fwd");
}

extern "C" int fu_rms_norm_sh_bwd(const float* x, const float* weight, const float* inv_rms, const float* g_out,
                                  const float* g_res, float* g_x, int64_t N, int32_t C, int32_t lmax, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_rms_norm_sh_bwd: bad shape");
  FU_LMAX_CHECK("fu_rms_norm_sh_bwd");
  if (N == 0) return FU_OK;
  if (!x || !weight || !inv_rms || !g_out || !g_x) return set_error(FU_ERR_NULL, "fu_rms_norm_sh_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  int st = launch_cpl_l(C, lmax, [&](auto cpl, auto lv) {
    hipLaunchKernelGGL((rms_norm_bwd_kernel<decltype(cpl)::value, decltype(lv)::value>), dim3(cdiv(N, 4)), dim3(256),
                       0, s, x, weight, inv_rms, g_out, g_res, g_x, N);
  });
  if (st != FU_OK) return set_error(st, "fu_rms_norm_sh_bwd: C=%d unsupported (64, 128 or 256)", C);
  return check_launch("fu_rms_norm_sh_bwd");
}

extern "C" int fu_gate_act_fwd(const float* pre, const float* h, float* out, int64_t N, int32_t H, int32_t lmax,
                               void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_gate_act_fwd: bad shape");
  FU_LMAX_CHECK("fu_gate_act_fwd");
  if (N == 0) return FU_OK;
  if (!pre || !h || !out) return set_error(FU_ERR_NULL, "fu_gate_act_fwd: NULL argument");
  hipStream_t s = as_stream(stream);
  int st = launch_cpl_l(H, lmax, [&](auto cpl, auto lv) {
    hipLaunchKernelGGL((gate_fwd_kernel<decltype(cpl)::value, decltype(lv)::value>), dim3(cdiv(N, 4)), dim3(256), 0,
                       s, pre, h, out, N);
  });
  if (st != FU_OK) return set_error(st, "fu_gate_act_fwd: H=%d unsupported (64, 128 or 256)", H);
  return check_launch("fu_gate_act_fwd");
}

extern "C" int fu_gate_act_bwd(const float* pre, const float* h, const float* g_out, float* g_pre, float* g_h,
                               int64_t N, int32_t H, int32_t lmax, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_gate_act_bwd: bad shape");
  FU_LMAX_CHECK("fu_gate_act_bwd");
  if (N == 0) return FU_OK;
  if (!pre || !h || !g_out || !g_pre || !g_h) return set_error(FU_ERR_NULL, "fu_gate_act_bwd: NULL argument");
  hipStream_t s = as_stream(stream);
  int st = launch_cpl_l(H, lmax, [&](auto cpl, auto lv) {
    hipLaunchKernelGGL((gate_bwd_kernel<decltype(cpl)::value, decltype(lv)::value>), dim3(cdiv(N, 4)), dim3(256), 0,
                       s, pre, h, g_out, g_pre, g_h, N);
  });
  if (st != FU_OK) return set_error(st, "fu_gate_act_bwd: H=%d unsupported (64, 128 or 256)", H);
  return check_launch("fu_gate_act_bwd");
}

extern "C" int fu_gather_rows(const float* src, const int64_t* idx, float* dst, int64_t rows, int32_t width,
                              void* stream) {
  if (rows < 0 || width <= 0) return set_error(FU_ERR_SHAPE, "fu_gather_rows: bad shape");
  if (rows == 0) return FU_OK;
  if (!src || !idx || !dst) return set_error(FU_ERR_NULL, "fu_gather_rows: NULL argument");
  const int64_t tot = rows * width;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)std::min<int64_t>(cdiv(tot, 256), 65536)), dim3(256), 0,
                     as_stream(stream), src, idx, dst, rows, width);
  return check_launch("fu_gather_rows");
}

extern "C" int fu_scatter_rows(const float* src, const int64_t* idx, float* dst, int64_t rows, int32_t width,
                               void* stream) {
  if (rows < 0 || width <= 0) return set_error(FU_ERR_SHAPE, "fu_scatter_rows: bad shape");
  if (rows == 0) return FU_OK;
  if (!src || !idx || !dst) return set_error(FU_ERR_NULL, "fu_scatter_rows: NULL argument");
  const int64_t tot = rows * width;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)std::min<int64_t>(cdiv(tot, 256), 65536)), dim3(256), 0,
                     as_stream(stream), src, idx, dst, rows, width);
  return check_launch("fu_scatter_rows");
}

extern "C" int fu_edge_shifts(const float* cell_offsets, const float* cell, const int64_t* perm, float* shifts,
                              int64_t E, void* stream) {
  if (E < 0) return set_error(FU_ERR_SHAPE, "fu_edge_shifts: bad shape");
  if (E == 0) return FU_OK;
  if (!cell_offsets || !cell || !shifts) return set_error(FU_ERR_NULL, "fu_edge_shifts: NULL argument");
  hipLaunchKernelGGL(edge_shifts_kernel, dim3((unsigned)std::min<int64_t>(cdiv(E, 256), 65536)), dim3(256), 0,
                     as_stream(stream), cell_offsets, cell, perm, shifts, E);
  return check_launch("fu_edge_shifts");
}

extern "C" int fu_outer_sum3(const float* A, const int64_t* perm_a, const float* B, float* out, double* partial,
                             int64_t partial_len, int64_t E, void* stream) {
  if (E < 0) return set_error(FU_ERR_SHAPE, "fu_outer_sum3: bad shape");
  if (!out || !partial) return set_error(FU_ERR_NULL, "fu_outer_sum3: NULL argument");
  if (partial_len < OS_BLOCKS * 9)
    return set_error(FU_ERR_WORKSPACE, "fu_outer_sum3: partial workspace needs %d doubles", OS_BLOCKS * 9);
  if (E > 0 && (!A || !B)) return set_error(FU_ERR_NULL, "fu_outer_sum3: NULL argument");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(outer_sum3_stage1, dim3(OS_BLOCKS), dim3(256), 0, s, A, perm_a, B, partial, E);
  hipLaunchKernelGGL(outer_sum3_stage2, dim3(1), dim3(64), 0, s, partial, OS_BLOCKS, out);
  return check_launch("fu_outer_sum3");
}
