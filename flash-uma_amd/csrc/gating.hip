// Gate activation over the rotated-frame m-blocks (ops/gating.py:32-185).
//
// Y_m0 (E,5C) = [gate_l1, gate_l2, y_l0, y_l1m0, y_l2m0], Y_m1 (E,4C) = [R_l1, R_l2, I_l1, I_l2],
// Y_m2 (E,2C) = [R, I].  Z_m0 = [silu(y_l0), y_l1m0*s1, y_l2m0*s2], Z_m1 = [R_l1*s1, R_l2*s2,
// I_l1*s1, I_l2*s2], Z_m2 = [R*s2, I*s2] with s1 = sigmoid(gate_l1), s2 = sigmoid(gate_l2).
//
// Pure streaming work (HBM-bound): one thread per (edge, 4 channels), float4 loads and
// stores, 64-bit offsets.  Forward moves 20 floats per (edge, channel) and backward 31.
//
// Y_m0 (and g_Y_m0) come in one of two column orders: layout 0 is the order above; layout 1
// is the gate-paired order of the fused conv1 epilogue (fu_linear_gate): 64-column pairs
// [gate_l1 | y_l1m0] x C/32, [gate_l2 | y_l2m0] x C/32, then y_l0.
#include "fu_common.h"

namespace fu {

// Column offsets of gate_l1, gate_l2, y_l0, y_l1m0, y_l2m0 for channel c (c % 4 == 0).
template <int L>
__device__ __forceinline__ void y0_offsets(int64_t c, int64_t C, int64_t* o) {
  if constexpr (L == 0) {
#pragma unroll
    for (int k = 0; k < 5; ++k) o[k] = k * C + c;
  } else {
    const int64_t blk = c >> 5, in = c & 31;
    o[0] = 64 * blk + in;
    o[3] = o[0] + 32;
    o[1] = 64 * ((C >> 5) + blk) + in;
    o[4] = o[1] + 32;
    o[2] = 4 * C + c;
  }
}

template <int L>
__global__ __launch_bounds__(256) void gating_fwd_kernel(const float* __restrict__ Y0,
                                                         const float* __restrict__ Y1,
                                                         const float* __restrict__ Y2,
                                                         float* __restrict__ Z0,
                                                         float* __restrict__ Z1,
                                                         float* __restrict__ Z2, int64_t total,
                                                         int32_t C4) {
  const int64_t C = 4 * (int64_t)C4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = t / C4;
    const int64_t c = 4 * (t - e * C4);
    int64_t o[5];
    y0_offsets<L>(c, C, o);
    const float* y0 = Y0 + e * 5 * C;
    const float* y1 = Y1 + e * 4 * C + c;
    const float* y2 = Y2 + e * 2 * C + c;
    const float4 a0 = ld4(y0 + o[0]), a1 = ld4(y0 + o[1]), l0 = ld4(y0 + o[2]), l1 = ld4(y0 + o[3]),
                 l2 = ld4(y0 + o[4]);
    const float4 r1 = ld4(y1), r2 = ld4(y1 + C), i1 = ld4(y1 + 2 * C), i2 = ld4(y1 + 3 * C);
    const float4 mr = ld4(y2), mi = ld4(y2 + C);
    const float4 s1 = make_float4(sigmoidf_(a0.x), sigmoidf_(a0.y), sigmoidf_(a0.z), sigmoidf_(a0.w));
    const float4 s2 = make_float4(sigmoidf_(a1.x), sigmoidf_(a1.y), sigmoidf_(a1.z), sigmoidf_(a1.w));
    const float4 sl = make_float4(sigmoidf_(l0.x), sigmoidf_(l0.y), sigmoidf_(l0.z), sigmoidf_(l0.w));
    float* z0 = Z0 + e * 3 * C + c;
    float* z1 = Z1 + e * 4 * C + c;
    float* z2 = Z2 + e * 2 * C + c;
    st4(z0, l0 * sl);
    st4(z0 + C, l1 * s1);
    st4(z0 + 2 * C, l2 * s2);
    st4(z1, r1 * s1);
    st4(z1 + C, r2 * s2);
    st4(z1 + 2 * C, i1 * s1);
    st4(z1 + 3 * C, i2 * s2);
    st4(z2, mr * s2);
    st4(z2 + C, mi * s2);
  }
}

__device__ __forceinline__ void gate_bwd_lane(float a0, float a1, float l0, float l1, float l2,
                                              float r1, float r2, float i1, float i2, float mr,
                                              float mi, float gl0, float gl1, float gl2, float gr1,
                                              float gr2, float gi1, float gi2, float gmr, float gmi,
                                              float* o) {
  const float s1 = sigmoidf_(a0), ds1 = s1 * (1.0f - s1);
  const float s2 = sigmoidf_(a1), ds2 = s2 * (1.0f - s2);
  const float sl = sigmoidf_(l0), dsl = sl * (1.0f - sl);
  o[0] = ds1 * (gl1 * l1 + gr1 * r1 + gi1 * i1);
  o[1] = ds2 * (gl2 * l2 + gr2 * r2 + gi2 * i2 + gmr * mr + gmi * mi);
  o[2] = gl0 * (sl + l0 * dsl);
  o[3] = gl1 * s1;
  o[4] = gl2 * s2;
  o[5] = gr1 * s1;
  o[6] = gr2 * s2;
  o[7] = gi1 * s1;
  o[8] = gi2 * s2;
  o[9] = gmr * s2;
  o[10] = gmi * s2;
}

template <int L>
__global__ __launch_bounds__(256) void gating_bwd_kernel(
    const float* __restrict__ gZ0, const float* __restrict__ gZ1, const float* __restrict__ gZ2,
    const float* __restrict__ Y0, const float* __restrict__ Y1, const float* __restrict__ Y2,
    float* __restrict__ gY0, float* __restrict__ gY1, float* __restrict__ gY2, int64_t total,
    int32_t C4) {
  const int64_t C = 4 * (int64_t)C4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = t / C4;
    const int64_t c = 4 * (t - e * C4);
    int64_t o[5];
    y0_offsets<L>(c, C, o);
    const float* y0 = Y0 + e * 5 * C;
    const float* y1 = Y1 + e * 4 * C + c;
    const float* y2 = Y2 + e * 2 * C + c;
    const float* g0 = gZ0 + e * 3 * C + c;
    const float* g1 = gZ1 + e * 4 * C + c;
    const float* g2 = gZ2 + e * 2 * C + c;
    const float* srcs[20] = {y0 + o[0], y0 + o[1], y0 + o[2], y0 + o[3], y0 + o[4], y1, y1 + C,
                             y1 + 2 * C, y1 + 3 * C, y2, y2 + C, g0, g0 + C, g0 + 2 * C, g1,
                             g1 + C, g1 + 2 * C, g1 + 3 * C, g2, g2 + C};
    float v[20][4];
#pragma unroll
    for (int s = 0; s < 20; ++s) {
      const float4 t4 = ld4(srcs[s]);
      v[s][0] = t4.x; v[s][1] = t4.y; v[s][2] = t4.z; v[s][3] = t4.w;
    }
    float out[4][11];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gate_bwd_lane(v[0][q], v[1][q], v[2][q], v[3][q], v[4][q], v[5][q], v[6][q], v[7][q],
                    v[8][q], v[9][q], v[10][q], v[11][q], v[12][q], v[13][q], v[14][q], v[15][q],
                    v[16][q], v[17][q], v[18][q], v[19][q], out[q]);
    }
    float* o0 = gY0 + e * 5 * C;
    float* o1 = gY1 + e * 4 * C + c;
    float* o2 = gY2 + e * 2 * C + c;
    float* dst[11] = {o0 + o[0], o0 + o[1], o0 + o[2], o0 + o[3], o0 + o[4], o1, o1 + C, o1 + 2 * C,
                      o1 + 3 * C, o2, o2 + C};
#pragma unroll
    for (int s = 0; s < 11; ++s) st4(dst[s], make_float4(out[0][s], out[1][s], out[2][s], out[3][s]));
  }
}

static int gating_check(const void* const* ptrs, int n, int64_t E, int32_t C, int32_t layout, const char* who) {
  if (E < 0 || C <= 0) return set_error(FU_ERR_SHAPE, "%s: bad shape E=%lld C=%d", who, (long long)E, C);
  if (C % 4 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 4", who, C);
  if (layout != 0 && layout != 1) return set_error(FU_ERR_UNSUPPORTED, "%s: layout %d", who, layout);
  if (layout == 1 && C % 64 != 0)
    return set_error(FU_ERR_UNSUPPORTED, "%s: the gate-paired layout needs C a multiple of 64", who);
  for (int k = 0; k < n && E > 0; ++k) {
    if (ptrs[k] == nullptr) return set_error(FU_ERR_NULL, "%s: pointer %d is NULL", who, k);
    if (!aligned16(ptrs[k])) return set_error(FU_ERR_ALIGN, "%s: pointer %d not 16-byte aligned", who, k);
  }
  return FU_OK;
}

}  // namespace fu

using namespace fu;

extern "C" int fu_gating_fwd(const float* Y_m0, const float* Y_m1, const float* Y_m2, float* Z_m0,
                             float* Z_m1, float* Z_m2, int64_t E, int32_t C, int32_t layout, void* stream) {
  const void* ptrs[] = {Y_m0, Y_m1, Y_m2, Z_m0, Z_m1, Z_m2};
  int st = gating_check(ptrs, 6, E, C, layout, "fu_gating_fwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  const int64_t total = E * (C / 4);
  const int64_t blocks = std::min<int64_t>(cdiv(total, 256), kMaxBlocks);
  if (layout)
    hipLaunchKernelGGL(gating_fwd_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       Y_m0, Y_m1, Y_m2, Z_m0, Z_m1, Z_m2, total, C / 4);
  else
    hipLaunchKernelGGL(gating_fwd_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       Y_m0, Y_m1, Y_m2, Z_m0, Z_m1, Z_m2, total, C / 4);
  return check_launch("fu_gating_fwd");
}

extern "C" int fu_gating_bwd(const float* g_Z_m0, const float* g_Z_m1, const float* g_Z_m2,
                             const float* Y_m0, const float* Y_m1, const float* Y_m2, float* g_Y_m0,
                             float* g_Y_m1, float* g_Y_m2, int64_t E, int32_t C, int32_t layout,
                             void* stream) {
  const void* ptrs[] = {g_Z_m0, g_Z_m1, g_Z_m2, Y_m0, Y_m1, Y_m2, g_Y_m0, g_Y_m1, g_Y_m2};
  int st = gating_check(ptrs, 9, E, C, layout, "fu_gating_bwd");
  if (st != FU_OK) return st;
  if (E == 0) return FU_OK;
  const int64_t total = E * (C / 4);
  const int64_t blocks = std::min<int64_t>(cdiv(total, 256), kMaxBlocks);
  if (layout)
    hipLaunchKernelGGL(gating_bwd_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       g_Z_m0, g_Z_m1, g_Z_m2, Y_m0, Y_m1, Y_m2, g_Y_m0, g_Y_m1, g_Y_m2, total, C / 4);
  else
    hipLaunchKernelGGL(gating_bwd_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       g_Z_m0, g_Z_m1, g_Z_m2, Y_m0, Y_m1, Y_m2, g_Y_m0, g_Y_m1, g_Y_m2, total, C / 4);
  return check_launch("fu_gating_bwd");
}
