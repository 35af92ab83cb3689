// Charge / spin channel balancing: FAIRChem's balance_channels_batched, which the reference
// applies after every message-passing block when the backbone reserves l = 0 channels for
// the system charge or spin (model.py:213-216; channel ranges read at wrapper.py:53-56).
//
// For every system s and channel c in [c0, c1), the l = 0 coefficients of the system's atoms
// are shifted by one common amount so that they sum to target[s] - offset:
//   out[a][0][c] = x[a][0][c] + (target[s] - offset - sum_{a' in s} x[a'][0][c]) / n_s
// and every other coefficient and channel is copied.  The map is affine; its input gradient
// is the same correction with target = offset = 0 applied to the output gradient (the
// per-system mean of each balanced channel's gradient is removed).
//
// Atoms of one system are contiguous (the Morton sort keys carry the system id in their high
// bits), so a system is the CSR segment [sys_ptr[s], sys_ptr[s + 1]).  One workgroup per
// system sums its segment in fp64 with a fixed lane assignment and a fixed tree: the result
// is deterministic.  A second, bandwidth-bound pass writes the output rows.
#include <mutex>

#include "fu_common.h"

namespace fu {

// corr[s * nch + c] = (t_s - offset - sum) / n_s (0 for an empty system); t_s = target[s]
// or 0 without target.  Thread t serves channel cb + (t mod W) and atom lanes t / W; W is
// the power of two >= nch (at most 64), so a row's channel range is read by adjacent lanes.
__global__ __launch_bounds__(256) void balance_sums_kernel(const float* __restrict__ x,
                                                           const int32_t* __restrict__ sys_ptr,
                                                           const float* __restrict__ target, float offset,
                                                           float* __restrict__ corr, int64_t row, int32_t c0,
                                                           int32_t nch, int32_t W) {
  __shared__ double red[256];
  const int s = blockIdx.x;
  const int lanes = 256 / W;
  const int ch = threadIdx.x % W, lane = threadIdx.x / W;
  const int64_t a0 = sys_ptr[s], a1 = sys_ptr[s + 1];
  const double t = (target ? (double)target[s] : 0.0) - (double)offset;
  for (int cb = 0; cb < nch; cb += W) {
    const int c = cb + ch;
    double acc0 = 0.0, acc1 = 0.0;
    if (c < nch) {
      const float* col = x + c0 + c;
      int64_t a = a0 + lane;
      for (; a + lanes < a1; a += 2 * lanes) {
        acc0 += (double)col[a * row];
        acc1 += (double)col[(a + lanes) * row];
      }
      if (a < a1) acc0 += (double)col[a * row];
    }
    red[threadIdx.x] = acc0 + acc1;
    __syncthreads();
    for (int h = lanes >> 1; h > 0; h >>= 1) {
      if (lane < h) red[threadIdx.x] += red[threadIdx.x + h * W];
      __syncthreads();
    }
    if (lane == 0 && c < nch) {
      const int64_t n = a1 - a0;
      corr[(int64_t)s * nch + c] = n > 0 ? (float)((t - red[ch]) / (double)n) : 0.0f;
    }
    __syncthreads();
  }
}

// out = x, plus corr[batch[a]][c - c0] on coefficient 0, channels [c0, c0 + nch).  One
// float4 per thread (row = K*C floats, a multiple of 4); grid-stride.
__global__ __launch_bounds__(256) void balance_apply_kernel(const float* __restrict__ x,
                                                            const int64_t* __restrict__ batch,
                                                            const float* __restrict__ corr, float* __restrict__ out,
                                                            int64_t n4, int64_t row, int32_t c0, int32_t nch) {
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n4; v += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = 4 * v;
    const int64_t a = i / row;
    const int64_t r = i - a * row;
    float4 val = ld4(x + i);
    if (nch > 0 && r < c0 + nch && r + 4 > c0) {
      const float* cr = corr + batch[a] * nch - c0;
      if (r + 0 >= c0 && r + 0 < c0 + nch) val.x += cr[r + 0];
      if (r + 1 >= c0 && r + 1 < c0 + nch) val.y += cr[r + 1];
      if (r + 2 >= c0 && r + 2 < c0 + nch) val.z += cr[r + 2];
      if (r + 3 >= c0 && r + 3 < c0 + nch) val.w += cr[r + 3];
    }
    st4(out + i, val);
  }
}

}  // namespace fu

using namespace fu;

namespace {

int balance_launch(const char* who, const float* x, float* out, const int64_t* batch, const int32_t* sys_ptr,
                   const float* target, float target_offset, float* corr, int64_t N, int32_t K, int32_t C,
                   int32_t S, int32_t c0, int32_t c1, hipStream_t s) {
  const int32_t nch = c1 - c0;
  const int64_t row = (int64_t)K * C;
  if (!x || !out || !batch || !sys_ptr || (nch > 0 && !corr)) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(x) || !aligned16(out)) return set_error(FU_ERR_ALIGN, "%s: x/out not 16-byte aligned", who);
  if (nch > 0) {
    int W = 1;
    while (W < nch && W < 64) W <<= 1;
    hipLaunchKernelGGL(balance_sums_kernel, dim3(S), dim3(256), 0, s, x, sys_ptr, target, target_offset, corr, row,
                       c0, nch, W);
  }
  const int64_t n4 = N * row / 4;
  hipLaunchKernelGGL(balance_apply_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n4, 256), 8192)), dim3(256), 0, s, x,
                     batch, corr, out, n4, row, c0, nch);
  return check_launch(who);
}

int balance_check_shape(const char* who, int64_t N, int32_t K, int32_t C, int32_t S, int32_t c0, int32_t c1) {
  if (N < 0 || K <= 0 || C <= 0 || S <= 0 || c0 < 0 || c1 < c0 || c1 > C)
    return set_error(FU_ERR_SHAPE, "%s: bad shape (N=%lld K=%d C=%d S=%d range [%d, %d))", who, (long long)N, K, C,
                     S, c0, c1);
  if (((int64_t)K * C) % 4 != 0)
    return set_error(FU_ERR_SHAPE, "%s: K*C=%lld not a multiple of 4", who, (long long)K * C);
  return FU_OK;
}

// Scratch of the allocation-free entry point: the per-(system, channel) corrections.  One
// copy per GPU, held until the process ends; every call on a GPU reuses it.
constexpr int64_t kBalanceScratchFloats = FU_BALANCE_NOALLOC_MAX_CORR;
__device__ __align__(256) float scratch[kBalanceScratchFloats];

// Device address of `scratch` on each GPU, looked up once per device (with that device
// current) on the first call there.  The device is the one the launch stream belongs to
// (the null stream: the current device), so a caller whose current device is another one
// still gets the copy on the stream's GPU.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {nullptr};

int scratch_for_stream(hipStream_t stream, float** ptr) {
  const char* who = "fu_balance_channels_noalloc";
  int dev = -1;
  const hipError_t ge = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(FU_ERR_LAUNCH, "%s: cannot find the stream's HIP device (or device id >= %d)", who, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return set_error(FU_ERR_LAUNCH, "%s: no current HIP device", who);
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return set_error(FU_ERR_LAUNCH, "%s: cannot make device %d current", who, dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return set_error(FU_ERR_LAUNCH, "%s: hipGetSymbolAddress failed on device %d: %s", who, dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_ptr[dev];
  return FU_OK;
}

}  // namespace

extern "C" int fu_balance_channels(const float* x, float* out, const int64_t* batch, const int32_t* sys_ptr,
                                   const float* target, float target_offset, float* corr, int64_t corr_len,
                                   int64_t N, int32_t K, int32_t C, int32_t S, int32_t c0, int32_t c1,
                                   void* stream) {
  const char* who = "fu_balance_channels";
  int st = balance_check_shape(who, N, K, C, S, c0, c1);
  if (st != FU_OK) return st;
  if (corr_len < (int64_t)S * (c1 - c0))
    return set_error(FU_ERR_WORKSPACE, "%s: corr workspace needs %lld floats", who, (long long)S * (c1 - c0));
  if (N == 0) return FU_OK;
  return balance_launch(who, x, out, batch, sys_ptr, target, target_offset, corr, N, K, C, S, c0, c1,
                        as_stream(stream));
}

extern "C" int fu_balance_channels_noalloc(const float* x, float* out, const int64_t* batch, const int32_t* sys_ptr,
                                           const float* target, float target_offset, int64_t N, int32_t K,
                                           int32_t C, int32_t S, int32_t c0, int32_t c1, void* stream) {
  const char* who = "fu_balance_channels_noalloc";
  int st = balance_check_shape(who, N, K, C, S, c0, c1);
  if (st != FU_OK) return st;
  if ((int64_t)S * (c1 - c0) > kBalanceScratchFloats)
    return set_error(FU_ERR_WORKSPACE, "%s: S * (c1 - c0) = %lld exceeds the built-in scratch of %lld floats", who,
                     (long long)S * (c1 - c0), (long long)kBalanceScratchFloats);
  if (N == 0) return FU_OK;
  float* corr = nullptr;
  st = scratch_for_stream(as_stream(stream), &corr);
  if (st != FU_OK) return st;
  return balance_launch(who, x, out, batch, sys_ptr, target, target_offset, corr, N, K, C, S, c0, c1,
                        as_stream(stream));
}
