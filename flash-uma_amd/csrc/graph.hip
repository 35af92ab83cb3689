// Integer graph preprocessing on the GPU (model.py:17-74): Morton sort keys, a stable
// radix sort of (key, value) pairs, permutation inversion, index remapping and the CSR row
// pointer of a sorted key array.  All results are bit-exact functions of the inputs.
#include <string.h>
#include <rocprim/rocprim.hpp>

#include "fu_common.h"

namespace fu {

// Spread the low 10 bits of v so that bit k lands on bit 3k.  The key places the x, y, z cell
// indices at 3k + 1, 3k + 2, 3k + 3, as the reference's helpers do (their spread has a fifth
// step that lifts bit 3k to 3k + 1, model.py:48-58), so keys equal the reference's bit for bit.
__device__ __forceinline__ int64_t spread3(int64_t v) {
  v &= 0x3ff;
  int64_t r = 0;
#pragma unroll
  for (int k = 0; k < 10; ++k) r |= ((v >> k) & 1) << (3 * k);
  return r;
}

// One workgroup: min/max of the positions, then one key per atom.  The quantisation uses
// the reference's fp32 operations: scale = 1023 / max(max - min, 1e-5),
// q = int32((pos - min) * scale)  (model.py:61-64).
__global__ __launch_bounds__(1024) void morton_keys_kernel(const float* __restrict__ pos,
                                                           const int64_t* __restrict__ batch,
                                                           int64_t* __restrict__ keys, int64_t N) {
  __shared__ float smin[3][1024], smax[3][1024];
  const int t = threadIdx.x;
  float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
  for (int64_t n = t; n < N; n += blockDim.x) {
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const float v = pos[3 * n + d];
      mn[d] = fminf(mn[d], v);
      mx[d] = fmaxf(mx[d], v);
    }
  }
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    smin[d][t] = mn[d];
    smax[d][t] = mx[d];
  }
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (t < s) {
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        smin[d][t] = fminf(smin[d][t], smin[d][t + s]);
        smax[d][t] = fmaxf(smax[d][t], smax[d][t + s]);
      }
    }
    __syncthreads();
  }
  float lo[3], scale[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    lo[d] = smin[d][0];
    const float rng = fmaxf(smax[d][0] - lo[d], 1e-5f);
    scale[d] = 1023.0f / rng;
  }
  for (int64_t n = t; n < N; n += blockDim.x) {
    int64_t code = 0;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const float sub = __fsub_rn(pos[3 * n + d], lo[d]);
      const int q = (int)__fmul_rn(sub, scale[d]);
      code |= spread3(q) << (d + 1);
    }
    keys[n] = code | (batch[n] << 32);
  }
}

__global__ void invert_perm_kernel(const int64_t* __restrict__ perm, int64_t* __restrict__ inv, int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
    inv[perm[k]] = k;
}

__global__ void take_i64_kernel(const int64_t* __restrict__ table, const int64_t* __restrict__ idx,
                                int64_t* __restrict__ out, int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
    out[k] = table[idx[k]];
}

// row_ptr[v] = number of keys < v (first position of key v in the sorted array).
__global__ void csr_row_ptr_kernel(const int64_t* __restrict__ keys, int64_t E, int32_t* __restrict__ row_ptr,
                                   int64_t N) {
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v <= N; v += (int64_t)gridDim.x * blockDim.x) {
    int64_t lo = 0, hi = E;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (keys[mid] < v) lo = mid + 1;
      else hi = mid;
    }
    row_ptr[v] = (int32_t)lo;
  }
}

__global__ void narrow_kernel(const int64_t* __restrict__ in, int32_t* __restrict__ out, int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
    out[k] = (int32_t)in[k];
}

static unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>(std::max<int64_t>(cdiv(n, 256), 1), 65536); }

}  // namespace fu

using namespace fu;

extern "C" int fu_morton_keys(const float* pos, const int64_t* batch, int64_t* keys, int64_t N, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_morton_keys: bad shape");
  if (N == 0) return FU_OK;
  if (!pos || !batch || !keys) return set_error(FU_ERR_NULL, "fu_morton_keys: NULL argument");
  hipLaunchKernelGGL(morton_keys_kernel, dim3(1), dim3(1024), 0, as_stream(stream), pos, batch, keys, N);
  return check_launch("fu_morton_keys");
}

extern "C" int fu_sort_pairs_i64(const int64_t* keys_in, int64_t* keys_out, const int64_t* vals_in, int64_t* vals_out,
                                 int64_t n, int32_t begin_bit, int32_t end_bit, void* workspace, size_t* ws_bytes,
                                 void* stream) {
  if (n < 0 || begin_bit < 0 || end_bit > 64 || begin_bit >= end_bit)
    return set_error(FU_ERR_SHAPE, "fu_sort_pairs_i64: bad arguments");
  if (!ws_bytes) return set_error(FU_ERR_NULL, "fu_sort_pairs_i64: ws_bytes is NULL");
  // the radix sort orders keys as unsigned integers; callers pass non-negative keys
  const uint64_t* kin = reinterpret_cast<const uint64_t*>(keys_in);
  uint64_t* kout = reinterpret_cast<uint64_t*>(keys_out);
  size_t need = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, need, kin, kout, vals_in, vals_out, (size_t)n,
                                           (unsigned)begin_bit, (unsigned)end_bit, as_stream(stream));
  if (e != hipSuccess) return set_error(FU_ERR_LAUNCH, "fu_sort_pairs_i64: size query failed: %s", hipGetErrorString(e));
  if (workspace == nullptr) {
    *ws_bytes = need;
    return FU_OK;
  }
  if (*ws_bytes < need)
    return set_error(FU_ERR_WORKSPACE, "fu_sort_pairs_i64: workspace %zu < %zu bytes", *ws_bytes, need);
  if (n == 0) return FU_OK;
  if (!keys_in || !keys_out || !vals_in || !vals_out) return set_error(FU_ERR_NULL, "fu_sort_pairs_i64: NULL array");
  e = rocprim::radix_sort_pairs(workspace, need, kin, kout, vals_in, vals_out, (size_t)n, (unsigned)begin_bit,
                                (unsigned)end_bit, as_stream(stream));
  if (e != hipSuccess) return set_error(FU_ERR_LAUNCH, "fu_sort_pairs_i64: sort failed: %s", hipGetErrorString(e));
  return check_launch("fu_sort_pairs_i64");
}

extern "C" int fu_invert_perm(const int64_t* perm, int64_t* inv, int64_t n, void* stream) {
  if (n < 0) return set_error(FU_ERR_SHAPE, "fu_invert_perm: bad shape");
  if (n == 0) return FU_OK;
  if (!perm || !inv) return set_error(FU_ERR_NULL, "fu_invert_perm: NULL argument");
  hipLaunchKernelGGL(invert_perm_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), perm, inv, n);
  return check_launch("fu_invert_perm");
}

extern "C" int fu_take_i64(const int64_t* table, int64_t table_len, const int64_t* idx, int64_t* out, int64_t n,
                           void* stream) {
  if (n < 0 || table_len < 0) return set_error(FU_ERR_SHAPE, "fu_take_i64: bad shape");
  if (n == 0) return FU_OK;
  if (!table || !idx || !out) return set_error(FU_ERR_NULL, "fu_take_i64: NULL argument");
  hipLaunchKernelGGL(take_i64_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), table, idx, out, n);
  return check_launch("fu_take_i64");
}

extern "C" int fu_csr_row_ptr(const int64_t* sorted_keys, int64_t E, int32_t* row_ptr, int64_t N, void* stream) {
  if (E < 0 || N < 0 || E > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_csr_row_ptr: bad shape");
  if (!row_ptr || (E > 0 && !sorted_keys)) return set_error(FU_ERR_NULL, "fu_csr_row_ptr: NULL argument");
  hipLaunchKernelGGL(csr_row_ptr_kernel, dim3(grid_for(N + 1)), dim3(256), 0, as_stream(stream), sorted_keys, E,
                     row_ptr, N);
  return check_launch("fu_csr_row_ptr");
}

extern "C" int fu_narrow_i64_i32(const int64_t* in, int32_t* out, int64_t n, void* stream) {
  if (n < 0) return set_error(FU_ERR_SHAPE, "fu_narrow_i64_i32: bad shape");
  if (n == 0) return FU_OK;
  if (!in || !out) return set_error(FU_ERR_NULL, "fu_narrow_i64_i32: NULL argument");
  hipLaunchKernelGGL(narrow_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), in, out, n);
  return check_launch("fu_narrow_i64_i32");
}
