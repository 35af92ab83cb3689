// Dense fp32 contractions on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Y[M, N] = A[M, K] @ W[N, K]^T (+ bias[N]).  Both operands are K-contiguous, so one kernel
// serves the SO(2) conv1/conv2 forward (W = packed weight, model.py:152,154), the radial-MLP
// linears (model.py:147-149) and every input-gradient GEMM of the backward pass (W = the
// pre-transposed weight).  No weight gradients are ever needed: parameters are frozen.
//
// Tiling: a 256-thread workgroup (4 wave64s in a 2x2 grid) owns a 128x128 output tile; each
// wave owns 64x64 = 2x2 MFMA blocks of 32x32 (64 fp32 accumulators per lane).  K advances in
// chunks of 32 staged through double-buffered LDS.  Within a chunk, lane l (row/col l%32,
// half h = l/32) feeds the MFMA k-slot h with chunk column 16h + t at step t, so each lane
// reads its 16 operands of a chunk with four 16-byte LDS reads.
#include "fu_common.h"

namespace fu {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 32;
constexpr int GLDS = GBK + 4;  // padded LDS row (floats) to spread banks

__global__ __launch_bounds__(256) void linear_mfma_kernel(const float* __restrict__ A, int64_t lda,
                                                          const float* __restrict__ W, int64_t ldw,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ Y, int64_t ldy,
                                                          int64_t M, int32_t N, int32_t K,
                                                          int32_t n_tiles, int64_t total_tiles) {
  __shared__ __attribute__((aligned(16))) float As[2][GBM * GLDS];
  __shared__ __attribute__((aligned(16))) float Bs[2][GBN * GLDS];

  // XCD-aware tile order: hardware deals consecutive workgroups round-robin over the 8 XCDs;
  // remap so that each XCD walks a contiguous range of tiles (tiles sharing an A row-panel
  // then share that XCD's L2).
  int64_t wg = blockIdx.x;
  if ((total_tiles & 7) == 0) wg = (wg & 7) * (total_tiles >> 3) + (wg >> 3);
  const int64_t m_tile = wg / n_tiles;
  const int n_tile = (int)(wg - m_tile * n_tiles);
  const int64_t row0 = m_tile * GBM;
  const int col0 = n_tile * GBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = (wave >> 1) * 64;  // wave's row offset inside the tile
  const int wc = (wave & 1) * 64;   // wave's col offset inside the tile

  // Global -> register staging: 4 float4 of A and 4 float4 of W per thread per chunk.
  float4 ra[4], rb[4];
  auto load_chunk = [&](int k0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int lin = tid + 256 * p;
      const int r = lin >> 3;
      const int kc = (lin & 7) * 4;
      const int64_t gr = row0 + r;
      const int gk = k0 + kc;
      ra[p] = (gr < M && gk < K) ? ld4(A + gr * lda + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
      const int gn = col0 + r;
      rb[p] = (gn < N && gk < K) ? ld4(W + (int64_t)gn * ldw + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int lin = tid + 256 * p;
      const int r = lin >> 3;
      const int kc = (lin & 7) * 4;
      st4(&As[buf][r * GLDS + kc], ra[p]);
      st4(&Bs[buf][r * GLDS + kc], rb[p]);
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (K + GBK - 1) / GBK;
  load_chunk(0);
  store_chunk(0);
  __syncthreads();

  const int fr = lane & 31;        // operand row (A) / column (W) within a 32-block
  const int fk = (lane >> 5) * 16;  // first chunk column this lane feeds

  for (int kc = 0; kc < nk; ++kc) {
    const int buf = kc & 1;
    if (kc + 1 < nk) load_chunk((kc + 1) * GBK);

    float af[2][16], bf[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float* pa = &As[buf][(wr + i * 32 + fr) * GLDS + fk];
      const float* pb = &Bs[buf][(wc + i * 32 + fr) * GLDS + fk];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 va = ld4(pa + 4 * q);
        const float4 vb = ld4(pb + 4 * q);
        af[i][4 * q + 0] = va.x; af[i][4 * q + 1] = va.y; af[i][4 * q + 2] = va.z; af[i][4 * q + 3] = va.w;
        bf[i][4 * q + 0] = vb.x; bf[i][4 * q + 1] = vb.y; bf[i][4 * q + 2] = vb.z; bf[i][4 * q + 3] = vb.w;
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][t], bf[j][t], acc[i][j], 0, 0, 0);
    }

    if (kc + 1 < nk) {
      store_chunk(buf ^ 1);
    }
    __syncthreads();
  }

  // Accumulator layout of the 32x32 MFMA: lane l, register r -> column l%32,
  // row 8*(r/4) + 4*(l/32) + r%4.
  const int oc = lane & 31;
  const int orow = (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int gc = col0 + wc + j * 32 + oc;
    if (gc >= N) continue;
    const float bv = bias ? bias[gc] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = row0 + wr + i * 32 + 8 * (r >> 2) + orow + (r & 3);
        if (gr < M) Y[gr * ldy + gc] = acc[i][j][r] + bv;
      }
    }
  }
}

}  // namespace fu

using namespace fu;

extern "C" int fu_linear(const float* A, int64_t lda, const float* W, int64_t ldw, const float* bias,
                         float* Y, int64_t ldy, int64_t M, int32_t N, int32_t K, void* stream) {
  if (M < 0 || N <= 0 || K <= 0)
    return set_error(FU_ERR_SHAPE, "fu_linear: bad shape M=%lld N=%d K=%d", (long long)M, N, K);
  if (K % 4 != 0 || lda % 4 != 0 || ldw % 4 != 0)
    return set_error(FU_ERR_UNSUPPORTED, "fu_linear: K=%d, lda=%lld, ldw=%lld must be multiples of 4",
                     K, (long long)lda, (long long)ldw);
  if (lda < K || ldw < K || ldy < N)
    return set_error(FU_ERR_SHAPE, "fu_linear: leading dimensions smaller than the rows");
  if (!A || !W || !Y) return set_error(FU_ERR_NULL, "fu_linear: NULL operand");
  if (!aligned16(A) || !aligned16(W)) return set_error(FU_ERR_ALIGN, "fu_linear: operands must be 16-byte aligned");
  if (M == 0) return FU_OK;
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t m_tiles = (M + GBM - 1) / GBM;
  const int64_t total = m_tiles * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_linear: M too large");
  hipLaunchKernelGGL(linear_mfma_kernel, dim3((unsigned)total), dim3(256), 0, as_stream(stream), A, lda,
                     W, ldw, bias, Y, ldy, M, N, K, n_tiles, total);
  return check_launch("fu_linear");
}
