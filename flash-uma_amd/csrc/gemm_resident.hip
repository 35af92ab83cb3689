// Y[M, N] = A[M, K] @ W[N, K]^T + bias for short K (16 <= K <= 128, K % 16 == 0) and wide N,
// in the split-fp16 form of split_f16.h, with each workgroup's A panel resident in LDS.
//
// The model's radial output layers (model.py:149, 205: rad = h2 W3^T + b3, K = C = 128,
// N = 6 lmax C = 1,536 at lmax 2) are the case: the tiled kernel of gemm.hip reads and splits
// every 128-row A panel once per 128-column tile (12 times), splits the weight tile again in
// every workgroup, and stages both through LDS each 16-wide chunk.  Here a workgroup
//  * loads its 128 rows of A once, takes each row's exact scale from the whole row (pass 1 of
//    split_f16.h: no first-chunk guess, no overflow), applies the window rule of split_f16.h
//    against the weight's precomputed column flags, and writes the fp16 planes of all K chunks
//    into LDS (64 KB at K = 128: two workgroups per CU); a panel that the rule sends to pass 2
//    holds the 2^11-scaled residual planes instead and runs the two K loops;
//  * then walks every 128-column tile of the output: 4 waves in a 2 x 2 grid, each 64 x 64 =
//    2 x 2 blocks of 32 x 32, the weight's fragments loaded from global memory (L2: the split
//    weight is 1.2 MB at 1,536 x 128) straight into registers in MFMA-fragment order, the A
//    fragments read from the resident planes, no barrier inside the loop;
//  * stages its accumulators through a private LDS slice of 8 rows x 64 columns and writes
//    them back as 16-byte row pieces, unscaled (exact powers of two) and with the bias, with
//    nontemporal stores (the outputs are read once, by a later kernel); the 4-byte stores of
//    the accumulator layout (two 128-byte row pieces per instruction) held the kernel at
//    2.8 TB/s of output.
#include "resident_panel.h"

namespace fu {

constexpr int RBM = kResRows;     // rows per workgroup
constexpr int RKC_MAX = 8;        // 16-wide K chunks: K <= 128
constexpr int RPLANE = kResPlane;  // fp16 per plane (one chunk of the panel)
constexpr int RES = 64 + 8;       // floats per row of a wave's epilogue slice: 4 RES = 32 mod 64 banks

// The pre-split weight's layout: split_f16.h (resident_frag_vectors, resident_cols).

__global__ void resident_weight_scale_kernel(const float* __restrict__ W, int64_t ldw, int32_t N, int32_t K,
                                             float* __restrict__ cinv, int* __restrict__ flag) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= resident_cols(N)) return;
  float m = 0.0f;
  if (n < N)
    for (int k = 0; k < K; ++k) m = fmaxf(m, fabsf(W[(int64_t)n * ldw + k]));
  const int e = f16_exp_row(m);
  cinv[n] = pow2i(-e);
  bool low = false;
  float pmin = m, pmax = 0.0f;
  if (n < N)
    for (int k0 = 0; k0 < K; k0 += 8) {
      float mp = 0.0f;
      for (int k = k0; k < k0 + 8; ++k) mp = fmaxf(mp, fabsf(W[(int64_t)n * ldw + k]));
      low = low || f16_lossy(mp * pow2i(e));
      pmin = fminf(pmin, mp);
      pmax = fmaxf(pmax, mp);
    }
  flag[n] = (low ? 1 : 0) | (f16_flat(pmin, pmax) ? 0 : 2);
}

// One workgroup ORs the column flags into the summary word.
__global__ __launch_bounds__(256) void resident_weight_summary_kernel(const int* __restrict__ flag, int64_t ncols,
                                                                      int* __restrict__ summary) {
  __shared__ int s_or[4];
  int v = 0;
  for (int64_t n = threadIdx.x; n < ncols; n += 256) v |= flag[n];
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) v |= __shfl_xor(v, s);
  if ((threadIdx.x & 63) == 0) s_or[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) *summary = s_or[0] | s_or[1] | s_or[2] | s_or[3];
}

// One thread per (32-column block, chunk, lane): the lane's 8 consecutive k of one column,
// zero past N.
__global__ void resident_weight_split_kernel(const float* __restrict__ W, int64_t ldw, int32_t N, int32_t K,
                                             const float* __restrict__ cinv, uint4* __restrict__ W2) {
  const int nkc = K / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= resident_frag_vectors(N, K) / 3) return;
  const int lane = (int)(t & 63);
  const int64_t q = t >> 6;  // (block, chunk)
  const int n = (int)(q / nkc) * 32 + (lane & 31);
  const int k0 = (int)(q % nkc) * 16 + (lane >> 5) * 8;
  const float sc = 1.0f / cinv[n];  // an exact power of two
  float v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = n < N ? W[(int64_t)n * ldw + k0 + u] * sc : 0.0f;
  const float4 v0 = make_float4(v[0], v[1], v[2], v[3]), v1 = make_float4(v[4], v[5], v[6], v[7]);
  uint4* o = W2 + q * 3 * 64 + lane;
  uint4 h, l;
  split2h(v0, v1, h, l);
  o[0] = h;
  o[64] = l;
  split2h_up(v0, v1, h, l);
  o[128] = l;
}

template <int KC, bool VEC>
__global__ __launch_bounds__(256, 2) void linear_resident_kernel(const float* __restrict__ A, int64_t lda,
                                                                 const uint4* __restrict__ W2,
                                                                 const float* __restrict__ cinv,
                                                                 const int* __restrict__ wsum,
                                                                 const float* __restrict__ bias, float* __restrict__ Y,
                                                                 int64_t ldy, int64_t M, int32_t N) {
  __shared__ __attribute__((aligned(16))) __bf16 sp[KC * 2 * RPLANE];  // [chunk][hi, lo or lo'][plane]
  __shared__ float s_rinv[RBM];
  __shared__ unsigned s_need[4];
  __shared__ __attribute__((aligned(16))) float s_ep[4][8 * RES];  // one slice per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * RBM;

  const bool need2 = resident_panel<KC>(A, lda, wsum, sp, s_rinv, s_need, row0, M);

  // ---- every 128-column tile of the output
  const int fr = lane & 31, fh = lane >> 5;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int nb = (N + 31) / 32;
  const int ntiles = (N + 127) / 128;
  const uint4* wf = W2 + lane;
  for (int nt = 0; nt < ntiles; ++nt) {
    int cb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int b = (nt * 128 + wc) / 32 + j;
      cb[j] = b < nb ? b : nb - 1;  // a block past N reads the last one; nothing of it is stored
    }
    floatx16 acc[2][2];
    resident_tile<KC, 2, 2, KC>(sp, wf, cb, acc, need2, wr, fr, fh);
    // epilogue, 8 rows at a time: lane (fr, fh) holds column fr of each block and rows
    // 8 (t / 4) + 4 fh + t % 4; it stages them in its wave's slice, then reads back 4 consecutive
    // columns (c4 = lane % 16) of rows lane / 16 and lane / 16 + 4 for 16-byte stores (VEC), or
    // column fr of rows 4 fh .. 4 fh + 3 as single floats
    float* ep = s_ep[wave];
    const int colv = nt * 128 + wc + 4 * (lane & 15);
    float4 cs4 = make_float4(0.f, 0.f, 0.f, 0.f), bv4 = cs4;
    if constexpr (VEC) {
      if (colv < N) {
        cs4 = ld4(cinv + colv);
        if (bias) bv4 = ld4(bias + colv);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g8 = 0; g8 < 4; ++g8) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int t = 0; t < 4; ++t) ep[(4 * fh + t) * RES + 32 * j + fr] = acc[i][j][4 * g8 + t];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int rb = wr + 32 * i + 8 * g8;  // first row of the slice in the panel
        if constexpr (VEC) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int rr = (lane >> 4) + 4 * u;
            const int64_t gr = row0 + rb + rr;
            if (gr < M && colv < N) {
              const float rf = s_rinv[rb + rr];
              const float4 a4 = ld4(ep + rr * RES + 4 * (lane & 15));
              st4_nt(Y + gr * ldy + colv, make_float4(a4.x * rf * cs4.x + bv4.x, a4.y * rf * cs4.y + bv4.y,
                                                     a4.z * rf * cs4.z + bv4.z, a4.w * rf * cs4.w + bv4.w));
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int col = nt * 128 + wc + 32 * j + fr;
            if (col < N) {
              const float cs = cinv[col];
              const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const int rr = 4 * fh + t;
                const int64_t gr = row0 + rb + rr;
                if (gr < M) __builtin_nontemporal_store(ep[rr * RES + 32 * j + fr] * s_rinv[rb + rr] * cs + bv,
                                                        Y + gr * ldy + col);
              }
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
  }
}

extern "C" int64_t fu_linear_weight_split_bytes(int32_t N, int32_t K) {
  if (N <= 0 || K < 16 || K % 16 != 0)
    return set_error(FU_ERR_SHAPE, "fu_linear_weight_split_bytes: N=%d K=%d (K a positive multiple of 16)", N, K);
  return resident_frag_vectors(N, K) * 16 + resident_cols(N) * 8 + 16;
}

extern "C" int fu_linear_weight_split(const float* W, int64_t ldw, int32_t N, int32_t K, void* W2, void* stream) {
  const char* who = "fu_linear_weight_split";
  if (N <= 0 || K < 16 || K % 16 != 0 || ldw < K)
    return set_error(FU_ERR_SHAPE, "%s: N=%d K=%d ldw=%lld (K a positive multiple of 16)", who, N, K, (long long)ldw);
  if (!W || !W2) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(W2)) return set_error(FU_ERR_ALIGN, "%s: W2 must be 16-byte aligned", who);
  uint4* w2 = static_cast<uint4*>(W2);
  float* cinv = reinterpret_cast<float*>(w2 + resident_frag_vectors(N, K));
  int* flag = reinterpret_cast<int*>(cinv + resident_cols(N));
  int* summary = flag + resident_cols(N);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(resident_weight_scale_kernel, dim3(cdiv(resident_cols(N), 256)), dim3(256), 0, s, W, ldw, N, K,
                     cinv, flag);
  hipLaunchKernelGGL(resident_weight_summary_kernel, dim3(1), dim3(256), 0, s, flag, resident_cols(N), summary);
  hipLaunchKernelGGL(resident_weight_split_kernel, dim3(cdiv(resident_frag_vectors(N, K) / 3, 256)), dim3(256), 0, s,
                     W, ldw, N, K, cinv, w2);
  return check_launch(who);
}

extern "C" int fu_linear_resident(const float* A, int64_t lda, const void* W2, const float* bias, float* Y, int64_t ldy,
                                  int64_t M, int32_t N, int32_t K, void* stream) {
  const char* who = "fu_linear_resident";
  if (M < 0 || N <= 0 || K < 16 || K > 16 * RKC_MAX || K % 16 != 0 || lda < K || ldy < N)
    return set_error(FU_ERR_SHAPE, "%s: M=%lld N=%d K=%d lda=%lld ldy=%lld (16 <= K <= 128, K %% 16 == 0)", who,
                     (long long)M, N, K, (long long)lda, (long long)ldy);
  if (M == 0) return FU_OK;
  if (!A || !W2 || !Y) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(A) || lda % 4 != 0 || !aligned16(W2))
    return set_error(FU_ERR_ALIGN, "%s: A and W2 must be 16-byte aligned and lda a multiple of 4", who);
  const uint4* w2 = static_cast<const uint4*>(W2);
  const float* cinv = reinterpret_cast<const float*>(w2 + resident_frag_vectors(N, K));
  const int* summary = reinterpret_cast<const int*>(cinv + resident_cols(N)) + resident_cols(N);
  const dim3 grid(cdiv(M, RBM)), block(256);
  hipStream_t s = as_stream(stream);
  // 16-byte output pieces when every row and column group of 4 is aligned
  const bool vec = N % 4 == 0 && ldy % 4 == 0 && aligned16(Y) && (!bias || aligned16(bias));
  switch (K / 16) {
#define FU_RES_CASE(kc)                                                                                            \
  case kc:                                                                                                         \
    if (vec)                                                                                                       \
      hipLaunchKernelGGL((linear_resident_kernel<kc, true>), grid, block, 0, s, A, lda, w2, cinv, summary, bias, Y, \
                         ldy, M, N);                                                                               \
    else                                                                                                           \
      hipLaunchKernelGGL((linear_resident_kernel<kc, false>), grid, block, 0, s, A, lda, w2, cinv, summary, bias,  \
                         Y, ldy, M, N);                                                                            \
    break;
    FU_RES_CASE(1) FU_RES_CASE(2) FU_RES_CASE(3) FU_RES_CASE(4) FU_RES_CASE(5) FU_RES_CASE(6) FU_RES_CASE(7)
    FU_RES_CASE(8)
#undef FU_RES_CASE
  }
  return check_launch(who);
}

}  // namespace fu
