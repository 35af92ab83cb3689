// Complex dense layer on the matrix cores.
//
// The SO(2) m = 1 and m = 2 convolutions of eSCN apply a complex weight R + iI to complex
// features x_r + i x_i.  The reference packs them into one real GEMM against
// [[R, -I], [I, R]] (model.py:108-138), which costs four real products.  This kernel computes
//     T1 = a_r P^T,  T2 = a_i Q^T,  T3 = (a_r + a_i)(P + Q)^T
//     out_r = T1 - T2,  out_i = T3 - T1 - T2
// i.e. out_r = a_r P^T - a_i Q^T and out_i = a_r Q^T + a_i P^T with three products: 25 % fewer
// MFMA flops for the same result up to fp32 rounding.  The sums a_r + a_i and P + Q are
// formed in registers from the operands already staged in LDS, so no extra memory traffic.
//
// K advances in chunks of 16 through double-buffered LDS.  Four main loops:
//  * split fp16 with a pre-split weight (the default matrix-core mode, with W3): as the bf16
//    form below, with two fp16 planes per operand (split_f16.h).  The weight's planes hold
//    its columns scaled by one power of two per output column (shared by P, Q and S, so the
//    three products stay combinable), computed when the weight is split; a row of
//    (a_r, a_i, a_s) gets one scale from its first chunk (or, for Kc <= 64, from a pre-pass),
//    with a second pass of the tile at exact scales if a row leaves the window.  Three MFMAs
//    per product and 32-row block instead of six; 24 KB of A planes per buffer.
//  * split bf16 with a pre-split weight (mode 0 when the caller passes W3, built once per
//    frozen weight by fu_complex_weight_split): P, Q and S = P + Q are stored as bf16 planes
//    in MFMA-fragment order ([32-column block][16-k chunk][P, Q, S][hi, mid, lo][lane], 16 B
//    per lane), so each wave loads its B fragments with 1 KB coalesced loads straight into
//    registers, one chunk ahead.  Only a_r, a_i and a_s = a_r + a_i are split in the kernel
//    and staged as planes in LDS (36 KB per buffer).  The output tile is 128 rows x 128
//    columns of both out_r and out_i, computed by 512 threads (8 waves, two per SIMD, one
//    workgroup per CU): wave (h, b) owns rows 64 h .. 64 h + 63 of 32-column block b (two
//    32-row blocks x T1, T2, T3: six accumulator chains, 96 registers), so every staged A
//    chunk feeds eight waves.  Measured on the model's shapes:
//      - against 64 x 32 per wave in 128 x 64 tiles (two workgroups of 4 waves per CU),
//        one 128 x 128 tile per CU halves the global loads per MFMA: 1.08-1.13x faster
//        (fetching the operands, not the MFMAs, was the limit: the same kernel without its
//        B loads, or without its A loads, ran 1.25-1.35x faster);
//      - against four waves of 128 rows each (12 chains, 192 accumulators, one wave per
//        SIMD), the second wave on each SIMD issues while the first waits on its LDS reads
//        and the chunk barrier: 1.01-1.10x faster, at the cost of loading each B fragment
//        twice (once per row half; the second load mostly hits the L1).
//  The two loops below use 256 threads and an output tile of 128 rows x 64 columns (2 x 2
//  waves of 64 x 32):
//  * split bf16 without W3: a_r, a_i, P and Q are all split as they are staged (36 KB of
//    planes per buffer); planes of a_r + a_i and P + Q as well would not fit two workgroups
//    per CU, so this loop runs the four products directly,
//        out_r = a_r P^T + a_i (-Q)^T,  out_i = a_r Q^T + a_i P^T,
//    with -Q formed by flipping the sign bits of the Q planes in registers (four chains).
//  * fp32 (fu_set_matmul_mode(1)): the three products on v_mfma_f32_32x32x2_f32, fp32 LDS
//    rows as in the real GEMM (a_r, a_i: 128 rows; P, Q: 64 rows).
// The epilogue stages the outputs through LDS and writes 16-byte row pieces.
#include "split_f16.h"

namespace fu {

constexpr int CBM = 128, CBN = 64;
constexpr int CTA = CBM * 16, CTB = CBN * 16;
constexpr int CBN_PRE = 128;  // output columns per tile of the pre-split path
constexpr int CBUF = 2 * CTA + 2 * CTB;          // fp32: a_r | a_i | P | Q
constexpr int CBUF_SPLIT = 6 * CTA + 6 * CTB;    // bf16: a_r, a_i planes (CTA each) | P, Q planes (CTB each)
constexpr int CBUF_PRE = 9 * CTA;                // bf16: a_r, a_i, a_s planes
constexpr int C_LDS_FLOATS = 2 * CBUF;
constexpr int C_LDS_FLOATS_SPLIT = CBUF_SPLIT;   // two buffers of bf16 = CBUF_SPLIT floats
static_assert(CBUF_PRE == CBUF_SPLIT, "both split loops use the same LDS size");

// Main loops of complex_linear_kernel.
enum { CPATH_FP32 = 0, CPATH_SPLIT4 = 1, CPATH_SPLIT3_PRE = 2, CPATH_F16_PRE = 3 };
constexpr bool pre_split(int path) { return path == CPATH_SPLIT3_PRE || path == CPATH_F16_PRE; }

// A pre-split complex weight holds, one after the other:
//  * bf16 planes in fragment order: per (32-column block, 16-k chunk), 9 x 64 lanes x 16 B
//    (P, Q, S = P + Q, each hi, mid, lo);
//  * fp16 planes in the same order: per (block, chunk), 9 x 64 lanes x 16 B: P hi, P lo, Q hi,
//    Q lo, S hi, S lo of the columns scaled by their power of two 2^e(n) (split_f16.h; one exact
//    scale per output column n, shared by P, Q and S so that the three products stay
//    combinable), then the lo' = 2^11 lo planes of P, Q and S (pass 2 of split_f16.h);
//  * the unscale factors 2^-e(n), one float per column of the 32-column blocks;
//  * one int per column of the 32-column blocks: bit 0 set when a piece of 8 consecutive k of
//    P or Q of that column is nonzero and below the window (2^-3) at the column's scale, bit 1
//    when the column is not flat (split_f16.h); the kernels' pass rules read them.
__host__ __device__ inline int64_t complex_weight_split_vectors(int32_t Nc, int32_t Kc) {
  return (int64_t)((Nc + 31) / 32) * ((Kc + 15) / 16) * 9 * 64;
}
__host__ __device__ inline int64_t complex_weight_f16_vectors(int32_t Nc, int32_t Kc) {
  return (int64_t)((Nc + 31) / 32) * ((Kc + 15) / 16) * 9 * 64;
}
__host__ __device__ inline int64_t complex_weight_scale_vectors(int32_t Nc) { return (int64_t)((Nc + 31) / 32) * 8; }

__device__ __forceinline__ int clds(int row, int chunk) {
  return row * 16 + 4 * (chunk ^ (((row >> 1) ^ (row >> 2)) & 3));
}

// Gate epilogues, s = sigmoid(gate) for gate-column index t = s_off + column (degree
// l = 1 + t / C, channel t % C), read from the gate-paired conv1 m = 0 output G = Y0:
// G[row][64 ((l - 1) C / 32 + c / 32) + c % 32] (fu_linear_gate's column order).
//   MODE 1 (conv1 m = 1, 2 fused with the gate activation): also writes Z_r = Y_r s, Z_i = Y_i s;
//   MODE 2 (conv2 m = 1, 2 input gradient fused with the gate backward): the product is
//   g_Z; Y receives g_Y = g_Z s and Pout the gate sum g_Zr F_r + g_Zi F_i, F being the
//   forward pre-activation of the same block.
struct CGate {
  float* Zr;
  float* Zi;
  int64_t ldz;
  const float* G;
  int64_t ldg;
  int32_t s_off;
  int32_t C;
  const float* Fr;
  const float* Fi;
  int64_t ldf;
  float* Pout;
  int64_t ldp;
};

// Output columns per tile, 32-row blocks per wave and workgroups per CU of each path.
constexpr int cbn_of(int path) { return pre_split(path) ? CBN_PRE : CBN; }
constexpr int wg_per_cu(int path) { return path == CPATH_FP32 ? 3 : pre_split(path) ? 1 : 2; }
constexpr int threads_of(int path) { return pre_split(path) ? 512 : 256; }

template <int MODE, int PATH, bool KTAIL = false>
__global__ __launch_bounds__(threads_of(PATH), wg_per_cu(PATH)) void complex_linear_kernel(
    const float* __restrict__ Ar, const float* __restrict__ Ai, int64_t lda, const float* __restrict__ P,
    const float* __restrict__ Q, int64_t ldw, const uint4* __restrict__ W3, float* __restrict__ Yr,
    float* __restrict__ Yi, int64_t ldy, int64_t M, int32_t Nc, int32_t Kc, int32_t n_tiles, int64_t total_tiles,
    CGate g) {
  constexpr bool SPLIT = PATH != CPATH_FP32;
  __shared__ __attribute__((aligned(16))) float smem[SPLIT ? C_LDS_FLOATS_SPLIT : C_LDS_FLOATS];
  // XCD-aware tile order, as in the real GEMM
  int64_t wg = blockIdx.x;
  if ((total_tiles & 7) == 0) wg = (wg & 7) * (total_tiles >> 3) + (wg >> 3);
  const int64_t m_tile = wg / n_tiles;
  const int n_tile = (int)(wg - m_tile * n_tiles);
  constexpr int RB = 2;  // 32-row blocks per wave
  const int64_t row0 = m_tile * CBM;
  const int col0 = n_tile * cbn_of(PATH);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // wave tile: RB 32-row blocks x one 32-column block (pre-split: 2 row halves x 4 column
  // blocks; otherwise 2 x 2)
  constexpr bool W8 = threads_of(PATH) == 512;
  const int wr = (wave >> (W8 ? 2 : 1)) * 64, wc = (wave & (W8 ? 3 : 1)) * 32;

  // four-product split: T[0] = out_r, T[1] = out_i; otherwise T1, T2, T3 of the three products
  constexpr int NT = PATH == CPATH_SPLIT4 ? 2 : 3;
  floatx16 T[NT][RB];
#pragma unroll
  for (int p = 0; p < NT; ++p)
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) T[p][i][r] = 0.0f;

  const int fr = lane & 31, fh = lane >> 5;
  if constexpr (pre_split(PATH)) {
    // [buf][a_r planes | a_i planes | a_s planes][CTA]: hi, mid, lo bf16, or hi, lo fp16 (F16,
    // the rows scaled by 2^e(row) as in split_f16.h)
    constexpr bool F16 = PATH == CPATH_F16_PRE;
    constexpr int NPL = F16 ? 2 : 3;     // planes per operand
    constexpr int NB = 3 * NPL;          // B fragments per chunk
    constexpr int BUF = 3 * NPL * CTA;   // bf16 per LDS buffer
    __bf16* sp = reinterpret_cast<__bf16*>(smem);
    // staging: thread -> tile row sr, k 4 sq .. 4 sq + 3 of the chunk (8-byte plane pieces)
    const int sr = tid >> 2, sq = tid & 3;
    const int soff = plane_off(sr, sq >> 1) + 4 * (sq & 1);
    const int nkc = (Kc + 15) / 16;
    const int nbt = (Nc + 31) / 32;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 gr, gi;
    // fixed row pointers (a row past M reads row M-1; its outputs are never stored).  Without a
    // K tail: plain 16-byte loads; with one (KTAIL): unconditional loads from a valid address
    // and selects zeroing the pieces at or past Kc.  No branch in the loader (an if/else
    // choosing the form per chunk was miscompiled here: a prefetched operand register reused
    // before its read).
    const int64_t row = row0 + sr;
    const int64_t ao = (row < M ? row : M - 1) * lda + 4 * sq;
    const float *par = Ar + ao, *pai = Ai + ao;
    auto load_chunk = [&](int k0) {
      if constexpr (!KTAIL) {
        gr = ld4(par + k0);
        gi = ld4(pai + k0);
      } else {  // Kc is a multiple of 4: a thread's 4 k are all in or all past Kc
        const bool ok = k0 + 4 * sq < Kc;
        const float4 r = ld4(ok ? par + k0 : Ar), i = ld4(ok ? pai + k0 : Ai);
        gr = ok ? r : z4;
        gi = ok ? i : z4;
      }
    };
    // F16: the row's scale, the running maximum of |a_r|, |a_i|, |a_s| (this thread's quarter)
    // and whether a piece staged in pass 0 fell below the window (split_f16.h)
    float sc = 1.0f, R = 0.0f, pmin = __builtin_huge_valf();
    int e = 0;
    bool lossy = false;
    auto chunk_max = [&]() { return fmaxf(fmaxf(amax4(gr), amax4(gi)), amax4(gr + gi)); };
    auto row_max = [&](float v) {  // over the row's four staging threads
      v = fmaxf(v, __shfl_xor(v, 1, 64));
      return fmaxf(v, __shfl_xor(v, 2, 64));
    };
    // ps: the pass kind (0: hi + lo planes, the pieces' window tracked; 1: hi and lo' = 2^11 lo
    // planes; 2: hi planes)
    auto store_chunk = [&](int buf, auto ps) {
      constexpr int PS = decltype(ps)::value;
      __bf16* b = sp + buf * BUF;
      if constexpr (F16) {
        auto put = [&](const float4& v, int plane) {
          uint2 h, l;
          if constexpr (PS == 0) split2h_4(v, h, l);
          else split2h_4_up(v, h, l);
          st_planes2_4(b + plane * CTA, CTA, soff, h, l);
        };
        const float4 vr = scale4(gr, sc), vi = scale4(gi, sc);
        if constexpr (PS == 0) {
          R = fmaxf(R, chunk_max());
          const float mr = amax4(vr), mi = amax4(vi);
          pmin = fminf(pmin, fminf(mr, mi));
          lossy |= f16_lossy(mr) || f16_lossy(mi);
        }
        put(vr, 0);
        put(vi, 2);
        put(scale4(gr + gi, sc), 4);
      } else {
        uint2 h, m, l;
        split3_4(gr, h, m, l);
        st_planes4(b, CTA, soff, h, m, l);
        split3_4(gi, h, m, l);
        st_planes4(b + 3 * CTA, CTA, soff, h, m, l);
        split3_4(gr + gi, h, m, l);
        st_planes4(b + 6 * CTA, CTA, soff, h, m, l);
      }
    };
    // this wave's B fragments of chunk kc (a column block past Nc reads block 0; its outputs
    // are never stored).  F16: per (block, chunk) the weight holds NBS vectors of 64 lanes, the
    // hi and lo planes of P, Q, S and then their lo' planes (pass kind 1 loads hi and lo').
    constexpr int NBS = F16 ? 9 : NB;
    const int nb_raw = (col0 + wc) / 32;
    const int nb = nb_raw < nbt ? nb_raw : 0;
    const uint4* wb = W3 + (int64_t)nb * nkc * NBS * 64 + lane;
    auto load_b = [&](int kc, uint4 (&bf)[NB], auto ps) {
      constexpr int PS = decltype(ps)::value;
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int v = (F16 && PS == 1 && (u & 1)) ? 6 + (u >> 1) : u;
        bf[u] = wb[(kc * NBS + v) * 64];
      }
    };
    auto step = [&](int kc, const uint4 (&bc)[NB], uint4 (&bn)[NB], auto ps) {
      constexpr int PS = decltype(ps)::value;
      constexpr int QB = PS == 2 ? 2 : 0, QE = PS == 1 ? 2 : 3;
      load_b(kc + 1 < nkc ? kc + 1 : nkc - 1, bn, ps);
      const __bf16* b = sp + (kc & 1) * BUF;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int off = plane_off(wr + 32 * i + fr, fh);
        if constexpr (F16) {
          f16x8 af[6];  // a_r, a_i, a_s planes
#pragma unroll
          for (int u = 0; u < 6; ++u) af[u] = *reinterpret_cast<const f16x8*>(b + u * CTA + off);
#pragma unroll
          for (int q = QB; q < QE; ++q)
#pragma unroll
            for (int op = 0; op < 3; ++op)
              T[op][i] = mfma_f16(af[2 * op + kF16A[q]], __builtin_bit_cast(f16x8, bc[2 * op + kF16B[q]]), T[op][i]);
        } else {
          bf16x8 af[9];  // a_r, a_i, a_s planes
#pragma unroll
          for (int u = 0; u < 9; ++u) af[u] = *reinterpret_cast<const bf16x8*>(b + u * CTA + off);
#pragma unroll
          for (int q = 0; q < 6; ++q)
#pragma unroll
            for (int op = 0; op < 3; ++op)
              T[op][i] = mfma_bf16(af[3 * op + kSplitA[q]], __builtin_bit_cast(bf16x8, bc[3 * op + kSplitB[q]]),
                                   T[op][i]);
        }
      }
      // chunk kc + 1 into the other buffer (its last readers finished before the previous
      // barrier), then prefetch chunk kc + 2
      store_chunk((kc & 1) ^ 1, ps);
      load_chunk((kc + 2 < nkc ? kc + 2 : nkc - 1) * 16);
      __syncthreads();
    };
    uint4 b0[NB], b1[NB];
    auto kloop = [&](auto ps) {
      load_chunk(0);
      store_chunk(0, ps);
      load_chunk((nkc > 1 ? 1 : 0) * 16);
      load_b(0, b0, ps);
      __syncthreads();
      // unrolled by two so that the fragment double buffer stays in fixed registers
      for (int kc = 0; kc < nkc; kc += 2) {
        step(kc, b0, b1, ps);
        if (kc + 1 < nkc) step(kc + 1, b1, b0, ps);
      }
    };
    if constexpr (!F16) {
      kloop(std::integral_constant<int, 0>{});
    } else {
      // The passes of split_f16.h.  Pass 0: scales from the rows' first chunk (rows of at most
      // F16_PREPASS_CHUNKS chunks skip it).  The tile is computed again at exact scales when a
      // row's running maximum overflowed, or when one operand has a piece below the window while
      // the other is not flat (the weight's columns carry both properties from
      // fu_complex_weight_split, at their exact scales); the exact scan applies the same rule at
      // its scales: pass 1 (one loop) or pass 2 (two loops).
      __shared__ unsigned f16_any[8];
      auto tile_bits = [&](unsigned v) {  // OR over the workgroup (every thread calls this)
        unsigned w = 0;
#pragma unroll
        for (int bit = 0; bit < 5; ++bit) w |= (__ballot((v >> bit) & 1u) != 0 ? 1u : 0u) << bit;
        __syncthreads();  // the previous call's readers are done with f16_any
        if (lane == 0) f16_any[wave] = w;
        __syncthreads();
        unsigned any = 0;
#pragma unroll
        for (int w8 = 0; w8 < 8; ++w8) any |= f16_any[w8];
        return any;
      };
      const float* cinv = reinterpret_cast<const float*>(W3 + complex_weight_f16_vectors(Nc, Kc));
      const int* cflag = reinterpret_cast<const int*>(cinv + nbt * 32);
      const int cf = nb_raw < nbt ? cflag[nb * 32 + fr] : 0;
      const unsigned wbits = tile_bits(((cf & 1) ? F16_LOW_W : 0u) | ((cf & 2) ? F16_ROUGH_W : 0u));
      // verdict bits of this thread's row (row-level over its four staging threads)
      auto verdict_a = [&](float pmn, float pmx, bool low) {
        pmn = fminf(pmn, __shfl_xor(pmn, 1, 64));
        pmn = fminf(pmn, __shfl_xor(pmn, 2, 64));
        return (low ? F16_LOW_A : 0u) | (f16_flat(pmn, row_max(pmx)) ? 0u : F16_ROUGH_A);
      };
      bool exact = nkc <= F16_PREPASS_CHUNKS;
      // one call site of the pass-0/1 loop (pass 0, or pass 1 after an exact scan); pass 2 has
      // its own two loops
      for (int pass = 0; pass < 2; ++pass) {
        if (!exact) {
          load_chunk(0);
          e = f16_exp_chunk(row_max(chunk_max()));
          sc = pow2i(e);
        } else {
          // exact scales from a pass over the rows, and the verdict at them
          const float inf = __builtin_huge_valf();
          float Rx = 0.0f, gmin = inf, zmin = inf;
#pragma unroll 4
          for (int kc = 0; kc < nkc; ++kc) {
            load_chunk(kc * 16);
            const float mr = amax4(gr), mi = amax4(gi);
            Rx = fmaxf(Rx, fmaxf(fmaxf(mr, mi), amax4(gr + gi)));
            zmin = fminf(zmin, fminf(mr, mi));
            gmin = fminf(gmin, fminf(mr > 0.0f ? mr : inf, mi > 0.0f ? mi : inf));
          }
          e = f16_exp_row(row_max(Rx));
          sc = pow2i(e);
          if (f16_needs_exact(tile_bits(verdict_a(zmin, Rx, f16_lossy(gmin * sc))) | wbits)) {
            kloop(std::integral_constant<int, 1>{});
#pragma unroll
            for (int p = 0; p < NT; ++p)
#pragma unroll
              for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) T[p][i][r] *= F16_LO_DOWN;
            kloop(std::integral_constant<int, 2>{});
            break;
          }
        }
        kloop(std::integral_constant<int, 0>{});
        if (exact) break;
        // every wave has left the loop (barrier in the last step): its buffers may be restaged
        const unsigned t = tile_bits(verdict_a(pmin, R * sc, lossy) |
                                     (f16_outside(row_max(R) * sc) ? F16_OVERFLOW : 0u)) | wbits;
        exact = (t & F16_OVERFLOW) != 0 || f16_needs_exact(t);
        if (!exact) break;
#pragma unroll
        for (int p = 0; p < NT; ++p)
#pragma unroll
          for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) T[p][i][r] = 0.0f;
      }
      // undo the scales: row factor from the staging threads, column factor from the weight
      __shared__ float f16_rinv[CBM];
      if (sq == 0) f16_rinv[sr] = pow2i(-e);
      __syncthreads();
      const float cs = cinv[nb * 32 + fr];
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float rs = f16_rinv[wr + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3)];
#pragma unroll
          for (int p = 0; p < NT; ++p) T[p][i][r] = T[p][i][r] * rs * cs;
        }
    }
  } else if constexpr (PATH == CPATH_SPLIT4) {
    // [buf][a_r hi, mid, lo | a_i hi, mid, lo (CTA each) | P hi, mid, lo | Q hi, mid, lo (CTB each)]
    __bf16* sp = reinterpret_cast<__bf16*>(smem);
    const int sr = tid >> 1, sh = tid & 1;                    // a_r, a_i: tile row sr, k 8 sh ..
    const int bq = tid >> 7, br = (tid & 127) >> 1, bh = tid & 1;  // P (bq 0) or Q (bq 1): row br, k 8 bh ..
    const int soff_a = plane_off(sr, sh), soff_b = plane_off(br, bh);
    const float* Bsrc = bq ? Q : P;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 gr[2], gi[2], gb[2];
    // fixed row pointers (a row past M / Nc reads the last row; its outputs are never
    // stored); K tail handled as in the pre-split path, without a branch in the loader
    const int64_t row = row0 + sr;
    const int64_t ao = (row < M ? row : M - 1) * lda + 8 * sh;
    const float *par = Ar + ao, *pai = Ai + ao;
    const int gn = col0 + br;
    const float* pb = Bsrc + (int64_t)(gn < Nc ? gn : Nc - 1) * ldw + 8 * bh;
    auto load_chunk = [&](int k0) {
      if constexpr (!KTAIL) {
        gr[0] = ld4(par + k0);
        gr[1] = ld4(par + k0 + 4);
        gi[0] = ld4(pai + k0);
        gi[1] = ld4(pai + k0 + 4);
        gb[0] = ld4(pb + k0);
        gb[1] = ld4(pb + k0 + 4);
      } else {
        const int gk = k0 + 8 * sh, gkb = k0 + 8 * bh;
        const bool a0 = gk < Kc, a1 = gk + 4 < Kc, b0 = gkb < Kc, b1 = gkb + 4 < Kc;
        const float4 r0 = ld4(a0 ? par + k0 : Ar), r1 = ld4(a1 ? par + k0 + 4 : Ar);
        const float4 i0 = ld4(a0 ? pai + k0 : Ai), i1 = ld4(a1 ? pai + k0 + 4 : Ai);
        const float4 w0 = ld4(b0 ? pb + k0 : Bsrc), w1 = ld4(b1 ? pb + k0 + 4 : Bsrc);
        gr[0] = a0 ? r0 : z4;
        gr[1] = a1 ? r1 : z4;
        gi[0] = a0 ? i0 : z4;
        gi[1] = a1 ? i1 : z4;
        gb[0] = b0 ? w0 : z4;
        gb[1] = b1 ? w1 : z4;
      }
    };
    auto store_chunk = [&](int buf) {
      __bf16* b = sp + buf * CBUF_SPLIT;
      uint4 h, m, l;
      split3(gr[0], gr[1], h, m, l);
      st_planes(b, CTA, soff_a, h, m, l);
      split3(gi[0], gi[1], h, m, l);
      st_planes(b + 3 * CTA, CTA, soff_a, h, m, l);
      split3(gb[0], gb[1], h, m, l);
      st_planes(b + 6 * CTA + bq * 3 * CTB, CTB, soff_b, h, m, l);
    };
    const int nk = (Kc + 15) / 16;
    load_chunk(0);
    store_chunk(0);
    load_chunk((nk > 1 ? 1 : 0) * 16);
    __syncthreads();
    for (int kc = 0; kc < nk; ++kc) {
      const __bf16* b = sp + (kc & 1) * CBUF_SPLIT;
      bf16x8 pf[3], qf[3], nqf[3];
      ld_planes(b + 6 * CTA, CTB, plane_off(wc + fr, fh), pf);
      ld_planes(b + 6 * CTA + 3 * CTB, CTB, plane_off(wc + fr, fh), qf);
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        uint4 u = __builtin_bit_cast(uint4, qf[p]);
        u.x ^= 0x80008000u; u.y ^= 0x80008000u; u.z ^= 0x80008000u; u.w ^= 0x80008000u;
        nqf[p] = __builtin_bit_cast(bf16x8, u);
      }
      bf16x8 arf[2][3], aif[2][3];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ld_planes(b, CTA, plane_off(wr + 32 * i + fr, fh), arf[i]);
        ld_planes(b + 3 * CTA, CTA, plane_off(wr + 32 * i + fr, fh), aif[i]);
      }
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        const int pa = kSplitA[q], pb = kSplitB[q];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          T[0][i] = mfma_bf16(arf[i][pa], pf[pb], T[0][i]);
          T[1][i] = mfma_bf16(arf[i][pa], qf[pb], T[1][i]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          T[0][i] = mfma_bf16(aif[i][pa], nqf[pb], T[0][i]);
          T[1][i] = mfma_bf16(aif[i][pa], pf[pb], T[1][i]);
        }
      }
      store_chunk((kc & 1) ^ 1);
      load_chunk((kc + 2 < nk ? kc + 2 : nk - 1) * 16);
      __syncthreads();
    }
  } else {
    float4 sr[2], si[2], sp, sq;
    auto load_chunk = [&](int k0) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int lin = tid + 256 * p, r = lin >> 2, kc = (lin & 3) * 4;
        const int64_t row = row0 + r;
        const int gk = k0 + kc;
        const bool ok = row < M && gk < Kc;
        sr[p] = ok ? ld4(Ar + row * lda + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
        si[p] = ok ? ld4(Ai + row * lda + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      const int r = tid >> 2, kc = (tid & 3) * 4;
      const int gn = col0 + r, gk = k0 + kc;
      const bool ok = gn < Nc && gk < Kc;
      sp = ok ? ld4(P + (int64_t)gn * ldw + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
      sq = ok ? ld4(Q + (int64_t)gn * ldw + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_chunk = [&](int buf) {
      float* b = smem + buf * CBUF;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int lin = tid + 256 * p;
        st4(&b[clds(lin >> 2, lin & 3)], sr[p]);
        st4(&b[CTA + clds(lin >> 2, lin & 3)], si[p]);
      }
      st4(&b[2 * CTA + clds(tid >> 2, tid & 3)], sp);
      st4(&b[2 * CTA + CTB + clds(tid >> 2, tid & 3)], sq);
    };

    const int nk = (Kc + 15) / 16;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int kc = 0; kc < nk; ++kc) {
      const int buf = kc & 1;
      if (kc + 1 < nk) load_chunk((kc + 1) * 16);
      const float* b = smem + buf * CBUF;
      float ar[2][8], ai[2][8], pv[8], qv[8];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float4 vr = ld4(&b[clds(wr + i * 32 + fr, 2 * fh + q)]);
          const float4 vi = ld4(&b[CTA + clds(wr + i * 32 + fr, 2 * fh + q)]);
          ar[i][4 * q] = vr.x; ar[i][4 * q + 1] = vr.y; ar[i][4 * q + 2] = vr.z; ar[i][4 * q + 3] = vr.w;
          ai[i][4 * q] = vi.x; ai[i][4 * q + 1] = vi.y; ai[i][4 * q + 2] = vi.z; ai[i][4 * q + 3] = vi.w;
        }
        const float4 vp = ld4(&b[2 * CTA + clds(wc + fr, 2 * fh + q)]);
        const float4 vq = ld4(&b[2 * CTA + CTB + clds(wc + fr, 2 * fh + q)]);
        pv[4 * q] = vp.x; pv[4 * q + 1] = vp.y; pv[4 * q + 2] = vp.z; pv[4 * q + 3] = vp.w;
        qv[4 * q] = vq.x; qv[4 * q + 1] = vq.y; qv[4 * q + 2] = vq.z; qv[4 * q + 3] = vq.w;
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float sv = pv[t] + qv[t];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          T[0][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(ar[i][t], pv[t], T[0][i], 0, 0, 0);
          T[1][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(ai[i][t], qv[t], T[1][i], 0, 0, 0);
          T[2][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(ar[i][t] + ai[i][t], sv, T[2][i], 0, 0, 0);
        }
      }
      if (kc + 1 < nk) store_chunk(buf ^ 1);
      __syncthreads();
    }
  }

  // Accumulator layout of the 32x32 MFMA: lane l, register r -> column l % 32, row
  // 8 (r / 4) + 4 (l / 32) + r % 4.  Each wave stages a 32-row slab of [out_r | out_i] (32 + 32
  // columns) in LDS and writes it back as 16-byte row pieces (plus the gated copies).
  constexpr int CES = 64 + 8;
  static_assert(4 * 32 * CES <= C_LDS_FLOATS && 8 * 32 * CES <= C_LDS_FLOATS_SPLIT,
                "epilogue staging must fit in the operand buffers");
  float* ws = smem + wave * 32 * CES;
  // The gate epilogues' global operands (the gate column; for MODE 2 also F_r and F_i) of a
  // lane's four 16-byte pieces of a 32-row block are loaded one block ahead, into alternating
  // register sets, so their latency overlaps the staging of the block before (with one
  // workgroup per CU nothing else would hide it): 1.04-1.33x on the gate shapes of the model.
  // A piece past M or Nc loads from row M - 1 / column 0 and is not stored.
  float4 eg[2][4], efr[2][4], efi[2][4];
  auto load_gate_operands = [&](int i, int set) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lin = lane + 64 * q;
      int64_t row = row0 + wr + i * 32 + (lin >> 3);
      row = row < M ? row : M - 1;
      int gc = col0 + wc + (lin & 7) * 4;
      gc = gc < Nc ? gc : 0;
      const int t = g.s_off + gc, l1 = t / g.C, ch = t - l1 * g.C;
      eg[set][q] = ld4_nt(g.G + row * g.ldg + 64 * (l1 * (g.C >> 5) + (ch >> 5)) + (ch & 31));
      if constexpr (MODE == 2) {
        efr[set][q] = ld4_nt(g.Fr + row * g.ldf + gc);
        efi[set][q] = ld4_nt(g.Fi + row * g.ldf + gc);
      }
    }
  };
  // (the fp32 path, three workgroups per CU, loads them after the staging instead: a set
  // ahead would spill)
  if constexpr (MODE != 0 && PATH != CPATH_FP32) load_gate_operands(0, 0);
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rr = 8 * (r >> 2) + 4 * fh + (r & 3);
      const float t1 = T[0][i][r], t2 = T[1][i][r];
      if constexpr (PATH == CPATH_SPLIT4) {
        ws[rr * CES + fr] = t1;
        ws[rr * CES + 32 + fr] = t2;
      } else {
        ws[rr * CES + fr] = t1 - t2;
        ws[rr * CES + 32 + fr] = T[NT - 1][i][r] - t1 - t2;
      }
    }
    __syncthreads();
    if constexpr (MODE != 0) {
      if constexpr (PATH == CPATH_FP32) load_gate_operands(i, i & 1);
      else if (i + 1 < RB) load_gate_operands(i + 1, (i + 1) & 1);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lin = lane + 64 * q;
      const int r = lin >> 3;
      const int c = (lin & 7) * 4;
      const int64_t row = row0 + wr + i * 32 + r;
      const int gc = col0 + wc + c;
      if (row >= M || gc >= Nc) continue;
      const float4 yr = ld4(&ws[r * CES + c]), yi = ld4(&ws[r * CES + 32 + c]);
      float4 sg;
      if constexpr (MODE != 0) {
        const float4 gp = eg[i & 1][q];
        sg = make_float4(sigmoidf_(gp.x), sigmoidf_(gp.y), sigmoidf_(gp.z), sigmoidf_(gp.w));
      }
      if constexpr (MODE == 2) {
        st4_nt(Yr + row * ldy + gc, yr * sg);
        st4_nt(Yi + row * ldy + gc, yi * sg);
        st4_nt(g.Pout + row * g.ldp + gc, yr * efr[i & 1][q] + yi * efi[i & 1][q]);
        continue;
      }
      st4_nt(Yr + row * ldy + gc, yr);
      st4_nt(Yi + row * ldy + gc, yi);
      if constexpr (MODE == 1) {
        st4_nt(g.Zr + row * g.ldz + gc, yr * sg);
        st4_nt(g.Zi + row * g.ldz + gc, yi * sg);
      }
    }
  }
}

}  // namespace fu

using namespace fu;

static int complex_check(const float* A_r, const float* A_i, int64_t lda, const float* P, const float* Q,
                         int64_t ldw, const float* Y_r, const float* Y_i, int64_t ldy, int64_t M, int32_t Nc,
                         int32_t Kc, const char* who) {
  if (M < 0 || Nc <= 0 || Kc <= 0) return set_error(FU_ERR_SHAPE, "%s: bad shape M=%lld Nc=%d Kc=%d", who, (long long)M, Nc, Kc);
  if (Kc % 4 != 0 || lda % 4 != 0 || ldw % 4 != 0)
    return set_error(FU_ERR_UNSUPPORTED, "%s: Kc=%d, lda=%lld, ldw=%lld must be multiples of 4", who, Kc,
                     (long long)lda, (long long)ldw);
  if (lda < Kc || ldw < Kc || ldy < Nc) return set_error(FU_ERR_SHAPE, "%s: leading dimensions smaller than the rows", who);
  if (Nc % 4 != 0 || ldy % 4 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: Nc and ldy must be multiples of 4", who);
  if (M == 0) return FU_OK;  // no rows: the operands may be empty (NULL) arrays
  if (!A_r || !A_i || !P || !Q || !Y_r || !Y_i) return set_error(FU_ERR_NULL, "%s: NULL operand", who);
  if (!aligned16(A_r) || !aligned16(A_i) || !aligned16(P) || !aligned16(Q) || !aligned16(Y_r) || !aligned16(Y_i))
    return set_error(FU_ERR_ALIGN, "%s: operands must be 16-byte aligned", who);
  const int64_t total = ((M + CBM - 1) / CBM) * ((Nc + CBN - 1) / CBN);   // the larger tile count
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  return FU_OK;
}

// The gate source of the gate epilogues: the gate-paired conv1 m = 0 output Y0, whose gate
// columns for degrees 1 + (s_off + column) / C must exist: s_off + Nc <= L C with
// (2L + 1) C <= ldy0 columns, i.e. (2 (s_off + Nc) / C + 1) C <= ldy0.
static int gate_source_check(const char* who, const float* Y0, int64_t ldy0, int32_t s_off, int32_t C, int32_t Nc) {
  if (C <= 0 || C % 32 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 32", who, C);
  if (s_off < 0 || s_off % 4 != 0 || ldy0 % 4 != 0)
    return set_error(FU_ERR_ALIGN, "%s: s_off and ldy0 must be non-negative multiples of 4", who);
  const int64_t degrees = ((int64_t)s_off + Nc + C - 1) / C;
  if ((2 * degrees + 1) * C > ldy0) return set_error(FU_ERR_SHAPE, "%s: Y0 rows too short for the gate columns", who);
  (void)Y0;
  return FU_OK;
}

template <int MODE>
static int complex_launch(const float* A_r, const float* A_i, int64_t lda, const float* P, const float* Q, int64_t ldw,
                          const void* W3, float* Y_r, float* Y_i, int64_t ldy, int64_t M, int32_t Nc, int32_t Kc,
                          CGate g, void* stream, const char* who) {
  if (W3 && !aligned16(W3)) return set_error(FU_ERR_ALIGN, "%s: W3 must be 16-byte aligned", who);
  const int mode = matmul_mode();
  // without a pre-split weight both split modes run the in-kernel bf16 four-product loop
  const int path = mode == FU_MATMUL_FP32 ? CPATH_FP32
                   : !W3                  ? CPATH_SPLIT4
                   : mode == FU_MATMUL_SPLIT_F16 ? CPATH_F16_PRE : CPATH_SPLIT3_PRE;
  const int tile_n = pre_split(path) ? CBN_PRE : CBN;
  const int n_tiles = (Nc + tile_n - 1) / tile_n;
  const int64_t total = ((M + CBM - 1) / CBM) * n_tiles;
  const bool tail = Kc % 16 != 0;
  auto kern = path == CPATH_FP32 ? complex_linear_kernel<MODE, CPATH_FP32>
              : path == CPATH_SPLIT4 ? (tail ? complex_linear_kernel<MODE, CPATH_SPLIT4, true>
                                             : complex_linear_kernel<MODE, CPATH_SPLIT4, false>)
              : path == CPATH_F16_PRE ? (tail ? complex_linear_kernel<MODE, CPATH_F16_PRE, true>
                                              : complex_linear_kernel<MODE, CPATH_F16_PRE, false>)
                                      : (tail ? complex_linear_kernel<MODE, CPATH_SPLIT3_PRE, true>
                                              : complex_linear_kernel<MODE, CPATH_SPLIT3_PRE, false>);
  // the fp16 path reads the fp16 planes (and, after them, the column factors)
  const uint4* w3 = static_cast<const uint4*>(W3);
  if (path == CPATH_F16_PRE) w3 += complex_weight_split_vectors(Nc, Kc);
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(threads_of(path)), 0, as_stream(stream), A_r, A_i, lda, P, Q,
                     ldw, w3, Y_r, Y_i, ldy, M, Nc, Kc, n_tiles, total, g);
  return check_launch(who);
}

// The unscale factor 2^-e(n) of every column of the 32-column blocks (1 past Nc): e(n) is the
// exact scale (split_f16.h) of the column's largest magnitude over P, Q and P + Q.  flag[n]
// bit 0 marks a column with a piece (8 consecutive k from a multiple of 8, as the fragments
// hold them) of P or Q that is nonzero and below 2^-3 at that scale, bit 1 a column that is not
// flat (a piece maximum, zero pieces included, below 2^-6 of the largest).
__global__ void complex_weight_scale_kernel(const float* __restrict__ P, const float* __restrict__ Q, int64_t ldw,
                                            int32_t Nc, int32_t Kc, float* __restrict__ cinv, int* __restrict__ flag) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= ((Nc + 31) / 32) * 32) return;
  float m = 0.0f;
  if (n < Nc)
    for (int k = 0; k < Kc; ++k) {
      const float p = P[(int64_t)n * ldw + k], q = Q[(int64_t)n * ldw + k];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(p), fabsf(q)), fabsf(p + q)));
    }
  const int e = f16_exp_row(m);
  cinv[n] = pow2i(-e);
  bool low = false;
  float pmin = m, pmax = 0.0f;
  if (n < Nc)
    for (int k0 = 0; k0 < Kc; k0 += 8) {
      float mp = 0.0f, mq = 0.0f;
      for (int k = k0; k < k0 + 8 && k < Kc; ++k) {
        mp = fmaxf(mp, fabsf(P[(int64_t)n * ldw + k]));
        mq = fmaxf(mq, fabsf(Q[(int64_t)n * ldw + k]));
      }
      low = low || f16_lossy(mp * pow2i(e)) || f16_lossy(mq * pow2i(e));
      pmin = fminf(pmin, fminf(mp, mq));
      pmax = fmaxf(pmax, fmaxf(mp, mq));
    }
  flag[n] = (low ? 1 : 0) | (f16_flat(pmin, pmax) ? 0 : 2);
}

// Builds the fragment-order planes of (P, Q, P + Q), bf16 and scaled fp16: one thread per
// (32-column block, 16-k chunk, lane) writes the lane's 8 consecutive k of one column,
// zero-padded past Nc / Kc.
__global__ void complex_weight_split_kernel(const float* __restrict__ P, const float* __restrict__ Q, int64_t ldw,
                                            int32_t Nc, int32_t Kc, uint4* __restrict__ W3) {
  const int nkc = (Kc + 15) / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= complex_weight_split_vectors(Nc, Kc) / 9) return;
  const int lane = (int)(t & 63);
  const int64_t q = t >> 6;  // (block, chunk)
  const int n = (int)(q / nkc) * 32 + (lane & 31);
  const int k0 = (int)(q % nkc) * 16 + (lane >> 5) * 8;
  float p[8], r[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const bool ok = n < Nc && k0 + u < Kc;
    p[u] = ok ? P[(int64_t)n * ldw + k0 + u] : 0.0f;
    r[u] = ok ? Q[(int64_t)n * ldw + k0 + u] : 0.0f;
  }
  uint4* o = W3 + q * 9 * 64 + lane;
  uint4 h, m, l;
  split3(make_float4(p[0], p[1], p[2], p[3]), make_float4(p[4], p[5], p[6], p[7]), h, m, l);
  o[0] = h; o[64] = m; o[128] = l;
  split3(make_float4(r[0], r[1], r[2], r[3]), make_float4(r[4], r[5], r[6], r[7]), h, m, l);
  o[192] = h; o[256] = m; o[320] = l;
  split3(make_float4(p[0] + r[0], p[1] + r[1], p[2] + r[2], p[3] + r[3]),
         make_float4(p[4] + r[4], p[5] + r[5], p[6] + r[6], p[7] + r[7]), h, m, l);
  o[384] = h; o[448] = m; o[512] = l;
  // fp16 planes of the scaled column (the factor 2^-e(n) is an exact power of two)
  uint4* f = W3 + complex_weight_split_vectors(Nc, Kc) + q * 9 * 64 + lane;
  const float* cinv = reinterpret_cast<const float*>(W3 + complex_weight_split_vectors(Nc, Kc) +
                                                     complex_weight_f16_vectors(Nc, Kc));
  const float sc = 1.0f / cinv[n];
  float ps[8], rs[8], ss[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    ps[u] = p[u] * sc;
    rs[u] = r[u] * sc;
    ss[u] = (p[u] + r[u]) * sc;
  }
  uint4 fh, fl;
  const float* planes[3] = {ps, rs, ss};
#pragma unroll
  for (int op = 0; op < 3; ++op) {
    const float* v = planes[op];
    const float4 v0 = make_float4(v[0], v[1], v[2], v[3]), v1 = make_float4(v[4], v[5], v[6], v[7]);
    split2h(v0, v1, fh, fl);
    f[128 * op] = fh;
    f[128 * op + 64] = fl;
    split2h_up(v0, v1, fh, fl);
    f[384 + 64 * op] = fl;
  }
}

extern "C" int64_t fu_complex_weight_split_bytes(int32_t Nc, int32_t Kc) {
  if (Nc <= 0 || Kc <= 0) return set_error(FU_ERR_SHAPE, "fu_complex_weight_split_bytes: Nc=%d Kc=%d", Nc, Kc);
  return (complex_weight_split_vectors(Nc, Kc) + complex_weight_f16_vectors(Nc, Kc) +
          2 * complex_weight_scale_vectors(Nc)) * 16;
}

extern "C" int fu_complex_weight_split(const float* P, const float* Q, int64_t ldw, int32_t Nc, int32_t Kc, void* W3,
                                       void* stream) {
  const char* who = "fu_complex_weight_split";
  if (Nc <= 0 || Kc <= 0 || ldw < Kc) return set_error(FU_ERR_SHAPE, "%s: Nc=%d Kc=%d ldw=%lld", who, Nc, Kc, (long long)ldw);
  if (!P || !Q || !W3) return set_error(FU_ERR_NULL, "%s: NULL argument", who);
  if (!aligned16(W3)) return set_error(FU_ERR_ALIGN, "%s: W3 must be 16-byte aligned", who);
  uint4* w3 = static_cast<uint4*>(W3);
  float* cinv = reinterpret_cast<float*>(w3 + complex_weight_split_vectors(Nc, Kc) + complex_weight_f16_vectors(Nc, Kc));
  int* flag = reinterpret_cast<int*>(cinv + (int64_t)((Nc + 31) / 32) * 32);
  hipLaunchKernelGGL(complex_weight_scale_kernel, dim3(cdiv((int64_t)((Nc + 31) / 32) * 32, 256)), dim3(256), 0,
                     as_stream(stream), P, Q, ldw, Nc, Kc, cinv, flag);
  const int64_t threads = complex_weight_split_vectors(Nc, Kc) / 9;
  hipLaunchKernelGGL(complex_weight_split_kernel, dim3(cdiv(threads, 256)), dim3(256), 0, as_stream(stream), P, Q, ldw,
                     Nc, Kc, w3);
  return check_launch(who);
}

extern "C" int fu_complex_linear(const float* A_r, const float* A_i, int64_t lda, const float* P, const float* Q,
                                 int64_t ldw, const void* W3, float* Y_r, float* Y_i, int64_t ldy, int64_t M,
                                 int32_t Nc, int32_t Kc, void* stream) {
  int st = complex_check(A_r, A_i, lda, P, Q, ldw, Y_r, Y_i, ldy, M, Nc, Kc, "fu_complex_linear");
  if (st != FU_OK || M == 0) return st;
  return complex_launch<0>(A_r, A_i, lda, P, Q, ldw, W3, Y_r, Y_i, ldy, M, Nc, Kc, CGate{}, stream,
                           "fu_complex_linear");
}

extern "C" int fu_complex_linear_gate(const float* A_r, const float* A_i, int64_t lda, const float* P, const float* Q,
                                      int64_t ldw, const void* W3, float* Y_r, float* Y_i, int64_t ldy, float* Z_r,
                                      float* Z_i, int64_t ldz, const float* Y0, int64_t ldy0, int32_t s_off, int32_t C,
                                      int64_t M, int32_t Nc, int32_t Kc, void* stream) {
  const char* who = "fu_complex_linear_gate";
  int st = complex_check(A_r, A_i, lda, P, Q, ldw, Y_r, Y_i, ldy, M, Nc, Kc, who);
  if (st != FU_OK) return st;
  st = gate_source_check(who, Y0, ldy0, s_off, C, Nc);
  if (st != FU_OK) return st;
  if (ldz < Nc) return set_error(FU_ERR_SHAPE, "%s: gate strides too small", who);
  if (M == 0) return FU_OK;
  if (!Z_r || !Z_i || !Y0) return set_error(FU_ERR_NULL, "%s: NULL gate operand", who);
  if (ldz % 4 != 0 || !aligned16(Z_r) || !aligned16(Z_i) || !aligned16(Y0))
    return set_error(FU_ERR_ALIGN, "%s: gate operands must be 16-byte aligned with strides multiples of 4", who);
  return complex_launch<1>(A_r, A_i, lda, P, Q, ldw, W3, Y_r, Y_i, ldy, M, Nc, Kc,
                           CGate{Z_r, Z_i, ldz, Y0, ldy0, s_off, C, nullptr, nullptr, 0, nullptr, 0}, stream, who);
}

extern "C" int fu_complex_linear_gate_bwd(const float* A_r, const float* A_i, int64_t lda, const float* P,
                                          const float* Q, int64_t ldw, const void* W3, float* gY_r, float* gY_i,
                                          int64_t ldg,
                                          const float* F_r, const float* F_i, int64_t ldf, const float* Y0,
                                          int64_t ldy0, int32_t s_off, int32_t C, float* Pout, int64_t ldp, int64_t M,
                                          int32_t Nc, int32_t Kc, void* stream) {
  const char* who = "fu_complex_linear_gate_bwd";
  int st = complex_check(A_r, A_i, lda, P, Q, ldw, gY_r, gY_i, ldg, M, Nc, Kc, who);
  if (st != FU_OK) return st;
  st = gate_source_check(who, Y0, ldy0, s_off, C, Nc);
  if (st != FU_OK) return st;
  if (ldf < Nc || ldp < Nc) return set_error(FU_ERR_SHAPE, "%s: gate strides too small", who);
  if (M == 0) return FU_OK;
  if (!F_r || !F_i || !Y0 || !Pout) return set_error(FU_ERR_NULL, "%s: NULL gate operand", who);
  if ((ldf | ldp) % 4 != 0 || !aligned16(F_r) || !aligned16(F_i) || !aligned16(Y0) || !aligned16(Pout))
    return set_error(FU_ERR_ALIGN, "%s: gate operands must be 16-byte aligned with strides multiples of 4", who);
  return complex_launch<2>(A_r, A_i, lda, P, Q, ldw, W3, gY_r, gY_i, ldg, M, Nc, Kc,
                           CGate{nullptr, nullptr, 0, Y0, ldy0, s_off, C, F_r, F_i, ldf, Pout, ldp}, stream, who);
}
