// Dense fp32 contractions on the gfx950 matrix cores.
//
// Y[M, N] = A[M, K] @ W[N, K]^T (+ bias[N]).  Both operands are K-contiguous, so one kernel
// serves the SO(2) conv1/conv2 forward (W = packed weight, model.py:152,154), the radial-MLP
// linears (model.py:147-149) and every input-gradient GEMM of the backward pass (W = the
// pre-transposed weight).  No weight gradients are ever needed: parameters are frozen.
//
// Tiling: a 256-thread workgroup (4 wave64s in a 2x2 grid) owns a 128x128 output tile; each
// wave owns 64x64 = 2x2 MFMA blocks of 32x32 (64 fp32 accumulators per lane, in VGPRs).
// K advances in chunks of 16 staged through double-buffered LDS.  Three main loops share the
// tiling and the epilogues (fu_set_matmul_mode):
//  * split fp16 (default, F16): each staged row is scaled by its power of two and split into
//    two fp16 planes (split_f16.h); three v_mfma_f32_32x32x16_f16 per 32x32 block and chunk.
//    The scales come from the first chunk (from a pre-pass over the rows when K <= 64 or when a
//    row's first chunk is zero); a tile whose accumulators came out non-finite (an fp16 piece
//    overflowed) runs its K loop again at exact scales.  The accumulators are unscaled before
//    the epilogue.
//  * split bf16: each staged fp32 element is split into three bf16 planes
//    (split_bf16.h) as it is written to LDS (48 KB of planes, two workgroups per CU); per chunk
//    a wave reads 3 planes of each operand fragment and issues six v_mfma_f32_32x32x16_bf16
//    per 32x32 block.  The loop body has no branches (the last prefetch re-reads the last
//    chunk), so the compiler interleaves the next chunk's split with this chunk's MFMAs.
//  * fp32: v_mfma_f32_32x32x2_f32, lane l (row/col l%32, half h = l/32) feeding k-slot h with
//    chunk column 8h + t at step t; fp32 LDS rows of 64 bytes (four 16-byte chunks) without
//    padding, the chunk index XOR-swizzled with f(row) = ((row >> 1) ^ (row >> 2)) & 3, so
//    the row-wise tile stores and the column-of-rows operand reads are free of bank
//    conflicts (32 KB of operands, 36 KB with the epilogue staging: four workgroups per CU).
// The epilogue stages each wave's 32-row slabs through LDS and writes rows with 16-byte stores.
#include "split_f16.h"

namespace fu {

constexpr int GBM = 128, GBN = 128, GBK = 16;
constexpr int GLDS = GBK;          // LDS operand row (floats): four swizzled 16-byte chunks
constexpr int GES = 64 + 8;        // LDS epilogue row (floats); 4 * GES = 32 mod 64 banks
constexpr int G_LDS_FLOATS = 2 * (GBM + GBN) * GLDS > 4 * 32 * GES ? 2 * (GBM + GBN) * GLDS : 4 * 32 * GES;
constexpr int G_PLANE = GBM * GBK;                       // bf16 per split plane of one tile
constexpr int G_LDS_FLOATS_SPLIT = 2 * 6 * G_PLANE / 2;  // [buf][A planes | W planes], 48 KB
static_assert(GBM == GBN, "the split planes of A and W tiles share one layout");
// Tall split tiles (TALL): 256 rows x 128 columns, each wave 128 x 64 (4 x 2 blocks of 32):
// per 16-wide K chunk a wave issues 48 MFMAs for 12 A and 6 W fragment reads, and a
// workgroup stages 256 + 128 rows.  A planes of 256 rows, W planes of 128 rows, 72 KB
// double-buffered (two workgroups per CU).
constexpr int G_PLANE_A_TALL = 2 * GBM * GBK;
constexpr int G_LDS_FLOATS_TALL = 2 * 3 * (G_PLANE_A_TALL + G_PLANE) / 2;
// fp16 split (F16): two planes per operand, 32 KB (the epilogue staging needs 36 KB) and 48 KB
constexpr int G_LDS_FLOATS_SPLIT_F16 = 2 * 2 * G_PLANE > 4 * 32 * GES ? 2 * 2 * G_PLANE : 4 * 32 * GES;
constexpr int G_LDS_FLOATS_TALL_F16 = 2 * 2 * (G_PLANE_A_TALL + G_PLANE) / 2;
static_assert(4 * 32 * GES <= G_LDS_FLOATS_TALL_F16, "epilogue staging must fit in the fp16 tall planes");
static_assert(4 * 32 * GES <= G_LDS_FLOATS_SPLIT, "epilogue staging must fit in the split planes");

// Float offset of 16-byte chunk `chunk` of LDS operand row `row`.
__device__ __forceinline__ int lds_chunk(int row, int chunk) {
  return row * GLDS + 4 * (chunk ^ (((row >> 1) ^ (row >> 2)) & 3));
}

// Extra outputs of the gate epilogue (conv1 m = 0 fused with the gate activation).
struct GateOut {
  float* Z;     // (M, (L+1)C): [silu(y_l0), y_l1m0 s1, ..., y_lLm0 sL]
  int64_t ldz;
  float* S;     // optional (M, LC): [s1, ..., sL] = sigmoid of the L gate blocks
  int64_t lds;
  int32_t C;
  int32_t L;    // lmax
};

// Operands of the gate-backward epilogue (conv2 m = 0 input gradient fused with the gate
// backward).  The GEMM computes g_Z_m0 (M, (L+1)C) = [g_l0, g_l1m0, ..., g_lLm0]; the epilogue
// writes g_Y_m0 (M, (2L+1)C) in the gate-paired order instead: g_y_l0 = g silu'(y_l0),
// g_y_lm0 = g s_l and g_gate_l = s_l (1 - s_l) (g y_lm0 + P1[l] (+ P2[l] for l >= 2)), where
// s_l = sigmoid(gate_l) is recomputed from the gate columns of Y0, and P1 (M, LC) and
// P2 (M, (L-1)C) are the gate sums sum_m g_z y of the m = 1 and m = 2 blocks (written by
// fu_complex_linear_gate_bwd).
struct GateBwd {
  const float* Y0;  // (M, (2L+1)C) forward pre-activation, gate-paired
  int64_t ldy0;
  const float* P1;
  int64_t ldp1;
  const float* P2;
  int64_t ldp2;
  int32_t C;
  int32_t L;
};

// Residual added by the plain epilogue (MODE 0): Y += R, R with row stride ldr, batch stride sR.
struct Resid {
  const float* R;
  int64_t ldr;
  int64_t sR;
};

// LayerNorm + SiLU epilogues over groups of LN_D = 128 columns (the radial-MLP hidden layers,
// ops/ln_silu.py:29-123, in the grouped form of fu_ln_silu_grouped_*).  Each N-tile is one
// group: group g = n_tile + batch index (a launch has either several N-tiles or several
// batches).  The LayerNorm input of row e, group g, column c is
//   v = (A W^T)[e][c] (+ GEMM bias) + tab_src[z[isrc[e]]][gD + c] + tab_dst[z[idst[e]]][gD + c]
//       + ln_bias[gD + c]
// (tables and ln_bias optional).  MODE 3 writes silu(LN(v) gamma + beta) to Y, the row
// statistics to mean / rstd[e G + g] and, when pre is set, the GEMM output (before tables
// and ln_bias) to pre (batch stride s_pre).  MODE 4 is the input gradient: with the forward's
// mean / rstd and the output gradient g_out (row stride ldgo, group g at column gD), Y
// receives dL/dv.  MODE 5 is the input gradient when the GEMM product is the output gradient
// g_out: v is then read from pre (row stride ldpre, group g at column gD).
constexpr int LN_D = 128;
struct LnEpi {
  const float* tab_src;
  const float* tab_dst;
  int64_t ldt;
  const int64_t* z;
  const int64_t* isrc;
  const int64_t* idst;
  const float* ln_bias;
  const float* gamma;
  const float* beta;
  float* mean;
  float* rstd;
  int32_t G;
  float eps;
  float* pre;
  int64_t ldpre;
  int64_t s_pre;
  const float* g_out;
  int64_t ldgo;
};

// conv1 m = 0's A operand gathered in the loader (fu_gather_linear_gate, lmax = 2): row e,
// column k = (so * 3 + q) C + c is the layout-1 gather output X_m0 of ops/gather.py,
//   rot_q(x[node_so(e)])[c] * rad[e][(so * 6 + q) C + c],   node_0 = idx_i, node_1 = idx_j,
// with rot_0 = x_l0 + csd[batch], rot_1 = (row 1 of D1) x_l1, rot_2 = (row 2 of D2) x_l2 (the
// m = 0 rows of the Wigner blocks, wigner[e][3..5] and [19..23]), so X_m0 is never stored.
struct GatherA {
  const float* x;
  const int64_t* idx_i;
  const int64_t* idx_j;
  const float* wig;
  const float* rad;
  const float* csd;
  const int64_t* batch;
  int32_t C;
};

// Batch index blockIdx.y offsets A, W and Y by sA, sW and sY floats; bias (stride sBias) is
// added in batches [0, bias_batches).
//
// MODE 0: plain.  MODE 1 (gate): Y has N = (2L+1)C columns in the gate-paired order -- every
// 64-column pair p holds [32 gate channels | the 32 channels they gate]: pairs
// (l-1) C/32 .. l C/32 - 1 are (gate_l, y_lm0) for l = 1..L, the last C/64 hold y_l0 -- so a
// wave's 64 staged columns are a gate and its values; the epilogue writes Y (kept for the
// backward), Z and S.  MODE 2 (gate backward): see GateBwd; Y receives g_Y_m0 ((2L+1)C
// columns).
template <int MODE, bool SPLIT, bool KTAIL = false, bool TALL = false, bool GATHER = false, bool F16 = false,
          bool WF = false>
__global__ __launch_bounds__(256, SPLIT ? (TALL ? 2 : 3) : 4) void linear_mfma_kernel(const float* __restrict__ A, int64_t lda, int64_t sA,
                                                          const float* __restrict__ W, int64_t ldw, int64_t sW,
                                                          const float* __restrict__ bias, int64_t sBias,
                                                          int32_t bias_batches, float* __restrict__ Y, int64_t ldy,
                                                          int64_t sY, int64_t M, int32_t N, int32_t K,
                                                          int32_t n_tiles, int64_t total_tiles, GateOut go,
                                                          GateBwd gb, Resid rs, LnEpi ln,
                                                          GatherA gx = GatherA{},
                                                          const uint4* __restrict__ W2 = nullptr) {
  {
    const int64_t bt = blockIdx.y;
    A += bt * sA;
    W += bt * sW;
    Y += bt * sY;
    if (ln.pre) ln.pre += bt * ln.s_pre;
    bias = (bias != nullptr && bt < bias_batches) ? bias + bt * sBias : nullptr;
    if (rs.R) rs.R += bt * rs.sR;
  }
  static_assert(SPLIT || !TALL, "tall tiles exist in the split mode only");
  static_assert(!GATHER || (SPLIT && !KTAIL && MODE == 1), "the gathered A operand feeds the split gate GEMM");
  static_assert(!F16 || (SPLIT && !GATHER), "the fp16 split is a split mode without the gathered loader");
  static_assert(!WF || (F16 && TALL && !KTAIL), "pre-split weight fragments feed the tall fp16 tile without a K tail");
  constexpr int RB = TALL ? 4 : 2;          // 32-row blocks per wave
  constexpr int BM = 64 * RB;               // tile rows
  constexpr int PA = BM * GBK, PW = G_PLANE;  // bf16 per A plane, per W plane
  __shared__ __attribute__((aligned(16))) float smem[TALL ? (F16 ? G_LDS_FLOATS_TALL_F16 : G_LDS_FLOATS_TALL)
                                                     : SPLIT ? (F16 ? G_LDS_FLOATS_SPLIT_F16 : G_LDS_FLOATS_SPLIT)
                                                             : G_LDS_FLOATS];

  // XCD-aware tile order: hardware deals consecutive workgroups round-robin over the 8 XCDs;
  // remap so that each XCD walks a contiguous range of tiles (the column tiles of one A
  // row-panel then share that XCD's L2).
  int64_t wg = blockIdx.x;
  if ((total_tiles & 7) == 0) wg = (wg & 7) * (total_tiles >> 3) + (wg >> 3);
  const int64_t m_tile = wg / n_tiles;
  const int n_tile = (int)(wg - m_tile * n_tiles);
  const int64_t row0 = m_tile * BM;
  const int col0 = n_tile * GBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = (wave >> 1) * 32 * RB;  // wave's row offset inside the tile
  const int wc = (wave & 1) * 64;        // wave's col offset inside the tile

  floatx16 acc[RB][2];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int fr = lane & 31;  // operand row (A) / column (W) within a 32-block
  const int fh = lane >> 5;  // this lane feeds chunk columns 8 fh .. 8 fh + 7
  if constexpr (SPLIT) {
    // [buf][A planes (NP x PA) | W planes (NP x PW)]: hi, mid, lo bf16, or hi, lo fp16 (F16)
    constexpr int NP = F16 ? 2 : 3;
    __bf16* sp = reinterpret_cast<__bf16*>(smem);
    const int sr = tid >> 1, sh = tid & 1;         // staging: tile row sr (+128 if TALL), k 8 sh ..
    const int soff = plane_off(sr, sh);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 ga[2], gw[2], ga2[2];
    // A thread stages the same tile row (of A and of W) for the whole K loop, so its row
    // pointers are fixed: a row past M (N) reads row M-1 (N-1) instead, whose products land in
    // output rows (columns) that are never stored.  Without a K tail (KTAIL false: K a multiple
    // of 16) every chunk is four plain 16-byte loads.  With one, every load is unconditional
    // from a valid address followed by a select that zeroes the pieces at or past K (guarded
    // loads would be scalarised into dword loads).  The loader has no branch either way:
    // an if/else here, selecting between the two forms per chunk, was miscompiled in the
    // pre-split complex kernel (a prefetched operand register reused before its read).
    const int64_t gr = row0 + sr, gr2 = row0 + 128 + sr;
    const int gn = col0 + sr;
    const float* pa = A + (gr < M ? gr : M - 1) * lda + 8 * sh;
    const float* pa2 = A + (gr2 < M ? gr2 : M - 1) * lda + 8 * sh;   // second staged row (TALL)
    const float* pw = W + (int64_t)(gn < N ? gn : N - 1) * ldw + 8 * sh;
    // GATHER: per staged row, its two node rows (csd rows for l = 0), its radial row and the
    // m = 0 Wigner rows, fixed for the whole K loop
    const float* xn[2][2];
    const float* cn[2][2];
    const float* rr[2];
    float w1[2][3], w2[2][5];
    if constexpr (GATHER) {
      const int64_t ers[2] = {gr < M ? gr : M - 1, gr2 < M ? gr2 : M - 1};
#pragma unroll
      for (int t = 0; t < (TALL ? 2 : 1); ++t) {
        const int64_t e = ers[t];
        const int64_t nd[2] = {gx.idx_i[e], gx.idx_j[e]};
#pragma unroll
        for (int so = 0; so < 2; ++so) {
          xn[t][so] = gx.x + nd[so] * 9 * gx.C + 8 * sh;
          cn[t][so] = gx.csd + gx.batch[nd[so]] * gx.C + 8 * sh;
        }
        rr[t] = gx.rad + e * 12 * gx.C + 8 * sh;
#pragma unroll
        for (int b = 0; b < 3; ++b) w1[t][b] = gx.wig[e * 34 + 3 + b];
#pragma unroll
        for (int b = 0; b < 5; ++b) w2[t][b] = gx.wig[e * 34 + 19 + b];
      }
    }
    // the 8 gathered values of staged row t at K offset k0 (+ 8 sh): the slot (so, q) of a
    // chunk is uniform, so the branch on q is a scalar one; the products and sums run in the
    // order of the gather kernel's rotation
    auto gather_row = [&](int t, int k0, float4& o0, float4& o1) {
      const int C = gx.C;
      const int so = k0 / (3 * C), q = (k0 - so * 3 * C) / C, c = k0 - (so * 3 + q) * C;
      const float* xb = xn[t][so] + c;
      float4 a0, a1;
      if (q == 0) {
        a0 = ld4(xb) + ld4(cn[t][so] + c);
        a1 = ld4(xb + 4) + ld4(cn[t][so] + c + 4);
      } else if (q == 1) {
        a0 = scale4(ld4(xb + C), w1[t][0]) + scale4(ld4(xb + 2 * C), w1[t][1]) + scale4(ld4(xb + 3 * C), w1[t][2]);
        a1 = scale4(ld4(xb + C + 4), w1[t][0]) + scale4(ld4(xb + 2 * C + 4), w1[t][1]) +
             scale4(ld4(xb + 3 * C + 4), w1[t][2]);
      } else {
        a0 = scale4(ld4(xb + 4 * C), w2[t][0]) + scale4(ld4(xb + 5 * C), w2[t][1]) + scale4(ld4(xb + 6 * C), w2[t][2]) +
             scale4(ld4(xb + 7 * C), w2[t][3]) + scale4(ld4(xb + 8 * C), w2[t][4]);
        a1 = scale4(ld4(xb + 4 * C + 4), w2[t][0]) + scale4(ld4(xb + 5 * C + 4), w2[t][1]) +
             scale4(ld4(xb + 6 * C + 4), w2[t][2]) + scale4(ld4(xb + 7 * C + 4), w2[t][3]) +
             scale4(ld4(xb + 8 * C + 4), w2[t][4]);
      }
      // plain loads: every column tile of the row panel reads the radial row again (from L2)
      const float* rp = rr[t] + (so * 6 + q) * C + c;
      o0 = a0 * ld4(rp);
      o1 = a1 * ld4(rp + 4);
    };
    auto load_chunk = [&](int k0) {
      if constexpr (GATHER) {
        gather_row(0, k0, ga[0], ga[1]);
        if constexpr (TALL) gather_row(1, k0, ga2[0], ga2[1]);
        gw[0] = ld4(pw + k0);
        gw[1] = ld4(pw + k0 + 4);
      } else if constexpr (!KTAIL) {
        ga[0] = ld4(pa + k0);
        ga[1] = ld4(pa + k0 + 4);
        if constexpr (TALL) {
          ga2[0] = ld4(pa2 + k0);
          ga2[1] = ld4(pa2 + k0 + 4);
        }
        if constexpr (!WF) {
          gw[0] = ld4(pw + k0);
          gw[1] = ld4(pw + k0 + 4);
        }
      } else {
        const int gk = k0 + 8 * sh;
        const bool k0ok = gk < K, k1ok = gk + 4 < K;
        const float4 va0 = ld4(k0ok ? pa + k0 : A), va1 = ld4(k1ok ? pa + k0 + 4 : A);
        const float4 vw0 = ld4(k0ok ? pw + k0 : W), vw1 = ld4(k1ok ? pw + k0 + 4 : W);
        ga[0] = k0ok ? va0 : z4;
        ga[1] = k1ok ? va1 : z4;
        gw[0] = k0ok ? vw0 : z4;
        gw[1] = k1ok ? vw1 : z4;
        if constexpr (TALL) {
          const float4 vb0 = ld4(k0ok ? pa2 + k0 : A), vb1 = ld4(k1ok ? pa2 + k0 + 4 : A);
          ga2[0] = k0ok ? vb0 : z4;
          ga2[1] = k1ok ? vb1 : z4;
        }
      }
    };
    // F16: the power-of-two scales of the staged rows (A row, second A row if TALL, W row), and
    // the window tracking of pass 0 (split_f16.h) per staged row, on its scaled pieces of 8
    // consecutive k: the largest and the smallest piece maximum (zero pieces included), and
    // whether a nonzero piece fell below the window (lowA for A, lowW for W)
    float scA = 1.0f, scA2 = 1.0f, scW = 1.0f;
    int eA = 0, eA2 = 0, eW = 0;
    float pmaxA = 0.0f, pminA = __builtin_huge_valf(), pmaxA2 = 0.0f, pminA2 = __builtin_huge_valf();
    float pmaxW = 0.0f, pminW = __builtin_huge_valf();
    bool lowA = false, lowW = false;
    // WF: a weight whose columns are all flat and have no piece below the window (summary word
    // of the pre-split weight 0) never makes the verdict ask for exact scales on A's account, so
    // A's pieces are not tracked (the overflow check on the accumulators stays): 5 % of the loop
    bool track = true;
    if constexpr (WF) track = reinterpret_cast<const int*>(W2 + resident_frag_vectors(N, K))[2 * resident_cols(N)] != 0;
    // ps: the pass kind of the K loop (0: hi + lo planes, the window tracked; 1: hi and
    // lo' = 2^11 lo planes of pass 2; 2: the hi planes of pass 2)
    auto store_chunk = [&](int buf, auto ps) {
      constexpr int PS = decltype(ps)::value;
      __bf16* b = sp + buf * NP * (PA + PW);
      if constexpr (F16) {
        auto put = [&](const float4& x0, const float4& x1, float s, __bf16* p0, int plane, int off, float& pmax,
                       float& pmin, bool& low) {
          const float4 v0 = scale4(x0, s), v1 = scale4(x1, s);
          uint4 h, l;
          if constexpr (PS == 0) {
            if (track) {
              const float m = amax8(v0, v1);
              pmax = fmaxf(pmax, m);
              pmin = fminf(pmin, m);
              low |= f16_lossy(m);
            }
            split2h(v0, v1, h, l);
          } else {
            split2h_up(v0, v1, h, l);
          }
          st_planes2(p0, plane, off, h, l);
        };
        put(ga[0], ga[1], scA, b, PA, soff, pmaxA, pminA, lowA);
        if constexpr (TALL) put(ga2[0], ga2[1], scA2, b, PA, plane_off(128 + sr, sh), pmaxA2, pminA2, lowA);
        if constexpr (!WF) put(gw[0], gw[1], scW, b + 2 * PA, PW, soff, pmaxW, pminW, lowW);
      } else {
        uint4 h, m, l;
        split3(ga[0], ga[1], h, m, l);
        st_planes(b, PA, soff, h, m, l);
        if constexpr (TALL) {
          split3(ga2[0], ga2[1], h, m, l);
          st_planes(b, PA, plane_off(128 + sr, sh), h, m, l);
        }
        split3(gw[0], gw[1], h, m, l);
        st_planes(b + 3 * PA, PW, soff, h, m, l);
      }
    };
    // the larger (smaller) value of this thread's and its partner's half of a staged row
    auto row_max = [&](float v) { return fmaxf(v, __shfl_xor(v, 1, 64)); };
    auto row_min = [&](float v) { return fminf(v, __shfl_xor(v, 1, 64)); };
    const int nk = (K + GBK - 1) / GBK;
    // One K loop.  F16 products per pass kind: 0 lo*hi + hi*lo + hi*hi, 1 lo'*hi + hi*lo',
    // 2 hi*hi.
    // WF: this wave's two 32-column blocks of the pre-split weight (a block past N reads the
    // last one; its outputs are never stored)
    int wfb[2] = {0, 0};
    if constexpr (WF) {
      const int nb = (N + 31) / 32;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int b_ = (col0 + wc) / 32 + j;
        wfb[j] = b_ < nb ? b_ : nb - 1;
      }
    }
    auto kloop = [&](auto ps) {
      constexpr int PS = decltype(ps)::value;
      constexpr int QB = PS == 2 ? 2 : 0, QE = PS == 1 ? 2 : 3;
      // WF: the fragments of chunk kc (hi, and lo or lo' in pass kind 1) straight from the
      // weight buffer into registers, one chunk ahead
      f16x8 bnx[2][2];
      auto load_frags = [&](int kc) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t base = ((int64_t)wfb[j] * nk + kc) * 3 * 64 + lane;
          bnx[j][0] = __builtin_bit_cast(f16x8, W2[base]);
          bnx[j][1] = __builtin_bit_cast(f16x8, W2[base + (PS == 1 ? 128 : 64)]);
        }
      };
      if constexpr (WF) load_frags(0);
      load_chunk(0);
      store_chunk(0, ps);
      load_chunk((nk > 1 ? 1 : 0) * GBK);
      __syncthreads();
      for (int kc = 0; kc < nk; ++kc) {
        const __bf16* b = sp + (kc & 1) * NP * (PA + PW);
        if constexpr (F16) {
          f16x8 bq[2][2];
          if constexpr (WF) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              bq[j][0] = bnx[j][0];
              bq[j][1] = bnx[j][1];
            }
            load_frags(kc + 1 < nk ? kc + 1 : nk - 1);
          } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) ld_planes2(b + 2 * PA, PW, plane_off(wc + 32 * j + fr, fh), bq[j]);
          }
#pragma unroll
          for (int i = 0; i < RB; ++i) {
            f16x8 aq[2];
            ld_planes2(b, PA, plane_off(wr + 32 * i + fr, fh), aq);
#pragma unroll
            for (int q = QB; q < QE; ++q)
#pragma unroll
              for (int j = 0; j < 2; ++j) acc[i][j] = mfma_f16(aq[kF16A[q]], bq[j][kF16B[q]], acc[i][j]);
          }
        } else {
          bf16x8 bq[2][3];
#pragma unroll
          for (int j = 0; j < 2; ++j) ld_planes(b + 3 * PA, PW, plane_off(wc + 32 * j + fr, fh), bq[j]);
#pragma unroll
          for (int i = 0; i < RB; ++i) {
            bf16x8 aq[3];
            ld_planes(b, PA, plane_off(wr + 32 * i + fr, fh), aq);
#pragma unroll
            for (int q = 0; q < 6; ++q)
#pragma unroll
              for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(aq[kSplitA[q]], bq[j][kSplitB[q]], acc[i][j]);
          }
        }
        // chunk kc + 1 (loaded during the previous iteration) into the other buffer, whose last
        // readers finished before the previous barrier; then prefetch chunk kc + 2
        store_chunk((kc & 1) ^ 1, ps);
        load_chunk((kc + 2 < nk ? kc + 2 : nk - 1) * GBK);
        __syncthreads();
      }
    };
    if constexpr (!F16) {
      kloop(std::integral_constant<int, 0>{});
    } else {
      // The passes of split_f16.h.  Pass 0 takes the scales from the rows' first chunk.  Its
      // tile is computed again at exact scales when an fp16 piece overflowed (its accumulators
      // are then non-finite) or when one operand has a piece below the window while the other
      // is not flat; exact scales come from a pass over the rows, which also applies the same
      // rule at those scales: pass 1 (one K loop) or pass 2 (two loops).
      const bool short_k = nk <= F16_PREPASS_CHUNKS;
      __shared__ unsigned f16_any[4];
      // OR over the workgroup of each thread's verdict bits (every thread calls this)
      auto tile_bits = [&](unsigned v) {
        unsigned w = 0;
#pragma unroll
        for (int bit = 0; bit < 5; ++bit) w |= (__ballot((v >> bit) & 1u) != 0 ? 1u : 0u) << bit;
        __syncthreads();  // the previous call's readers are done with f16_any
        if (lane == 0) f16_any[wave] = w;
        __syncthreads();
        return f16_any[0] | f16_any[1] | f16_any[2] | f16_any[3];
      };
      // a thread's verdict bits for its rows (row-level max / min over the two staging threads)
      // WF: the weight's side from its precomputed flags (the staged column of this thread)
      int wflag = 0;
      if constexpr (WF) {
        const int* flags = reinterpret_cast<const int*>(W2 + resident_frag_vectors(N, K)) + resident_cols(N);
        wflag = flags[gn < N ? gn : N - 1];
      }
      auto verdict = [&](float pa, float ga, float pa2, float ga2, float pw, float gw, bool la, bool lw) {
        bool flatA = f16_flat(row_min(ga), row_max(pa));
        if constexpr (TALL) flatA = flatA && f16_flat(row_min(ga2), row_max(pa2));
        bool flatW;
        if constexpr (WF) {
          flatW = (wflag & 2) == 0;
          lw = (wflag & 1) != 0;
        } else {
          flatW = f16_flat(row_min(gw), row_max(pw));
        }
        return (la ? F16_LOW_A : 0u) | (flatA ? 0u : F16_ROUGH_A) | (lw ? F16_LOW_W : 0u) | (flatW ? 0u : F16_ROUGH_W);
      };
      // exact scales, and the verdict bits at them
      auto exact_scales = [&]() {
        const float inf = __builtin_huge_valf();
        float RA = 0.0f, RA2 = 0.0f, RW = 0.0f, gA = inf, gA2 = inf, gW = inf, zA = inf, zA2 = inf, zW = inf;
#pragma unroll 4
        for (int kc = 0; kc < nk; ++kc) {
          load_chunk(kc * GBK);
          const float mA = amax8(ga[0], ga[1]);
          RA = fmaxf(RA, mA);
          zA = fminf(zA, mA);
          gA = fminf(gA, mA > 0.0f ? mA : inf);
          if constexpr (!WF) {
            const float mW = amax8(gw[0], gw[1]);
            RW = fmaxf(RW, mW);
            zW = fminf(zW, mW);
            gW = fminf(gW, mW > 0.0f ? mW : inf);
          }
          if constexpr (TALL) {
            const float mA2 = amax8(ga2[0], ga2[1]);
            RA2 = fmaxf(RA2, mA2);
            zA2 = fminf(zA2, mA2);
            gA2 = fminf(gA2, mA2 > 0.0f ? mA2 : inf);
          }
        }
        eA = f16_exp_row(row_max(RA));
        if constexpr (!WF) eW = f16_exp_row(row_max(RW));
        bool la = f16_lossy(gA * pow2i(eA));
        if constexpr (TALL) {
          eA2 = f16_exp_row(row_max(RA2));
          la = la || f16_lossy(gA2 * pow2i(eA2));
        }
        return verdict(RA, zA, RA2, zA2, RW, zW, la, f16_lossy(gW * pow2i(eW)));
      };
      auto set_scales = [&]() {
        scA = pow2i(eA);
        scA2 = pow2i(eA2);
        scW = pow2i(eW);
      };
      // one call site of the pass-0/1 loop (pass 0, or pass 1 after an exact scan); pass 2 has
      // its own two loops
      bool exact = short_k;
      for (int pass = 0; pass < 2; ++pass) {
        if (!exact) {
          load_chunk(0);
          const float mA = row_max(fmaxf(amax4(ga[0]), amax4(ga[1])));
          const float mA2 = TALL ? row_max(fmaxf(amax4(ga2[0]), amax4(ga2[1]))) : 1.0f;
          const float mW = WF ? 1.0f : row_max(fmaxf(amax4(gw[0]), amax4(gw[1])));
          eA = f16_exp_chunk(mA);
          if constexpr (TALL) eA2 = f16_exp_chunk(mA2);
          if constexpr (!WF) eW = f16_exp_chunk(mW);
          exact = tile_bits(mA == 0.0f || mA2 == 0.0f || mW == 0.0f) != 0;
        }
        if (exact) {
          const bool two = f16_needs_exact(tile_bits(exact_scales()));
          set_scales();
          if (two) {
            kloop(std::integral_constant<int, 1>{});
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
              for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] *= F16_LO_DOWN;
            kloop(std::integral_constant<int, 2>{});
            break;
          }
        } else {
          set_scales();
        }
        kloop(std::integral_constant<int, 0>{});
        if (exact) break;
        // every wave has left the loop (barrier above): its buffers may be restaged
        bool bad = false;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) bad = bad || !__builtin_isfinite(acc[i][j][r]);
        const unsigned t = tile_bits(verdict(pmaxA, pminA, pmaxA2, pminA2, pmaxW, pminW, lowA, lowW) |
                                     (bad ? F16_OVERFLOW : 0u));
        exact = (t & F16_OVERFLOW) != 0 || f16_needs_exact(t);
        if (!exact) break;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
      }
    }
    if constexpr (F16) {
      // undo the scales: output (row, column) times 2^-e(row) 2^-e(column), exact
      __shared__ float f16_rinv[2 * GBM], f16_cinv[GBN];
      if (sh == 0) {
        f16_rinv[sr] = pow2i(-eA);
        if constexpr (TALL) f16_rinv[128 + sr] = pow2i(-eA2);
        if constexpr (WF)
          f16_cinv[sr] = reinterpret_cast<const float*>(W2 + resident_frag_vectors(N, K))[gn < N ? gn : N - 1];
        else
          f16_cinv[sr] = pow2i(-eW);
      }
      __syncthreads();
      const float c0 = f16_cinv[wc + fr], c1 = f16_cinv[wc + 32 + fr];
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float rs = f16_rinv[wr + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3)];
          acc[i][0][r] = acc[i][0][r] * rs * c0;
          acc[i][1][r] = acc[i][1][r] * rs * c1;
        }
    }
  } else {
    // Global -> register staging: 2 float4 of A and 2 float4 of W per thread per chunk
    // (4 threads cover the 16 floats of one row).
    float* As = smem;                      // [2][GBM][GLDS]
    float* Bs = smem + 2 * GBM * GLDS;     // [2][GBN][GLDS]
    float4 ra[2], rb[2];
    auto load_chunk = [&](int k0) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int lin = tid + 256 * p;
        const int r = lin >> 2;
        const int kc = (lin & 3) * 4;
        const int64_t gr = row0 + r;
        const int gk = k0 + kc;
        ra[p] = (gr < M && gk < K) ? ld4(A + gr * lda + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
        const int gn = col0 + r;
        rb[p] = (gn < N && gk < K) ? ld4(W + (int64_t)gn * ldw + gk) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int lin = tid + 256 * p;
        const int r = lin >> 2;
        st4(&As[buf * GBM * GLDS + lds_chunk(r, lin & 3)], ra[p]);
        st4(&Bs[buf * GBN * GLDS + lds_chunk(r, lin & 3)], rb[p]);
      }
    };
    const int nk = (K + GBK - 1) / GBK;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int kc = 0; kc < nk; ++kc) {
      const int buf = kc & 1;
      if (kc + 1 < nk) load_chunk((kc + 1) * GBK);

      float af[2][8], bf[2][8];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float4 va = ld4(&As[buf * GBM * GLDS + lds_chunk(wr + i * 32 + fr, 2 * fh + q)]);
          const float4 vb = ld4(&Bs[buf * GBN * GLDS + lds_chunk(wc + i * 32 + fr, 2 * fh + q)]);
          af[i][4 * q + 0] = va.x; af[i][4 * q + 1] = va.y; af[i][4 * q + 2] = va.z; af[i][4 * q + 3] = va.w;
          bf[i][4 * q + 0] = vb.x; bf[i][4 * q + 1] = vb.y; bf[i][4 * q + 2] = vb.z; bf[i][4 * q + 3] = vb.w;
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][t], bf[j][t], acc[i][j], 0, 0, 0);
      }

      if (kc + 1 < nk) store_chunk(buf ^ 1);
      __syncthreads();
    }
  }

  // Accumulator layout of the 32x32 MFMA: lane l, register r -> column l%32,
  // row 8*(r/4) + 4*(l/32) + r%4.
  const int oc = lane & 31;
  const int orow = (lane >> 5) * 4;
  if constexpr (MODE >= 3) {
    // The two waves of a row half (2p: columns 0-63, 2p + 1: columns 64-127 of the group)
    // stage one 32-row slab each; then each of them normalises 16 of the slab's rows, 32
    // lanes per row and 4 columns per lane, with 32-lane butterfly sums for the statistics.
    const int grp = (int)blockIdx.y + n_tile;
    const int pair = wave >> 1;
    const float* wsl = smem + (2 * pair) * 32 * GES;
    const float* wsr = smem + (2 * pair + 1) * 32 * GES;
    const int sub = lane & 31, hl = lane >> 5;
    const int cl = 4 * sub;
    const float* src = (cl < 64 ? wsl : wsr) + (cl & 63);
    const float4 gm = ld4(ln.gamma + grp * LN_D + cl), bt = ld4(ln.beta + grp * LN_D + cl);
    float4 cb = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bias) cb = ld4(bias + col0 + cl);
    float4 lb = make_float4(0.f, 0.f, 0.f, 0.f);
    if (ln.ln_bias) lb = ld4(ln.ln_bias + grp * LN_D + cl);
    float* ws = smem + wave * 32 * GES;
    const bool tabs = ln.tab_src != nullptr;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      // this wave's 16 rows of the slab: lane k < 16 fetches row k's element ids (two
      // dependent loads) and, for the backward, its statistics, once per slab; each row's
      // values are then taken by shuffle.  The table rows and g_out of a row pair are loaded
      // one pair ahead of their use (the first before the slab is staged; loading all 8 pairs
      // ahead measured slower for the backward, 616 against 553 us at bcc Fe)
      const int64_t rbase = row0 + wr + i * 32 + (wave & 1) * 16;
      int64_t rk = rbase + (lane & 15);
      rk = rk < M ? rk : M - 1;
      int zs = 0, zd = 0;
      float mu = 0.0f, rsd = 0.0f;
      if (tabs) {
        zs = (int)ln.z[ln.isrc[rk]];
        zd = (int)ln.z[ln.idst[rk]];
      }
      if constexpr (MODE >= 4) {
        mu = ln.mean[rk * ln.G + grp];
        rsd = ln.rstd[rk * ln.G + grp];
      }
      // operands of row pair `it` (lanes 0-31: row 2 it, 32-63: row 2 it + 1)
      auto fetch = [&](int it, float4& t, float4& go) {
        const int k = 2 * it + hl;
        const int64_t gr = rbase + k;
        const int64_t rc = gr < M ? gr : M - 1;
        t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tabs) {
          const int a = __shfl(zs, k, 64), b = __shfl(zd, k, 64);
          t = ld4(ln.tab_src + (int64_t)a * ln.ldt + grp * LN_D + cl) + ld4(ln.tab_dst + (int64_t)b * ln.ldt + grp * LN_D + cl);
        }
        if constexpr (MODE == 4) go = ld4(ln.g_out + rc * ln.ldgo + grp * LN_D + cl);
        if constexpr (MODE == 5) go = ld4(ln.pre + rc * ln.ldpre + grp * LN_D + cl);  // v
      };
      constexpr int PD = 2;   // ring of row-pair operands: PD - 1 pairs in flight
      float4 tq[PD], gq[PD];
#pragma unroll
      for (int it = 0; it < PD - 1; ++it) fetch(it, tq[it], gq[it]);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) ws[(8 * (r >> 2) + orow + (r & 3)) * GES + j * 32 + oc] = acc[i][j][r];
      __syncthreads();
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        if (it + PD - 1 < 8) fetch(it + PD - 1, tq[(it + PD - 1) % PD], gq[(it + PD - 1) % PD]);
        const float4 tcur = tq[it % PD], gcur = gq[it % PD];
        const int k = 2 * it + hl;
        const int r = (wave & 1) * 16 + k;
        const int64_t gr = rbase + k;
        const bool live = gr < M;
        // the same additions in the same order as fu_ln_silu_grouped_* on a stored product
        const float4 p = ld4(src + r * GES) + cb;
        float4 v = p;
        if (tabs) v = v + tcur;
        if (ln.ln_bias) v = v + lb;
        if constexpr (MODE == 3) {
          if (ln.pre && live) st4_nt(ln.pre + gr * ln.ldpre + col0 + cl, p);
          const float mean = group_sum<32>(v.x + v.y + v.z + v.w) / LN_D;
          const float4 xc = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
          const float var = group_sum<32>(xc.x * xc.x + xc.y * xc.y + xc.z * xc.z + xc.w * xc.w) / LN_D;
          const float rstd = 1.0f / sqrtf(var + ln.eps);
          float4 y;
          y.x = xc.x * rstd * gm.x + bt.x;
          y.y = xc.y * rstd * gm.y + bt.y;
          y.z = xc.z * rstd * gm.z + bt.z;
          y.w = xc.w * rstd * gm.w + bt.w;
          if (live) {
            st4_nt(Y + gr * ldy + col0 + cl, make_float4(y.x * sigmoidf_(y.x), y.y * sigmoidf_(y.y),
                                                      y.z * sigmoidf_(y.z), y.w * sigmoidf_(y.w)));
            if (sub == 0) {
              ln.mean[gr * ln.G + grp] = mean;
              ln.rstd[gr * ln.G + grp] = rstd;
            }
          }
        } else {
          const float mean = __shfl(mu, k, 64), rstd = __shfl(rsd, k, 64);
          // MODE 4: v from the product, g_out loaded; MODE 5: the other way round
          const float4 x = MODE == 5 ? gcur : v, go = MODE == 5 ? v : gcur;
          const float xh[4] = {(x.x - mean) * rstd, (x.y - mean) * rstd, (x.z - mean) * rstd, (x.w - mean) * rstd};
          const float gg[4] = {gm.x, gm.y, gm.z, gm.w}, bb[4] = {bt.x, bt.y, bt.z, bt.w};
          const float gov[4] = {go.x, go.y, go.z, go.w};
          float gxh[4];
          float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float y = xh[q] * gg[q] + bb[q];
            const float sg = sigmoidf_(y);
            gxh[q] = gov[q] * (sg + y * sg * (1.0f - sg)) * gg[q];
            s1 += gxh[q];
            s2 += gxh[q] * xh[q];
          }
          s1 = group_sum<32>(s1);
          s2 = group_sum<32>(s2);
          if (live)
            st4_nt(Y + gr * ldy + col0 + cl,
                make_float4(rstd * (gxh[0] - (s1 + xh[0] * s2) / LN_D), rstd * (gxh[1] - (s1 + xh[1] * s2) / LN_D),
                            rstd * (gxh[2] - (s1 + xh[2] * s2) / LN_D), rstd * (gxh[3] - (s1 + xh[3] * s2) / LN_D)));
        }
      }
    }
    return;
  }
  if constexpr (MODE == 2) {
    // Stage 32-row slabs of g_Z in LDS; each lane then handles 16-byte pieces (4 channels of
    // one degree, inside one 32-channel group of the gate-paired order).
    const int C = gb.C, n1 = C / 32, L = gb.L;
    float* ws = smem + wave * 32 * GES;
    // A wave's 64 columns lie in one degree block kb (C is a multiple of 64), so the branch on
    // kb is uniform.  The global operands of a lane's pieces (the gate column and y of Y0, the
    // gate sums P1 (+ P2)) do not depend on the product: those of pieces 0-3 are loaded before
    // the slab is staged and those of pieces 4-7 before pieces 0-3 are computed, so their
    // latency overlaps the staging and the work before them; each is read once, with the
    // nontemporal hint (the complex gate backward 410 -> 397 us per launch, this one 527 -> 522).
    // A row past M loads row M - 1 and is not stored.
    const int gcw = col0 + wc;
    const int kb = gcw / C;
    // N is a multiple of 64, so a wave's columns are all below N or all at or past it; a wave
    // past N (the last column tile when N is not a multiple of 128) loads and stores nothing
    const bool wave_live = gcw < N;
    auto load_ops = [&](int i, int q, float4& gp, float4& y, float4& p) {
      if (!wave_live) return;
      const int lin = lane + 64 * q;
      int64_t gr = row0 + wr + i * 32 + (lin >> 4);
      gr = gr < M ? gr : M - 1;
      const int ch = gcw + (lin & 15) * 4 - kb * C;
      const float* y0 = gb.Y0 + gr * gb.ldy0;
      if (kb == 0) {
        y = ld4_nt(y0 + 2 * L * C + ch);
      } else {
        const int gate_col = 64 * ((kb - 1) * n1 + (ch >> 5)) + (ch & 31);
        gp = ld4_nt(y0 + gate_col);
        y = ld4_nt(y0 + gate_col + 32);
        p = ld4_nt(gb.P1 + gr * gb.ldp1 + (kb - 1) * C + ch);
        if (kb >= 2) p = p + ld4_nt(gb.P2 + gr * gb.ldp2 + (kb - 2) * C + ch);
      }
    };
    auto piece = [&](int i, int q, const float4& gp, const float4& y, const float4& p) {
      const int lin = lane + 64 * q;
      const int r = lin >> 4;
      const int c = (lin & 15) * 4;
      const int64_t gr = row0 + wr + i * 32 + r;
      const int gc = gcw + c;
      if (gr >= M || gc >= N) return;
      const float4 g = ld4(&ws[r * GES + c]);
      const int ch = gc - kb * C;
      float* out = Y + gr * ldy;
      if (kb == 0) {
        float4 o;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float yt = (&y.x)[t], sl = sigmoidf_(yt);
          (&o.x)[t] = (&g.x)[t] * (sl + yt * (sl * (1.0f - sl)));
        }
        st4_nt(out + 2 * L * C + ch, o);
      } else {
        const int gate_col = 64 * ((kb - 1) * n1 + (ch >> 5)) + (ch & 31);
        float4 og, ov;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float st = sigmoidf_((&gp.x)[t]), gt = (&g.x)[t];
          (&ov.x)[t] = gt * st;
          (&og.x)[t] = (st * (1.0f - st)) * (gt * (&y.x)[t] + (&p.x)[t]);
        }
        st4_nt(out + gate_col, og);
        st4_nt(out + gate_col + 32, ov);
      }
    };
    // split modes: a ring of four operand slots, two filled before the staging; piece q + 4 is
    // loaded into piece q's slot once q is done.  The fp32 mode (four workgroups per CU, 128
    // VGPRs) keeps one slot.
    constexpr int SLOTS = SPLIT ? 4 : 1, PRE = SPLIT ? 2 : 0;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      float4 gp[SLOTS], yv[SLOTS], pv[SLOTS];
#pragma unroll
      for (int q = 0; q < PRE; ++q) load_ops(i, q, gp[q], yv[q], pv[q]);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) ws[(8 * (r >> 2) + orow + (r & 3)) * GES + j * 32 + oc] = acc[i][j][r];
      __syncthreads();
#pragma unroll
      for (int q = PRE; q < SLOTS; ++q) load_ops(i, q, gp[q], yv[q], pv[q]);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        piece(i, q, gp[q % SLOTS], yv[q % SLOTS], pv[q % SLOTS]);
        if (q + SLOTS < 8) load_ops(i, q + SLOTS, gp[q % SLOTS], yv[q % SLOTS], pv[q % SLOTS]);
      }
    }
    return;
  }
  if constexpr (MODE == 1) {
    // Each wave stages its 32-row slabs of (gate | value) in LDS, then every lane handles
    // 16-byte pieces: Y rows (64 columns), and for gate pairs S and Z rows (32 columns).
    const int C = go.C, n1 = C / 32, L = go.L;
    const int q0 = col0 + wc;  // first column of this wave's pair
    const int p = q0 / 64;
    const bool live = q0 < N;
    float* ws = smem + wave * 32 * GES;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) ws[(8 * (r >> 2) + orow + (r & 3)) * GES + j * 32 + oc] = acc[i][j][r];
      __syncthreads();
      if (!live) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lin = lane + 64 * q;
        const int r = lin >> 3;
        const int c = (lin & 7) * 4;  // 0..28 within the 32-column half
        const int64_t row = row0 + wr + i * 32 + r;
        if (row >= M) continue;
        float4 g = ld4(&ws[r * GES + c]), v = ld4(&ws[r * GES + 32 + c]);
        if (bias) {
          g = g + ld4(bias + q0 + c);
          v = v + ld4(bias + q0 + 32 + c);
        }
        st4_nt(Y + row * ldy + q0 + c, g);
        st4_nt(Y + row * ldy + q0 + 32 + c, v);
        if (p < L * n1) {
          const int kind = p / n1;
          const int ch = 32 * (p - kind * n1) + c;
          const float4 sg = make_float4(sigmoidf_(g.x), sigmoidf_(g.y), sigmoidf_(g.z), sigmoidf_(g.w));
          if (go.S) st4_nt(go.S + row * go.lds + kind * C + ch, sg);
          st4_nt(go.Z + row * go.ldz + (1 + kind) * C + ch, v * sg);
        } else {
          const int ch = q0 - 2 * L * C + c;
          st4_nt(go.Z + row * go.ldz + ch,
              make_float4(g.x * sigmoidf_(g.x), g.y * sigmoidf_(g.y), g.z * sigmoidf_(g.z), g.w * sigmoidf_(g.w)));
          st4_nt(go.Z + row * go.ldz + ch + 32,
              make_float4(v.x * sigmoidf_(v.x), v.y * sigmoidf_(v.y), v.z * sigmoidf_(v.z), v.w * sigmoidf_(v.w)));
        }
      }
    }
    return;
  }
  // Each wave stages one 32x64 slab at a time in LDS and writes it back as rows of 16-byte
  // stores.
  float* ws = smem + wave * 32 * GES;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) ws[(8 * (r >> 2) + orow + (r & 3)) * GES + j * 32 + oc] = acc[i][j][r];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int lin = lane + 64 * q;
      const int r = lin >> 4;
      const int c = (lin & 15) * 4;
      const int64_t gr = row0 + wr + i * 32 + r;
      const int gc = col0 + wc + c;
      if (gr < M && gc < N) {
        float4 v = ld4(&ws[r * GES + c]);
        if (bias) {
          v.x += bias[gc]; v.y += bias[gc + 1]; v.z += bias[gc + 2]; v.w += bias[gc + 3];
        }
        if (rs.R) v = v + ld4(rs.R + gr * rs.ldr + gc);
        st4_nt(Y + gr * ldy + gc, v);
      }
    }
  }
}

}  // namespace fu

using namespace fu;

// Rows from which the split mode uses tall (256-row) tiles: below it the 128-row tiles keep
// more workgroups in flight than the CU count (the node GEMMs have 8,192 rows).
constexpr int64_t TALL_MIN_ROWS = 65536;

// Rows per tile of the kernel linear_kernel picks.
static int64_t linear_tile_rows(int64_t M) {
  return (matmul_mode() != FU_MATMUL_FP32 && M >= TALL_MIN_ROWS) ? 2 * GBM : GBM;
}

// The kernel for MODE in the current matrix-core mode; KTAIL instances handle K % 16 != 0.
template <int MODE, bool F16>
static auto split_kernel(int32_t K, bool tall) {
  return (K % GBK != 0)
             ? (tall ? linear_mfma_kernel<MODE, true, true, true, false, F16> : linear_mfma_kernel<MODE, true, true, false, false, F16>)
             : (tall ? linear_mfma_kernel<MODE, true, false, true, false, F16> : linear_mfma_kernel<MODE, true, false, false, false, F16>);
}
// The LayerNorm-SiLU GEMMs of the radial MLPs (K = 64 and 128): 128-row tiles in the
// split-fp16 mode, where their epilogue rather than the K loop bounds them; same-box A/B at
// bcc Fe, us per launch, tall -> 128 rows: first layer 400 -> 374, second 530 -> 512, first
// layer's backward 516 -> 480 (the plain batched GEMMs of the same K stay tall: 312 -> 336).
static int64_t ln_tile_rows(int32_t K, int64_t M) {
  return (K <= 128 && matmul_mode() == FU_MATMUL_SPLIT_F16) ? GBM : linear_tile_rows(M);
}

template <int MODE>
static auto linear_kernel(int32_t K, int64_t M, int64_t bm = 0) {
  const bool tall = (bm ? bm : linear_tile_rows(M)) != GBM;
  const int mode = matmul_mode();
  return mode == FU_MATMUL_FP32 ? linear_mfma_kernel<MODE, false>
         : mode == FU_MATMUL_SPLIT_F16 ? split_kernel<MODE, true>(K, tall) : split_kernel<MODE, false>(K, tall);
}

// With a pre-split weight (W2, fu_linear_weight_split of the same N x K weight): the tall fp16
// tile reading its weight fragments from W2 (split-fp16 mode, tall tiles, K % 16 == 0);
// otherwise W2 is not used.
static bool use_w2(const void* W2, int32_t K, int64_t M) {
  return W2 != nullptr && matmul_mode() == FU_MATMUL_SPLIT_F16 && linear_tile_rows(M) != GBM && K % GBK == 0;
}
template <int MODE>
static auto linear_kernel_w2(int32_t K, int64_t M, const void* W2) {
  return use_w2(W2, K, M) ? linear_mfma_kernel<MODE, true, false, true, false, true, true> : linear_kernel<MODE>(K, M);
}
static int w2_check(const void* W2, const char* who) {
  return (W2 && !aligned16(W2)) ? set_error(FU_ERR_ALIGN, "%s: W2 must be 16-byte aligned", who) : FU_OK;
}

static int linear_check(const float* A, int64_t lda, const float* W, int64_t ldw, const float* Y, int64_t ldy,
                        int64_t M, int32_t N, int32_t K, const char* who) {
  if (M < 0 || N <= 0 || K <= 0)
    return set_error(FU_ERR_SHAPE, "%s: bad shape M=%lld N=%d K=%d", who, (long long)M, N, K);
  if (K % 4 != 0 || lda % 4 != 0 || ldw % 4 != 0)
    return set_error(FU_ERR_UNSUPPORTED, "%s: K=%d, lda=%lld, ldw=%lld must be multiples of 4", who, K,
                     (long long)lda, (long long)ldw);
  if (N % 4 != 0 || ldy % 4 != 0)
    return set_error(FU_ERR_UNSUPPORTED, "%s: N=%d and ldy=%lld must be multiples of 4", who, N, (long long)ldy);
  if (lda < K || ldw < K || ldy < N) return set_error(FU_ERR_SHAPE, "%s: leading dimensions smaller than the rows", who);
  if (M == 0) return FU_OK;  // no rows: the operands may be empty (NULL) arrays
  if (!A || !W || !Y) return set_error(FU_ERR_NULL, "%s: NULL operand", who);
  if (!aligned16(A) || !aligned16(W) || !aligned16(Y))
    return set_error(FU_ERR_ALIGN, "%s: operands must be 16-byte aligned", who);
  return FU_OK;
}

static int linear_launch(const float* A, int64_t lda, int64_t sA, const float* W, int64_t ldw, int64_t sW,
                         const float* bias, int64_t sBias, int32_t bias_batches, float* Y, int64_t ldy, int64_t sY,
                         int64_t M, int32_t N, int32_t K, int32_t batch, hipStream_t stream, const char* who,
                         Resid rs = Resid{}, const void* W2 = nullptr) {
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = linear_tile_rows(M);
  const int64_t m_tiles = (M + bm - 1) / bm;
  const int64_t total = m_tiles * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  auto kern = linear_kernel_w2<0>(K, M, W2);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, (unsigned)batch), dim3(256), 0, stream, A, lda, sA, W, ldw, sW, bias,
                     sBias, bias_batches, Y, ldy, sY, M, N, K, n_tiles, total, GateOut{}, GateBwd{}, rs, LnEpi{}, GatherA{},
                     static_cast<const uint4*>(W2));
  return check_launch(who);
}

extern "C" int fu_linear(const float* A, int64_t lda, const float* W, int64_t ldw, const float* bias, float* Y,
                         int64_t ldy, int64_t M, int32_t N, int32_t K, const void* W2, void* stream) {
  int st = linear_check(A, lda, W, ldw, Y, ldy, M, N, K, "fu_linear");
  if (st == FU_OK) st = w2_check(W2, "fu_linear");
  if (st != FU_OK) return st;
  if (M == 0) return FU_OK;
  return linear_launch(A, lda, 0, W, ldw, 0, bias, 0, 1, Y, ldy, 0, M, N, K, 1, as_stream(stream), "fu_linear",
                       Resid{}, W2);
}

extern "C" int fu_linear_batched(const float* A, int64_t lda, int64_t stride_a, const float* W, int64_t ldw,
                                 int64_t stride_w, const float* bias, int64_t stride_bias, int32_t bias_batches,
                                 const float* R, int64_t ldr, int64_t stride_r, float* Y, int64_t ldy,
                                 int64_t stride_y, int64_t M, int32_t N, int32_t K, int32_t batch, void* stream) {
  int st = linear_check(A, lda, W, ldw, Y, ldy, M, N, K, "fu_linear_batched");
  if (st != FU_OK) return st;
  if (batch < 1 || batch > 65535) return set_error(FU_ERR_SHAPE, "fu_linear_batched: batch=%d out of range", batch);
  if ((stride_a | stride_w | stride_y) % 4 != 0 || stride_a < 0 || stride_w < 0 || stride_y < 0)
    return set_error(FU_ERR_ALIGN, "fu_linear_batched: batch strides must be non-negative multiples of 4");
  if (R && ((ldr | stride_r) % 4 != 0 || ldr < N || stride_r < 0 || !aligned16(R)))
    return set_error(FU_ERR_ALIGN, "fu_linear_batched: R must be 16-byte aligned with ldr >= N, strides multiples of 4");
  if (M == 0) return FU_OK;
  return linear_launch(A, lda, stride_a, W, ldw, stride_w, bias, stride_bias, bias_batches, Y, ldy, stride_y, M, N, K,
                       batch, as_stream(stream), "fu_linear_batched", Resid{R, ldr, stride_r});
}

extern "C" int fu_linear_gate(const float* A, int64_t lda, const float* W, int64_t ldw, const float* bias, float* Y,
                              int64_t ldy, float* Z, int64_t ldz, float* S, int64_t lds, int64_t M, int32_t C,
                              int32_t K, int32_t lmax, const void* W2, void* stream) {
  const char* who = "fu_linear_gate";
  if (w2_check(W2, who) != FU_OK) return FU_ERR_ALIGN;
  if (C <= 0 || C % 64 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 64", who, C);
  if (lmax < 2 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d unsupported (2, 3 or 4)", who, lmax);
  const int32_t N = (2 * lmax + 1) * C;
  int st = linear_check(A, lda, W, ldw, Y, ldy, M, N, K, who);
  if (st != FU_OK) return st;
  if (ldz < (lmax + 1) * C || (S && lds < lmax * C))
    return set_error(FU_ERR_SHAPE, "%s: Z / S row strides too small", who);
  if (M == 0) return FU_OK;
  if (!Z) return set_error(FU_ERR_NULL, "%s: NULL output", who);
  if (ldz % 4 != 0 || !aligned16(Z) || (S && (lds % 4 != 0 || !aligned16(S))) || (bias && !aligned16(bias)))
    return set_error(FU_ERR_ALIGN, "%s: Z, S and bias must be 16-byte aligned with row strides multiples of 4", who);
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = linear_tile_rows(M);
  const int64_t total = ((M + bm - 1) / bm) * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  auto kern = linear_kernel_w2<1>(K, M, W2);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, 1u), dim3(256), 0, as_stream(stream), A, lda,
                     (int64_t)0, W, ldw, (int64_t)0, bias, (int64_t)0, 1, Y, ldy, (int64_t)0, M, N, K, n_tiles, total,
                     GateOut{Z, ldz, S, lds, C, lmax}, GateBwd{}, Resid{}, LnEpi{}, GatherA{},
                     static_cast<const uint4*>(W2));
  return check_launch(who);
}

extern "C" int fu_gather_linear_gate(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                                     const float* rad, const float* csd, const int64_t* batch, const float* W,
                                     int64_t ldw, const float* bias, float* Y, int64_t ldy, float* Z, int64_t ldz,
                                     int64_t E, int32_t C, void* stream) {
  const char* who = "fu_gather_linear_gate";
  if (C <= 0 || C % 64 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 64", who, C);
  if (matmul_mode() == FU_MATMUL_FP32)
    return set_error(FU_ERR_UNSUPPORTED, "%s: only in the split matrix-core modes", who);
  const int32_t lmax = 2, K = 6 * C, N = 5 * C;
  if (E < 0) return set_error(FU_ERR_SHAPE, "%s: E=%lld", who, (long long)E);
  if (ldw < K || ldy < N || ldz < 3 * C || (ldw | ldy | ldz) % 4 != 0)
    return set_error(FU_ERR_SHAPE, "%s: ldw >= 6C, ldy >= 5C, ldz >= 3C (multiples of 4) required", who);
  if (E == 0) return FU_OK;
  if (!x || !idx_i || !idx_j || !wigner || !rad || !csd || !batch || !W || !Y || !Z)
    return set_error(FU_ERR_NULL, "%s: NULL operand", who);
  if (!aligned16(x) || !aligned16(rad) || !aligned16(csd) || !aligned16(W) || !aligned16(Y) || !aligned16(Z) ||
      (bias && !aligned16(bias)))
    return set_error(FU_ERR_ALIGN, "%s: x, rad, csd, W, bias, Y and Z must be 16-byte aligned", who);
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = linear_tile_rows(E);
  const int64_t total = ((E + bm - 1) / bm) * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: E too large", who);
  // the gathered loader keeps the bf16 split in both split modes: its per-row gather state and
  // the fp16 scales together exceed the register file of the tall tile
  auto kern = bm != GBM ? linear_mfma_kernel<1, true, false, true, true> : linear_mfma_kernel<1, true, false, false, true>;
  // A is unused (the loader gathers it); x stands in as a valid pointer
  hipLaunchKernelGGL(kern, dim3((unsigned)total, 1u), dim3(256), 0, as_stream(stream), x, (int64_t)0, (int64_t)0, W,
                     ldw, (int64_t)0, bias, (int64_t)0, 1, Y, ldy, (int64_t)0, E, N, K, n_tiles, total,
                     GateOut{Z, ldz, nullptr, 0, C, lmax}, GateBwd{}, Resid{}, LnEpi{},
                     GatherA{x, idx_i, idx_j, wigner, rad, csd, batch, C}, (const uint4*)nullptr);
  return check_launch(who);
}

extern "C" int fu_linear_gate_bwd(const float* gZo, int64_t ldgz, const float* Wt, int64_t ldw, const float* Y0,
                                  int64_t ldy0, const float* P1, int64_t ldp1, const float* P2, int64_t ldp2,
                                  float* gY0, int64_t ldg, int64_t M, int32_t C, int32_t K, int32_t lmax,
                                  const void* W2, void* stream) {
  const char* who = "fu_linear_gate_bwd";
  if (w2_check(W2, who) != FU_OK) return FU_ERR_ALIGN;
  if (C <= 0 || C % 64 != 0) return set_error(FU_ERR_UNSUPPORTED, "%s: C=%d must be a multiple of 64", who, C);
  if (lmax < 2 || lmax > 4) return set_error(FU_ERR_UNSUPPORTED, "%s: lmax=%d unsupported (2, 3 or 4)", who, lmax);
  const int32_t N = (lmax + 1) * C;
  // the GEMM's own output (g_Z_m0, N = (L+1)C columns) is never stored; gY0 ((2L+1)C) is checked here
  int st = linear_check(gZo, ldgz, Wt, ldw, gY0, ldg, M, N, K, who);
  if (st != FU_OK) return st;
  if (ldg < (2 * lmax + 1) * C || ldy0 < (2 * lmax + 1) * C || ldp1 < lmax * C || ldp2 < (lmax - 1) * C)
    return set_error(FU_ERR_SHAPE, "%s: row strides too small", who);
  if (M == 0) return FU_OK;
  if (!Y0 || !P1 || !P2) return set_error(FU_ERR_NULL, "%s: NULL operand", who);
  if ((ldy0 | ldp1 | ldp2) % 4 != 0 || !aligned16(Y0) || !aligned16(P1) || !aligned16(P2))
    return set_error(FU_ERR_ALIGN, "%s: operands must be 16-byte aligned with row strides multiples of 4", who);
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = linear_tile_rows(M);
  const int64_t total = ((M + bm - 1) / bm) * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  auto kern = linear_kernel_w2<2>(K, M, W2);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, 1u), dim3(256), 0, as_stream(stream), gZo, ldgz,
                     (int64_t)0, Wt, ldw, (int64_t)0, (const float*)nullptr, (int64_t)0, 1, gY0, ldg, (int64_t)0, M, N,
                     K, n_tiles, total, GateOut{}, GateBwd{Y0, ldy0, P1, ldp1, P2, ldp2, C, lmax}, Resid{}, LnEpi{}, GatherA{},
                     static_cast<const uint4*>(W2));
  return check_launch(who);
}

// Shared checks of the LayerNorm-SiLU GEMMs: whole 128-column groups, one per N-tile or per
// batch, and the LayerNorm operands.
static int ln_epi_check(const char* who, int64_t M, int32_t N, int32_t batch, int32_t G, const float* tab_src,
                        const float* tab_dst, int64_t ldt, const int64_t* z, const int64_t* isrc, const int64_t* idst,
                        const float* ln_bias, const float* gamma, const float* beta, const float* mean,
                        const float* rstd) {
  if (N % LN_D != 0 || G < 1 || !((batch == 1 && N == LN_D * G) || (N == LN_D && batch == G)))
    return set_error(FU_ERR_UNSUPPORTED,
                     "%s: N=%d, batch=%d, G=%d: the row must be G groups of 128 columns, one per N-tile or per batch",
                     who, N, batch, G);
  if (M == 0) return FU_OK;  // no rows: the per-row arrays may be empty (NULL)
  if (!gamma || !beta || !mean || !rstd) return set_error(FU_ERR_NULL, "%s: NULL LayerNorm operand", who);
  if (tab_src && (!tab_dst || !z || !isrc || !idst || ldt < (int64_t)G * LN_D || ldt % 4 != 0))
    return set_error(FU_ERR_SHAPE, "%s: element tables need tab_dst, z, isrc, idst and ldt >= %d (multiple of 4)", who,
                     G * LN_D);
  if (!aligned16(gamma) || !aligned16(beta) || (ln_bias && !aligned16(ln_bias)) ||
      (tab_src && (!aligned16(tab_src) || !aligned16(tab_dst))))
    return set_error(FU_ERR_ALIGN, "%s: gamma, beta, ln_bias and the tables must be 16-byte aligned", who);
  return FU_OK;
}

extern "C" int fu_linear_ln_silu(const float* A, int64_t lda, int64_t stride_a, const float* W, int64_t ldw,
                                 int64_t stride_w, const float* bias, int64_t stride_bias, int32_t bias_batches,
                                 float* Y, int64_t ldy, int64_t stride_y, float* pre, int64_t ldpre, int64_t stride_pre,
                                 int64_t M, int32_t N, int32_t K, int32_t batch, const float* tab_src,
                                 const float* tab_dst, int64_t ldt, const int64_t* z, const int64_t* isrc,
                                 const int64_t* idst, const float* ln_bias, const float* gamma, const float* beta,
                                 float* mean, float* rstd, int32_t G, float eps, void* stream) {
  const char* who = "fu_linear_ln_silu";
  int st = linear_check(A, lda, W, ldw, Y, ldy, M, N, K, who);
  if (st != FU_OK) return st;
  if (batch < 1 || batch > 65535) return set_error(FU_ERR_SHAPE, "%s: batch=%d out of range", who, batch);
  st = ln_epi_check(who, M, N, batch, G, tab_src, tab_dst, ldt, z, isrc, idst, ln_bias, gamma, beta, mean, rstd);
  if (st != FU_OK) return st;
  if ((stride_a | stride_w | stride_y | stride_pre) % 4 != 0 || stride_a < 0 || stride_w < 0 || stride_y < 0 ||
      stride_pre < 0)
    return set_error(FU_ERR_ALIGN, "%s: batch strides must be non-negative multiples of 4", who);
  if (pre && (ldpre < N || ldpre % 4 != 0 || !aligned16(pre)))
    return set_error(FU_ERR_ALIGN, "%s: pre must be 16-byte aligned with ldpre >= N, a multiple of 4", who);
  if (bias && !aligned16(bias)) return set_error(FU_ERR_ALIGN, "%s: bias must be 16-byte aligned", who);
  if (M == 0) return FU_OK;
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = ln_tile_rows(K, M);
  const int64_t total = ((M + bm - 1) / bm) * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  auto kern = linear_kernel<3>(K, M, bm);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, (unsigned)batch), dim3(256), 0, as_stream(stream), A, lda, stride_a,
                     W, ldw, stride_w, bias, stride_bias, bias_batches, Y, ldy, stride_y, M, N, K, n_tiles, total,
                     GateOut{}, GateBwd{}, Resid{},
                     LnEpi{tab_src, tab_dst, ldt, z, isrc, idst, ln_bias, gamma, beta, mean, rstd, G, eps, pre, ldpre,
                           stride_pre, nullptr, 0}, GatherA{}, (const uint4*)nullptr);
  return check_launch(who);
}

extern "C" int fu_linear_ln_silu_bwd(const float* A, int64_t lda, const float* W, int64_t ldw, float* g_x, int64_t ldgx,
                                     int64_t M, int32_t N, int32_t K, const float* g_out, int64_t ldgo,
                                     const float* tab_src, const float* tab_dst, int64_t ldt, const int64_t* z,
                                     const int64_t* isrc, const int64_t* idst, const float* ln_bias,
                                     const float* gamma, const float* beta, const float* mean, const float* rstd,
                                     int32_t G, void* stream) {
  const char* who = "fu_linear_ln_silu_bwd";
  int st = linear_check(A, lda, W, ldw, g_x, ldgx, M, N, K, who);
  if (st != FU_OK) return st;
  st = ln_epi_check(who, M, N, 1, G, tab_src, tab_dst, ldt, z, isrc, idst, ln_bias, gamma, beta, mean, rstd);
  if (st != FU_OK) return st;
  if (M == 0) return FU_OK;
  if (!g_out || ldgo < N || ldgo % 4 != 0 || !aligned16(g_out))
    return set_error(FU_ERR_ALIGN, "%s: g_out must be 16-byte aligned with ldgo >= N, a multiple of 4", who);
  const int n_tiles = (N + GBN - 1) / GBN;
  const int64_t bm = ln_tile_rows(K, M);
  const int64_t total = ((M + bm - 1) / bm) * n_tiles;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  auto kern = linear_kernel<4>(K, M, bm);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, 1u), dim3(256), 0, as_stream(stream), A, lda, (int64_t)0, W, ldw,
                     (int64_t)0, (const float*)nullptr, (int64_t)0, 0, g_x, ldgx, (int64_t)0, M, N, K, n_tiles, total,
                     GateOut{}, GateBwd{}, Resid{},
                     LnEpi{tab_src, tab_dst, ldt, z, isrc, idst, ln_bias, gamma, beta, const_cast<float*>(mean),
                           const_cast<float*>(rstd), G, 0.0f, nullptr, 0, 0, g_out, ldgo}, GatherA{},
                     (const uint4*)nullptr);
  return check_launch(who);
}

extern "C" int fu_linear_dgrad_ln_silu_bwd(const float* A, int64_t lda, const float* W, int64_t ldw, float* g_x,
                                           int64_t ldgx, int64_t M, int32_t K, const float* x, int64_t ldx,
                                           const float* gamma, const float* beta, const float* mean, const float* rstd,
                                           int32_t G, int32_t group, const void* W2, void* stream) {
  const char* who = "fu_linear_dgrad_ln_silu_bwd";
  if (w2_check(W2, who) != FU_OK) return FU_ERR_ALIGN;
  int st = linear_check(A, lda, W, ldw, g_x, ldgx, M, LN_D, K, who);
  if (st != FU_OK) return st;
  if (G < 1 || group < 0 || group >= G)
    return set_error(FU_ERR_SHAPE, "%s: group=%d outside [0, G=%d)", who, group, G);
  if (ldx < (int64_t)G * LN_D || ldx % 4 != 0)
    return set_error(FU_ERR_SHAPE, "%s: ldx=%lld must be >= 128 G and a multiple of 4", who, (long long)ldx);
  if (M == 0) return FU_OK;
  if (!x || !gamma || !beta || !mean || !rstd) return set_error(FU_ERR_NULL, "%s: NULL LayerNorm operand", who);
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(beta))
    return set_error(FU_ERR_ALIGN, "%s: x, gamma and beta must be 16-byte aligned", who);
  const int64_t bm = linear_tile_rows(M);
  const int64_t total = (M + bm - 1) / bm;
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: M too large", who);
  // the kernel addresses group 0 of its operands; the group's columns and statistics are
  // selected here
  const int64_t go = (int64_t)group * LN_D;
  auto kern = linear_kernel_w2<5>(K, M, W2);
  hipLaunchKernelGGL(kern, dim3((unsigned)total, 1u), dim3(256), 0, as_stream(stream), A, lda, (int64_t)0, W, ldw,
                     (int64_t)0, (const float*)nullptr, (int64_t)0, 0, g_x, ldgx, (int64_t)0, M, (int32_t)LN_D, K, 1,
                     total, GateOut{}, GateBwd{}, Resid{},
                     LnEpi{nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, gamma + go, beta + go,
                           const_cast<float*>(mean) + group, const_cast<float*>(rstd) + group, G, 0.0f,
                           const_cast<float*>(x) + go, ldx, 0, nullptr, 0}, GatherA{}, static_cast<const uint4*>(W2));
  return check_launch(who);
}
