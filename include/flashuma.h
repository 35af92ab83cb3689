/*
 * flashuma.h — C-ABI of libflashuma_hip.so, the gfx950 (MI355X) kernels behind the
 * FlashUMA ZeroAllocBackbone hot path.
 *
 * Conventions shared by every entry point:
 *   - All tensors are device pointers to dense, row-major (C-contiguous) arrays.
 *     Features are fp32, graph indices are int64 (edge_index, Z, batch) and CSR arrays
 *     are int32, exactly as in the reference (model.py:20-26 and the ops/ modules).
 *   - Sizes are int64_t (E, N, M) or int32_t (channel widths).  Edge-feature offsets are
 *     computed in 64 bits, so E * row_width may exceed 2^31.
 *   - `stream` is a hipStream_t passed as void*; work is only enqueued, never awaited.
 *   - Zero rows: with E = 0 (or M, n = 0) an entry point writes only what it owes per
 *     node (a scatter's residual copy, a zeroed node gradient, a CSR of zeros) and arrays
 *     sized by the zero count may be NULL, as the storage of an empty torch tensor is.
 *     An isolated atom or a graph without edges therefore needs no special casing.
 *   - No entry point allocates memory.  Scratch space, where needed, is an argument.
 *   - Return value: FU_OK (0) or a negative FU_ERR_* code; fu_last_error() returns the
 *     message of the last failure on the calling host thread.
 *
 * Edge layout contract (ops/constants.py:7-35): wigner is (E, 34) = row-major L=1 3x3
 * block (0..8) then L=2 5x5 block (9..33).  Rotated-frame m-blocks are
 *   X_m0 (E, 6C)  X_m1 (E, 8C)  X_m2 (E, 4C)     (gather output / conv1 input)
 *   Y_m0 (E, 5C)  Y_m1 (E, 4C)  Y_m2 (E, 2C)     (conv1 output / gate input)
 *   Z_m0 (E, 3C)  Z_m1 (E, 4C)  Z_m2 (E, 2C)     (gate output, conv2 in/out)
 * with the slot orders of ops/gather.py:132-154 and ops/gating.py:63-103.
 */
#ifndef FLASHUMA_H_
#define FLASHUMA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FU_OK 0
#define FU_ERR_SHAPE (-1)       /* a size is negative, zero where it may not be, or unsupported */
#define FU_ERR_UNSUPPORTED (-2) /* a configuration the kernels do not implement */
#define FU_ERR_ALIGN (-3)       /* a pointer lacks the alignment the vector loads need */
#define FU_ERR_LAUNCH (-4)      /* the HIP runtime rejected a launch */
#define FU_ERR_NULL (-5)        /* a required pointer is NULL */
#define FU_ERR_WORKSPACE (-6)   /* the workspace is too small */

/* Library version (major*10000 + minor*100 + patch): 600 (0.6.0) for the signatures in this
 * header.  0.2.0 added the int32 `accumulate` argument (before the stream) of fu_gather_bwd,
 * fu_scatter_bwd, fu_init_scatter_bwd, their _lmax forms and fu_complex_linear_gate(_bwd), and
 * dropped one pointer/stride pair of fu_linear_gate_bwd; 0.3.0 changed the layout and size of
 * the fu_complex_weight_split buffer (fu_complex_weight_split_bytes) and added the four CSR
 * arguments of fu_gather_fwd_lmax; 0.4.0 added fu_linear_weight_split_bytes,
 * fu_linear_weight_split and fu_linear_resident (nothing changed); 0.5.0 added the W2 argument
 * (before the stream) of fu_linear, fu_linear_gate, fu_linear_gate_bwd and
 * fu_linear_dgrad_ln_silu_bwd; 0.6.0 added fu_radial_gather_fwd, fu_radial_gather_perm and
 * their _lmax forms (nothing changed).  A caller built against
 * another version must not call into this library. */
int fu_version(void);

/* Message of the last error returned on the calling host thread ("" if none). */
const char* fu_last_error(void);

/* Matrix-core mode of every fp32 contraction (fu_linear*, fu_complex_linear*); no reference
 * counterpart (the reference's dense layers are cuBLAS fp32 GEMMs with TF32 off, model.py:152,154,
 * reached through torch.nn.functional.linear).
 *   0: each fp32 operand is split exactly into three bf16 planes (x = hi + mid + lo)
 *      and the six significant partial products run on v_mfma_f32_32x32x16_bf16 with fp32
 *      accumulation; error against fp64 at or below that of the fp32 MFMA.
 *   1: v_mfma_f32_32x32x2_f32.
 *   2 (default): each operand row (a row of A, or a row of W: an output column) is scaled by a power of
 *      two, each element split into two fp16 values (x 2^e = hi + lo, 22 significant bits) and
 *      three partial products run on v_mfma_f32_32x32x16_f16 with fp32 accumulation, unscaled
 *      exactly afterwards.  Scales come from the row's first 16 elements (or, for K <= 64, from
 *      the whole row); a tile whose 8-element pieces leave the fp16 window while the other
 *      operand is not flat (or that overflows) is computed again with exact scales, in two K
 *      loops with 2^11-scaled residuals when needed (split_f16.h states the rules).  Row-relative
 *      error against fp64 at most 1.1x (rms) / 1.5x (max) that of the fp32 MFMA on the tested
 *      shapes and operand families.  fu_gather_linear_gate and
 *      fu_complex_linear* without W3 keep the bf16 split in this mode.
 * The mode is process-wide and read at each launch; switch it only between launches.
 * fu_set_matmul_mode returns FU_OK or FU_ERR_UNSUPPORTED; fu_matmul_mode returns the mode. */
int fu_set_matmul_mode(int32_t mode);
int fu_matmul_mode(void);

/* ------------------------------------------------------------------------------------
 * Geometry (replaces PrecomputeGeometry, ops/geom.py:496-589)
 * ------------------------------------------------------------------------------------ */

/* Per-edge geometry, ops/geom.py:36-214 (_geom_fwd_kernel).
 * d = pos[idx_i] - pos[idx_j] + shifts[e]; env = polynomial envelope; the B Gaussians
 * exp(coeff_g (|d| - offset_g[b])^2) go to x_edge_raw[e, 0:B]; when W_src and W_tgt are
 * non-NULL, W_src[Z[idx_i]] and W_tgt[Z[idx_j]] (each C wide) go to x_edge_raw[e, B:B+2C].
 * ld_xe is the row stride of x_edge_raw in floats (>= B, or >= B+2C with embeddings).
 * wigner receives the 34 quaternion-Wigner scalars of the edge frame. */
int fu_geom_fwd(const float* pos, const int64_t* Z, const int64_t* idx_i, const int64_t* idx_j,
                const float* shifts, const float* W_src, const float* W_tgt, const float* offset_g,
                float* x_edge_raw, int64_t ld_xe, float* wigner, float* env, int64_t E, int64_t N,
                int32_t B, int32_t C, float cutoff, float coeff_g, void* stream);

/* Per-edge vector-Jacobian product of fu_geom_fwd w.r.t. the edge vector d,
 * ops/geom.py:220-493 (_geom_bwd_kernel) without its atomics: writes g_d (E, 3), which is
 * also dE/dshifts (ops/geom.py:490-493).  g_x_edge_raw (row stride ld_gxe; only columns
 * 0..B-1 are read), g_wigner and g_env may each be NULL (treated as zero). */
int fu_geom_bwd(const float* pos, const int64_t* idx_i, const int64_t* idx_j, const float* shifts,
                const float* offset_g, const float* g_x_edge_raw, int64_t ld_gxe,
                const float* g_wigner, const float* g_env, float* g_d, int64_t E, int64_t N,
                int32_t B, float cutoff, float coeff_g, void* stream);

/* Deterministic replacement for the g_pos atomics of ops/geom.py:483-488:
 * g_pos[n] = sum_{e in send(n)} g_d[e] - sum_{e in recv(n)} g_d[e], summed in CSR order
 * in fp64.  send/recv are CSRs over senders (idx_i) and receivers (idx_j). */
int fu_edge_vec_reduce(const float* g_d, const int32_t* recv_ptr, const int32_t* recv_idx,
                       const int32_t* send_ptr, const int32_t* send_idx, float* g_pos, int64_t N,
                       int64_t E, void* stream);

/* ------------------------------------------------------------------------------------
 * Gather-rotate (replaces GatherWignerSplit, ops/gather.py:408-514)
 * ------------------------------------------------------------------------------------ */

/* ops/gather.py:34-154 (_gather_split_fwd_kernel): rotate sender/receiver rows of
 * x (N, 9, C) (+ csd_emb[batch] on l=0) into the edge frame, scale by rad (E, 12C) and
 * write the X_m0/X_m1/X_m2 blocks.
 * layout 0: the reference column-block order of X and rad (sender/receiver slots
 * interleaved, ops/gather.py:132-154).  layout 1: X_m0 and rad side-major (all sender
 * blocks, then all receiver blocks); X_m1 as [real half | imaginary half], each half
 * side-major; X_m2 in reference order.  The model pairs it with conv1 / radial weights
 * permuted the same way, which leaves every product unchanged.  X_m0 may be NULL: the m = 0
 * blocks are then not formed (fu_gather_linear_gate gathers them inside conv1 m = 0). */
int fu_gather_fwd(const float* x, const int64_t* idx_i, const int64_t* idx_j, const float* wigner,
                  const float* rad, const float* csd_emb, const int64_t* batch, float* X_m0,
                  float* X_m1, float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C,
                  int32_t layout, void* stream);

/* ops/gather.py:160-405 (both backward kernels) without atomics.  One workgroup per node
 * sums the node's receiver segment (recv CSR) and sender segment (send CSR) in CSR order,
 * writing g_x (N, 9, C), g_rad (E, 12C) and g_wigner (E, 34).  g_wig_ws is an (E, 34)
 * scratch array for the sender-side halves of g_wigner.  layout as in fu_gather_fwd (g_X and
 * g_rad use the same order as X and rad).  accumulate: bit 0 set adds this call's g_wigner to
 * the array's contents instead of overwriting it (the model sums the contributions of all its
 * blocks in place this way, replacing the per-tensor sums autograd would add; bit 1, used by
 * the scatters for g_env, is ignored here). */
int fu_gather_bwd(const float* g_X_m0, const float* g_X_m1, const float* g_X_m2, const float* x,
                  const int64_t* idx_i, const int64_t* idx_j, const float* wigner, const float* rad,
                  const float* csd_emb, const int64_t* batch, const int32_t* recv_ptr,
                  const int32_t* recv_idx, const int32_t* send_ptr, const int32_t* send_idx,
                  float* g_x, float* g_wigner, float* g_rad, float* g_wig_ws, int64_t E,
                  int64_t N, int64_t S, int32_t C, int32_t layout, int32_t accumulate,
                  void* stream);

/* ------------------------------------------------------------------------------------
 * Gate activation (replaces FusedGatingSplit, ops/gating.py:188-234)
 * ------------------------------------------------------------------------------------ */

/* ops/gating.py:32-103 (_gating_split_fwd_kernel).  layout 0: Y_m0 in the reference column
 * order [gate_l1, gate_l2, y_l0, y_l1m0, y_l2m0]; layout 1: the gate-paired order of
 * fu_linear_gate (64-column pairs [gate_l1 | y_l1m0] x C/32, [gate_l2 | y_l2m0] x C/32, then
 * y_l0; C a multiple of 64). */
int fu_gating_fwd(const float* Y_m0, const float* Y_m1, const float* Y_m2, float* Z_m0,
                  float* Z_m1, float* Z_m2, int64_t E, int32_t C, int32_t layout, void* stream);

/* ops/gating.py:109-185 (_gating_split_bwd_kernel).  layout as in fu_gating_fwd, for Y_m0 and
 * g_Y_m0. */
int fu_gating_bwd(const float* g_Z_m0, const float* g_Z_m1, const float* g_Z_m2, const float* Y_m0,
                  const float* Y_m1, const float* Y_m2, float* g_Y_m0, float* g_Y_m1,
                  float* g_Y_m2, int64_t E, int32_t C, int32_t layout, void* stream);

/* ------------------------------------------------------------------------------------
 * Rotate-scatter (replaces RotateScatterSplit, ops/scatter.py:295-352)
 * ------------------------------------------------------------------------------------ */

/* ops/scatter.py:45-140 (_scatter_split_fwd_kernel): x_out[j] = x_res[j] +
 * sum_{e in CSR(j)} env_e * D_e^T * Zout_e, accumulated in fp64 in CSR order. */
int fu_scatter_fwd(const int32_t* row_ptr, const int32_t* col_idx, const float* Z_m0,
                   const float* Z_m1, const float* Z_m2, const float* wigner, const float* env,
                   const float* x_res, float* x_out, int64_t N, int64_t E, int32_t C,
                   void* stream);

/* ops/scatter.py:146-292 (both backward kernels, fused into one pass over the edges):
 * g_Z = env * D * g_out[idx_j], g_wigner and g_env channel reductions.  accumulate: bit 0
 * adds g_wigner to the array's contents, bit 1 adds g_env (as in fu_gather_bwd). */
int fu_scatter_bwd(const float* g_out, const int64_t* idx_j, const float* Z_m0, const float* Z_m1,
                   const float* Z_m2, const float* wigner, const float* env, float* g_Z_m0,
                   float* g_Z_m1, float* g_Z_m2, float* g_wigner, float* g_env, int64_t E,
                   int64_t N, int32_t C, int32_t accumulate, void* stream);

/* ops/scatter.py:360-423 (_init_scatter_fwd_kernel): edge-degree embedding,
 * x0[j] = [W_sphere[Z_j] + csd_emb[batch_j], 0...] + sum_e env/5 * (r0; r1 D1[1,:]; r2 D2[2,:]). */
int fu_init_scatter_fwd(const int32_t* row_ptr, const int32_t* col_idx, const float* rad,
                        const float* wigner, const float* env, const int64_t* Z,
                        const int64_t* batch, const float* W_sphere, const float* csd_emb,
                        float* x_out, int64_t N, int64_t E, int64_t num_z, int64_t S, int32_t C,
                        void* stream);

/* ops/scatter.py:426-481 (_init_scatter_bwd_kernel): g_rad (E, 3C), g_wigner (E, 34; the
 * 26 entries the forward does not read are written as 0, or left as they are when
 * accumulating) and g_env (E).  accumulate as in fu_scatter_bwd. */
int fu_init_scatter_bwd(const float* g_out, const int64_t* idx_j, const float* rad,
                        const float* wigner, const float* env, float* g_rad, float* g_wigner,
                        float* g_env, int64_t E, int64_t N, int32_t C, int32_t accumulate,
                        void* stream);

/* ------------------------------------------------------------------------------------
 * LayerNorm + SiLU (replaces _LayerNormSiLUFn, ops/ln_silu.py:126-185)
 * ------------------------------------------------------------------------------------ */

/* ops/ln_silu.py:29-72: out = silu(gamma * (x - mean) * rstd + beta) over rows of D. */
int fu_ln_silu_fwd(const float* x, const float* gamma, const float* beta, float* out, float* mean,
                   float* rstd, int64_t M, int32_t D, float eps, void* stream);

/* ops/ln_silu.py:77-123: g_x only (gamma/beta are frozen). */
int fu_ln_silu_bwd(const float* x, const float* gamma, const float* beta, const float* mean,
                   const float* rstd, const float* g_out, float* g_x, int64_t M, int32_t D,
                   void* stream);

/* The first LayerNorm+SiLU of every radial MLP at once (model.py:147, 203 with
 * ops/ln_silu.py:29-72 per block).  Row e of x (stride ldx) holds G groups of D values, the
 * Gaussian part W1[:, :B] g_e of each block's first linear.  Group g is normalised after
 * adding bias[g*D:], tab_src[z[isrc[e]]][g*D:] and tab_dst[z[idst[e]]][g*D:] (the
 * element-embedding part of the same linear, precomputed per element; tables optional,
 * stride ldt); gamma/beta are G*D long.  mean/rstd hold M*G entries, (row, group) order. */
int fu_ln_silu_grouped_fwd(const float* x, int64_t ldx, const float* tab_src, const float* tab_dst,
                           int64_t ldt, const int64_t* z, const int64_t* isrc, const int64_t* idst,
                           const float* bias, const float* gamma, const float* beta, float* out,
                           int64_t ldo, float* mean, float* rstd, int64_t M, int32_t G, int32_t D,
                           float eps, void* stream);

/* Input gradient of fu_ln_silu_grouped_fwd (ops/ln_silu.py:77-123 per group); the gradient
 * with respect to x equals the gradient with respect to the table rows and bias. */
int fu_ln_silu_grouped_bwd(const float* x, int64_t ldx, const float* tab_src, const float* tab_dst,
                           int64_t ldt, const int64_t* z, const int64_t* isrc, const int64_t* idst,
                           const float* bias, const float* gamma, const float* beta,
                           const float* mean, const float* rstd, const float* g_out, int64_t ldg,
                           float* g_x, int64_t ldgx, int64_t M, int32_t G, int32_t D, void* stream);

/* A radial-MLP linear followed by its LayerNorm + SiLU in one kernel (model.py:147-149 with
 * ops/ln_silu.py:29-76 per group): fu_linear / fu_linear_batched whose epilogue applies
 * fu_ln_silu_grouped_fwd to the GEMM output instead of storing it.  Row e holds G groups of
 * 128 columns, one per N-tile (batch = 1, N = 128 G) or one per batch (N = 128, batch = G,
 * strides as in fu_linear_batched).  The LayerNorm input is the GEMM output (+ bias) plus the
 * optional element-table rows and ln_bias, as in fu_ln_silu_grouped_fwd; Y receives the
 * SiLU output, mean / rstd (M x G) the statistics, and pre (optional, batch stride
 * stride_pre) the GEMM output before tables and ln_bias. */
int fu_linear_ln_silu(const float* A, int64_t lda, int64_t stride_a, const float* W, int64_t ldw,
                      int64_t stride_w, const float* bias, int64_t stride_bias, int32_t bias_batches,
                      float* Y, int64_t ldy, int64_t stride_y, float* pre, int64_t ldpre,
                      int64_t stride_pre, int64_t M, int32_t N, int32_t K, int32_t batch,
                      const float* tab_src, const float* tab_dst, int64_t ldt, const int64_t* z,
                      const int64_t* isrc, const int64_t* idst, const float* ln_bias,
                      const float* gamma, const float* beta, float* mean, float* rstd, int32_t G,
                      float eps, void* stream);

/* The LayerNorm-SiLU input gradient fused the same way (ops/ln_silu.py:77-123 per group):
 * the GEMM (batch 1, N = 128 G) recomputes the LayerNorm input's product part A W^T, and the
 * epilogue applies fu_ln_silu_grouped_bwd with the forward's mean / rstd and the output
 * gradient g_out (row stride ldgo), writing g_x. */
int fu_linear_ln_silu_bwd(const float* A, int64_t lda, const float* W, int64_t ldw, float* g_x,
                          int64_t ldgx, int64_t M, int32_t N, int32_t K, const float* g_out,
                          int64_t ldgo, const float* tab_src, const float* tab_dst, int64_t ldt,
                          const int64_t* z, const int64_t* isrc, const int64_t* idst,
                          const float* ln_bias, const float* gamma, const float* beta,
                          const float* mean, const float* rstd, int32_t G, void* stream);

/* The LayerNorm-SiLU input gradient of one group when its output gradient is a GEMM product
 * (the radial MLP's output layer backward followed by the second hidden layer's LayerNorm-SiLU
 * backward, model.py:147-149 and ops/ln_silu.py:77-123): g = A W^T (M x 128, W 128 x K) is
 * dL/dy for y = silu(LN(x_group) gamma + beta) on columns 128 group .. 128 group + 127 of x
 * (M x ldx, ldx >= 128 G; gamma, beta of length 128 G; mean / rstd (M x G) the forward's
 * statistics); the epilogue writes dL/dx_group to g_x (M x 128, row stride ldgx).  g is never
 * stored. */
int fu_linear_dgrad_ln_silu_bwd(const float* A, int64_t lda, const float* W, int64_t ldw,
                                float* g_x, int64_t ldgx, int64_t M, int32_t K, const float* x,
                                int64_t ldx, const float* gamma, const float* beta,
                                const float* mean, const float* rstd, int32_t G, int32_t group,
                                const void* W2, void* stream);

/* ------------------------------------------------------------------------------------
 * Dense contractions on fp32 MFMA (replaces torch F.linear at model.py:147-154,203-205)
 * ------------------------------------------------------------------------------------ */

/* Y[M, N] = A[M, K] @ W[N, K]^T (+ bias[N] when non-NULL), fp32 in and out, fp32 MFMA
 * accumulation.  lda/ldw/ldy are row strides in floats; K, N, lda, ldw and ldy must be
 * multiples of 4 and A, W, Y 16-byte aligned.
 * W2 (here and in fu_linear_gate, fu_linear_gate_bwd, fu_linear_dgrad_ln_silu_bwd): NULL, or
 * the same weight pre-split by fu_linear_weight_split (16-byte aligned).  In matrix-core mode 2
 * with tall tiles (M >= 65,536) and K % 16 == 0 the kernel then loads its weight fragments from
 * W2 straight into registers (exact column scales and window flags from W2) instead of staging
 * and splitting W; otherwise W2 is not read.  No reference counterpart (an argument of this
 * build's kernels). */
int fu_linear(const float* A, int64_t lda, const float* W, int64_t ldw, const float* bias,
              float* Y, int64_t ldy, int64_t M, int32_t N, int32_t K, const void* W2, void* stream);

/* Strided batch of fu_linear in one launch: for b < batch,
 * Y_b = A_b @ W_b^T (+ bias_b for b < bias_batches) (+ R_b), X_b = X + b * stride_x (floats).
 * Used for the per-degree SO(3) linears of the atom-wise FFN (W_b = the weight of the
 * degree of coefficient b, bias on l = 0 only) and the radial bank's second layers.  R
 * (NULL, or row stride ldr >= N, batch stride stride_r, 16-byte aligned) is a residual added
 * in the epilogue: the skip x_mid + atom_wise(...) of model.py:157 without a separate add. */
int fu_linear_batched(const float* A, int64_t lda, int64_t stride_a, const float* W, int64_t ldw,
                      int64_t stride_w, const float* bias, int64_t stride_bias, int32_t bias_batches,
                      const float* R, int64_t ldr, int64_t stride_r, float* Y, int64_t ldy,
                      int64_t stride_y, int64_t M, int32_t N, int32_t K, int32_t batch, void* stream);

/* Complex dense layer, the SO(2) m = 1, 2 convolutions (model.py:152,154 with the packed
 * weights of model.py:108-138): for features a_r + i a_i (two (M, Kc) arrays, row stride lda)
 * and weight P + iQ ((Nc, Kc) each, row stride ldw),
 *   Y_r = A_r P^T - A_i Q^T,   Y_i = A_r Q^T + A_i P^T      ((M, Nc), row stride ldy),
 * i.e. X [[P, -Q], [Q, P]]^T with X = [A_r | A_i] -- the reference's packed product -- computed
 * with three real products (Gauss) instead of four.  The input gradient of the layer is
 * the same operation with (P^T, -Q^T).  Kc, lda, ldw multiples of 4; A_r, A_i, P, Q 16-byte
 * aligned.  W3: NULL, or the same weight pre-split by fu_complex_weight_split (16-byte
 * aligned); in the split matrix-core modes (fu_set_matmul_mode) it is read instead of P and Q
 * (three split products, B fragments loaded straight into registers: its bf16 planes in mode 0,
 * its fp16 planes and column scales in mode 2); without it the operands are split in the kernel
 * (four bf16 split products).  The fp32 mode ignores W3. */
int fu_complex_linear(const float* A_r, const float* A_i, int64_t lda, const float* P, const float* Q,
                      int64_t ldw, const void* W3, float* Y_r, float* Y_i, int64_t ldy, int64_t M,
                      int32_t Nc, int32_t Kc, void* stream);

/* Pre-split complex weight for the W3 argument of fu_complex_linear*; no reference counterpart
 * (a frozen weight of model.py:108-138, prepared once at freeze time).  P, Q (Nc, Kc) with row
 * stride ldw; W3 receives the exact three-way bf16 splits of P, Q and P + Q in MFMA-fragment
 * order ([32-column block][16-k chunk][P, Q, P + Q][hi, mid, lo][64 lanes] x 16 bytes, zero
 * padded to Nc = 32 n, Kc = 16 k), then the two-way fp16 splits of the same three operands with
 * each column n scaled by a power of two 2^e(n) ([block][chunk][P hi, P lo, Q hi, Q lo, S hi,
 * S lo, P lo', Q lo', S lo'][64 lanes], lo' = 2^11 lo for the two-loop pass of the fp16 mode),
 * then the factors 2^-e(n) (one float per padded column), then one int32 per padded column:
 * bit 0 when 8 consecutive k of P or Q in that column are below the fp16 window at its scale,
 * bit 1 when the column is not flat (a piece of 8 k more than 2^6 below its largest; the fp16
 * mode's pass rules read both): fu_complex_weight_split_bytes(Nc, Kc) bytes, 16-byte
 * aligned, valid in every matrix-core mode.  The bytes query returns a negative FU_ERR_* for Nc
 * or Kc <= 0. */
int64_t fu_complex_weight_split_bytes(int32_t Nc, int32_t Kc);
int fu_complex_weight_split(const float* P, const float* Q, int64_t ldw, int32_t Nc, int32_t Kc, void* W3,
                            void* stream);

/* Pre-split real weight for fu_linear_resident and the W2 argument of fu_linear and its
 * relatives; no reference counterpart (a frozen weight of model.py:147-154, 203-205, prepared
 * once at freeze time).  W (N, K) with row stride ldw, K a positive multiple of 16
 * (fu_linear_resident: K <= 128).  W2 receives the fp16 splits of every column n scaled by its
 * exact power of two 2^e(n) in MFMA-fragment order ([32-column block][16-k chunk][hi, lo, lo'
 * = 2^11 lo][64 lanes] x 16 bytes, zero padded to N = 32 n), then the factors 2^-e(n) (one float
 * per padded column), then one int32 per padded column (bit 0: 8 consecutive k below the fp16
 * window at the column's scale; bit 1: the column is not flat), then their OR (one int32,
 * padded to 16 bytes): fu_linear_weight_split_bytes(N, K) bytes, 16-byte aligned.  The bytes
 * query returns a negative FU_ERR_* for a shape outside those bounds. */
int64_t fu_linear_weight_split_bytes(int32_t N, int32_t K);
int fu_linear_weight_split(const float* W, int64_t ldw, int32_t N, int32_t K, void* W2, void* stream);

/* Y[M, N] = A[M, K] W^T (+ bias[N]) for short K, replacing F.linear of the radial output layers
 * (model.py:149, 205: rad_out = h2 W_rad1_3^T + b_rad1_3, K = C, N = 6 lmax C).  W is given
 * pre-split by fu_linear_weight_split.  Always computed in the split-fp16 form of matrix-core
 * mode 2, whatever fu_set_matmul_mode selects, with each row of A at its exact scale (taken from
 * the whole row) and the two-loop pass of split_f16.h for a 128-row panel whose pieces leave the
 * window against a rough weight column (or the reverse): a workgroup keeps its 128-row panel of
 * A, split, in LDS and walks all N, so A is read and split once instead of once per 128-column
 * tile.  16 <= K <= 128, K % 16 == 0; A 16-byte aligned, lda a multiple of 4; ldy >= N; bias
 * may be NULL.  M = 0 is a no-op. */
int fu_linear_resident(const float* A, int64_t lda, const void* W2, const float* bias, float* Y, int64_t ldy,
                       int64_t M, int32_t N, int32_t K, void* stream);

/* The radial output layer fused with the gather-rotate forward (lmax 2, C = 128; replaces
 * model.py:149 rad_out = h2 W_rad1_3^T + b_rad1_3 followed by ops/gather.py:34-154
 * gather_wigner_split, whose only reader of rad_out in the forward is the gather): writes rad
 * (E, 12C) in the natural order (as fu_linear_resident with the unpermuted weight would, for the
 * gather backward) and X_m0 (E, 6C), X_m1 (E, 8C), X_m2 (E, 4C) exactly as fu_gather_fwd with
 * that rad (bitwise).  W2 is the radial weight (12C x K) with its rows permuted by
 * fu_radial_gather_perm, pre-split by fu_linear_weight_split; bias is the bias permuted the same
 * way (may be NULL).  h2: (E, K) rows with stride ldh.  C = K = 128, layout 0 or 1 (as
 * fu_gather_fwd); every array 16-byte aligned, ldh a multiple of 4.  Split-fp16 products as
 * fu_linear_resident, whatever fu_set_matmul_mode selects.  E = 0 is a no-op. */
int fu_radial_gather_fwd(const float* h2, int64_t ldh, const void* W2, const float* bias, const float* x,
                         const int64_t* idx_i, const int64_t* idx_j, const float* wigner, const float* csd_emb,
                         const int64_t* batch, float* rad, float* X_m0, float* X_m1, float* X_m2, int64_t E,
                         int64_t N, int64_t S, int32_t C, int32_t K, int32_t layout, void* stream);

/* Host-only: perm[p] (12C entries) = the radial column that fu_radial_gather_fwd computes as its
 * weight's row p.  Output tile t (96 columns) holds the three radial blocks of degrees 0 and 1
 * (even t) or of degree 2 (odd t) of side t / 8 for channels 32 ((t / 2) % 4) .. + 31
 * (radial_gather.hip).  C = 128, layout 0 or 1. */
int fu_radial_gather_perm(int32_t C, int32_t layout, int32_t* perm);

/* The radial output layer fused with the lmax 3 / 4 gather forward (replaces model.py:149 and
 * the lmax form of the gather, fu_gather_fwd_lmax): rad (E, 6 lmax C) and X_m0 (E, 2(lmax+1)C),
 * X_m1 (E, 4 lmax C), X_m2 (E, 4(lmax-1)C) in the lmax kernels' block order, bitwise as
 * fu_linear_resident with the unpermuted weight followed by fu_gather_fwd_lmax.  W2: the
 * weight (6 lmax C x K) with its rows permuted by fu_radial_gather_perm_lmax, pre-split by
 * fu_linear_weight_split; bias permuted the same way (may be NULL).  wig_ext: the degree-3/4
 * Wigner rows (fu_wigner_ext_fwd).  C = K = 128; 16-byte alignment as fu_radial_gather_fwd. */
int fu_radial_gather_fwd_lmax(const float* h2, int64_t ldh, const void* W2, const float* bias, const float* x,
                              const int64_t* idx_i, const int64_t* idx_j, const float* wigner, const float* wig_ext,
                              const float* csd_emb, const int64_t* batch, float* rad, float* X_m0, float* X_m1,
                              float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C, int32_t K, int32_t lmax,
                              void* stream);

/* Host-only: perm[p] (6 lmax C entries) = the radial column that fu_radial_gather_fwd_lmax
 * computes as its weight's row p: tile t (96 columns) holds, for side t / (4 lmax) and
 * channels 32 ((t / lmax) % 4) .. + 31, the radial blocks of degrees 0 and 1 (t % lmax = 0)
 * or of degree t % lmax + 1.  C = 128, lmax 3 or 4. */
int fu_radial_gather_perm_lmax(int32_t C, int32_t lmax, int32_t* perm);

/* conv1 m = 0 fused with the gate activation (model.py:152-153 with ops/gating.py:32-103):
 * Y = A W^T + bias with N = (2L+1)C columns (L = lmax) in the gate-paired order: 64-column
 * pairs [gate_l | y_lm0] x C/32 for l = 1..L, then y_l0 (W and bias rows permuted to it; at
 * lmax 2 this is fu_gating_fwd layout 1), written for the backward, plus Z (M, (L+1)C) =
 * [silu(y_l0), y_l1m0 s1, ..., y_lLm0 sL], and, if S is not NULL, S (M, LC) = [s1 .. sL],
 * s = sigmoid(gate) (the model passes NULL: the gate epilogues below recompute s from Y).
 * lmax 2..4; C a multiple of 64; other constraints as fu_linear. */
int fu_linear_gate(const float* A, int64_t lda, const float* W, int64_t ldw, const float* bias,
                   float* Y, int64_t ldy, float* Z, int64_t ldz, float* S, int64_t lds, int64_t M,
                   int32_t C, int32_t K, int32_t lmax, const void* W2, void* stream);

/* conv1 m = 0 with its A operand gathered in the GEMM loader (the gather-rotate fused with the
 * m = 0 SO(2) linear, ops/gather.py:128-154 -> model.py:152, lmax 2): the result of
 * fu_gather_fwd (layout 1) followed by fu_linear_gate on X_m0 (W: 5C x 6C gate-paired, ldw),
 * without X_m0 ever being stored: each loader chunk rotates the two node rows of its edges by
 * the m = 0 Wigner rows (csd_emb[batch] added on l = 0) and scales them by the radial row.
 * Y (E x 5C) and Z (E x 3C) as fu_linear_gate.  Split-bf16 matrix-core mode only
 * (FU_ERR_UNSUPPORTED in the fp32 mode); C a multiple of 64. */
int fu_gather_linear_gate(const float* x, const int64_t* idx_i, const int64_t* idx_j,
                          const float* wigner, const float* rad, const float* csd_emb,
                          const int64_t* batch, const float* W, int64_t ldw, const float* bias,
                          float* Y, int64_t ldy, float* Z, int64_t ldz, int64_t E, int32_t C,
                          void* stream);

/* conv1 m = 1, 2 fused with the gate activation: fu_complex_linear, then
 * Z_r = Y_r s, Z_i = Y_i s with s = sigmoid(gate) of gate column t = s_off + column (degree
 * 1 + t / C, channel t % C), read from Y0, the gate-paired output of fu_linear_gate (row
 * stride ldy0): s_off = 0 for m = 1, whose columns are [l1 | .. | lL]; s_off = C for m = 2,
 * columns [l2 | .. | lL].  C a multiple of 32, s_off and ldy0 multiples of 4. */
int fu_complex_linear_gate(const float* A_r, const float* A_i, int64_t lda, const float* P,
                           const float* Q, int64_t ldw, const void* W3, float* Y_r, float* Y_i,
                           int64_t ldy, float* Z_r, float* Z_i, int64_t ldz, const float* Y0,
                           int64_t ldy0, int32_t s_off, int32_t C, int64_t M, int32_t Nc, int32_t Kc,
                           void* stream);

/* conv2 m = 0 input gradient (model.py:154) fused with the gate backward (ops/gating.py:
 * 109-185): the GEMM g_Z_m0 = gZo (M, (L+1)C) @ Wt^T is not stored; gY0 (M, (2L+1)C,
 * gate-paired as Y0) receives g_y_l0 = g silu'(y_l0), g_y_lm0 = g s_l and
 * g_gate_l = s_l (1 - s_l) (g y_lm0 + P1[:, (l-1)C:] + (l >= 2: P2[:, (l-2)C:])).  Y0: the
 * forward output of fu_linear_gate (s_l = sigmoid of its gate columns); P1 (M, LC),
 * P2 (M, (L-1)C): the m = 1, 2 gate sums from fu_complex_linear_gate_bwd.  K = (L+1)C (the
 * conv2 m = 0 width), Wt = W2_m0^T (no bias).  lmax 2..4; C a multiple of 64. */
int fu_linear_gate_bwd(const float* gZo, int64_t ldgz, const float* Wt, int64_t ldw, const float* Y0,
                       int64_t ldy0, const float* P1, int64_t ldp1, const float* P2, int64_t ldp2,
                       float* gY0, int64_t ldg, int64_t M, int32_t C, int32_t K, int32_t lmax,
                       const void* W2, void* stream);

/* conv2 m = 1 or 2 input gradient fused with the gate backward: the complex product
 * g_Z = (A_r + i A_i)(P + iQ)^T (P = R^T, Q = -I^T of the conv2 weight) is not stored;
 * gY_r/gY_i = g_Z s with s recomputed from Y0 as in fu_complex_linear_gate (same s_off, C),
 * and Pout = g_Zr F_r + g_Zi F_i (the gate sum of this block; F = the forward pre-activation
 * Y from fu_complex_linear_gate). */
int fu_complex_linear_gate_bwd(const float* A_r, const float* A_i, int64_t lda, const float* P,
                               const float* Q, int64_t ldw, const void* W3, float* gY_r, float* gY_i,
                               int64_t ldg, const float* F_r, const float* F_i, int64_t ldf,
                               const float* Y0, int64_t ldy0, int32_t s_off, int32_t C, float* Pout,
                               int64_t ldp, int64_t M, int32_t Nc, int32_t Kc, void* stream);

/* ------------------------------------------------------------------------------------
 * Node-level modules attached to the backbone (model.py:145,157,218) and input plumbing
 * ------------------------------------------------------------------------------------ */

/* Equivariant RMS norm over SH coefficients (FAIRChem rms_norm_sh, the norm_1 / norm_2 /
 * final norm of model.py:145,157,218): l=0 centred over channels, scaled by
 * (mean_c sum_k x_kc^2 / ((2 l_k + 1)(lmax + 1)) + eps)^-1/2, per-(l, c) weight, l=0 bias.
 * x, out (N, (lmax + 1)^2, C), lmax 2..4; weight (lmax + 1, C); bias (C); inv_rms (N) is
 * saved for the backward.  The backward adds g_res (NULL or the shape of x) to g_x: the
 * gradient of a residual branch that read the same x (the x_in + ... and x_mid + ... skips of
 * model.py:143-157), which then needs no separate accumulation. */
int fu_rms_norm_sh_fwd(const float* x, const float* weight, const float* bias, float* out,
                       float* inv_rms, int64_t N, int32_t C, int32_t lmax, float eps, void* stream);
int fu_rms_norm_sh_bwd(const float* x, const float* weight, const float* inv_rms,
                       const float* g_out, const float* g_res, float* g_x, int64_t N, int32_t C,
                       int32_t lmax, void* stream);

/* Gate activation of the atom-wise FFN: gate_l = sigmoid(silu(pre[:, l-1])) for l >= 1,
 * out_0 = silu(h_0), out_k = h_k * gate_{l_k}.  pre (N, lmax * H), h and out
 * (N, (lmax + 1)^2, H), lmax 2..4. */
int fu_gate_act_fwd(const float* pre, const float* h, float* out, int64_t N, int32_t H,
                    int32_t lmax, void* stream);
int fu_gate_act_bwd(const float* pre, const float* h, const float* g_out, float* g_pre,
                    float* g_h, int64_t N, int32_t H, int32_t lmax, void* stream);

/* Charge / spin channel balancing (FAIRChem balance_channels_batched, called per block at
 * model.py:213-216).  x, out (N, K, C) fp32; batch (N) sorted ascending with ids in [0, S);
 * sys_ptr (S + 1, int32) the system segments of batch (fu_csr_row_ptr over batch).  For
 * each system s and channel c in [c0, c1):
 *   out[a][0][c] = x[a][0][c] + (target[s] - target_offset - sum_{a in s} x[a][0][c]) / n_s,
 * everything else copied.  target NULL means 0 (the input gradient: pass the output
 * gradient as x and target_offset 0).  corr is a workspace of S * (c1 - c0) floats.  Sums
 * in fp64 in a fixed order (deterministic). */
int fu_balance_channels(const float* x, float* out, const int64_t* batch, const int32_t* sys_ptr,
                        const float* target, float target_offset, float* corr, int64_t corr_len,
                        int64_t N, int32_t K, int32_t C, int32_t S, int32_t c0, int32_t c1,
                        void* stream);

/* Allocation-free variant of fu_balance_channels: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The corr workspace is a library-owned device
 * array of FU_BALANCE_NOALLOC_MAX_CORR floats per GPU (256 KiB, held until the process ends;
 * its address is looked up on the first call on each device, which must be the current
 * device); S * (c1 - c0) above that returns FU_ERR_WORKSPACE.  Results equal
 * fu_balance_channels bit for bit.  Calls that overlap on one GPU (several streams or host
 * threads at once) share that array and race. */
#define FU_BALANCE_NOALLOC_MAX_CORR 65536
int fu_balance_channels_noalloc(const float* x, float* out, const int64_t* batch,
                                const int32_t* sys_ptr, const float* target, float target_offset,
                                int64_t N, int32_t K, int32_t C, int32_t S, int32_t c0, int32_t c1,
                                void* stream);

/* Row permutations (model.py:72-74,221): gather dst[r] = src[idx[r]]; scatter
 * dst[idx[r]] = src[r] (idx a permutation, each destination row written once). */
int fu_gather_rows(const float* src, const int64_t* idx, float* dst, int64_t rows, int32_t width,
                   void* stream);
int fu_scatter_rows(const float* src, const int64_t* idx, float* dst, int64_t rows,
                    int32_t width, void* stream);

/* PBC shifts (wrapper.py:193-194): shifts[e] = cell_offsets[perm[e]] @ cell for a single
 * system (perm NULL = identity). */
int fu_edge_shifts(const float* cell_offsets, const float* cell, const int64_t* perm,
                   float* shifts, int64_t E, void* stream);

/* out (3x3) = sum_e A[perm_a[e]]^T B[e] over E rows of 3 (perm_a NULL = identity), in fp64
 * with a fixed two-stage order (deterministic); the cell gradient of the shifts product.
 * partial is a workspace of at least 256 * 9 doubles. */
int fu_outer_sum3(const float* A, const int64_t* perm_a, const float* B, float* out,
                  double* partial, int64_t partial_len, int64_t E, void* stream);

/* ------------------------------------------------------------------------------------
 * Graph preprocessing (replaces reorder_graph_morton / _build_csr_uncached, model.py:20-74)
 * ------------------------------------------------------------------------------------ */

/* model.py:60-68: sort keys morton3d(quantised pos) | batch << 32 for N atoms. */
int fu_morton_keys(const float* pos, const int64_t* batch, int64_t* keys, int64_t N,
                   void* stream);

/* Stable LSD radix sort of (key, value) int64 pairs on bits [begin_bit, end_bit).
 * With workspace == NULL, stores the needed workspace size in *ws_bytes and returns. */
int fu_sort_pairs_i64(const int64_t* keys_in, int64_t* keys_out, const int64_t* vals_in,
                      int64_t* vals_out, int64_t n, int32_t begin_bit, int32_t end_bit,
                      void* workspace, size_t* ws_bytes, void* stream);

/* inv[perm[k]] = k for k < n (model.py:71-72). */
int fu_invert_perm(const int64_t* perm, int64_t* inv, int64_t n, void* stream);

/* out[e] = table[idx[e]] for int64 arrays; every idx must lie in [0, table_len). */
int fu_take_i64(const int64_t* table, int64_t table_len, const int64_t* idx, int64_t* out,
                int64_t n, void* stream);

/* row_ptr (N+1, int32) of a CSR whose edge keys are sorted ascending, model.py:22-24:
 * row_ptr[v] = #{e : sorted_keys[e] < v} for v = 0..N.  The caller guarantees keys in
 * [0, N) (the op layer checks index ranges before building a topology). */
int fu_csr_row_ptr(const int64_t* sorted_keys, int64_t E, int32_t* row_ptr, int64_t N,
                   void* stream);

/* int64 -> int32 narrowing copy (col_idx = sort_order.to(int32), model.py:25). */
int fu_narrow_i64_i32(const int64_t* in, int32_t* out, int64_t n, void* stream);

/* ------------------------------------------------------------------------------------
 * Radius graph (the input graph of the reference: FAIRChem a2g, readme.md:34; definition of
 * the host builder systems.neighbor_list).  For receiver j: all (i, o), o an integer cell
 * offset (0 on non-periodic axes), (i, o) != (j, 0), with d = (pos_i - pos_j) +
 * ((o0 c0 + o1 c1) + o2 c2) evaluated in float64 from the float32 inputs in that order and
 * |d|^2 = (dx dx + dy dy) + dz dz < cutoff^2; ordered by (|d|^2, i, o0, o1, o2); the first
 * max_neighbors kept; receivers ascending.  Geometry arguments are HOST arrays: cell (9
 * doubles, lattice vectors as rows), inv_cell (its inverse), nbins / reach / pbc (3 int32
 * each: cell-list bins per axis, at least cutoff + 1e-3 wide; bins searched per side; axis
 * periodicity).  Non-periodic axes use nbins = 1, reach = 0.
 * ------------------------------------------------------------------------------------ */

/* Cell-list bin key (N int64) and wrap count floor(s) per axis (N x 3 int32) of each atom. */
int fu_nlist_bin(const float* pos, int64_t N, const double* cell, const double* inv_cell,
                 const int32_t* nbins, const int32_t* reach, const int32_t* pbc, int64_t* bin_key,
                 int32_t* wrap, void* stream);

/* Per receiver: the max_neighbors first candidates (out_sender N x K int32, out_off N x K x 3
 * int32), the number kept (nout) and the number within the cutoff (count; results are only
 * complete when every count <= 512).  sorted_atoms: atoms stably sorted by bin_key; bin_ptr:
 * nbins_total + 1 bin starts into sorted_atoms. */
int fu_nlist_search(const float* pos, const int64_t* sorted_atoms, const int32_t* bin_ptr,
                    const int32_t* wrap, const int64_t* bin_key, int64_t N, const double* cell,
                    const double* inv_cell, const int32_t* nbins, const int32_t* reach,
                    const int32_t* pbc, double cutoff, int32_t max_neighbors, int32_t* out_sender,
                    int32_t* out_off, int32_t* count, int32_t* nout, void* stream);

/* row_ptr (N + 1 int64) = exclusive scan of nout; row_ptr[N] = E. */
int fu_nlist_scan(const int32_t* nout, int64_t* row_ptr, int64_t N, void* stream);

/* edge_index (2 x E int64: senders, then receivers) and cell_offsets (E x 3 float32). */
int fu_nlist_emit(const int32_t* sender, const int32_t* off, const int32_t* nout, const int64_t* row_ptr,
                  int64_t N, int32_t max_neighbors, int64_t* edge_index, float* cell_offsets, int64_t E,
                  void* stream);

/* ------------------------------------------------------------------------------------
 * Degrees above 2 (lmax = 3 or 4, mmax = 2).  The reference rejects lmax != 2
 * (wrapper.py:105-118); these entry points generalise its lmax = 2 kernels degree by degree.
 * They also accept lmax = 2, where every array has the reference's shape and order.
 *
 * Shapes (C channels, L = lmax): node rows x (N, (L+1)^2, C); rad (E, 6L C); X_m0 (E, 2(L+1) C),
 * X_m1 (E, 4L C), X_m2 (E, 4(L-1) C); Y_m0 (E, (2L+1) C), Y_m1 (E, 2L C), Y_m2 (E, 2(L-1) C);
 * Z_m0 (E, (L+1) C), Z_m1 (E, 2L C), Z_m2 (E, 2(L-1) C); init rad (E, (L+1) C).  Column blocks
 * follow the reference order extended by degree (csrc/edge_lmax.hip states the map).
 * wigner is the reference's (E, 34) array; wig_ext (E, fu_wigner_ext_width(L)) holds rows
 * m = -2..2 of D^3 (5 x 7) and D^4 (5 x 9), row-major; it may be NULL for L = 2.
 * ------------------------------------------------------------------------------------ */

/* Scalars per edge of wig_ext: 0 (lmax 2), 35 (lmax 3), 80 (lmax 4); -1 otherwise. */
int fu_wigner_ext_width(int32_t lmax);

/* wig_ext from the reference's L=1 and L=2 blocks, by the recursion
 * D^l = U_l^T (D^(l-1) (x) D^1) U_l (no reference counterpart: ops/geom.py:137-178 stops at
 * L=2).  lmax 3 or 4. */
int fu_wigner_ext_fwd(const float* wigner, float* wig_ext, int64_t E, int32_t lmax, void* stream);

/* Vector-Jacobian product of fu_wigner_ext_fwd: g_wigner (E, 34) = dL/dwigner through wig_ext
 * (overwritten, not accumulated). */
int fu_wigner_ext_bwd(const float* wigner, const float* g_wig_ext, float* g_wigner, int64_t E,
                      int32_t lmax, void* stream);

/* fu_gather_fwd for lmax 2..4 in the extended reference order (ops/gather.py:34-154).  With the
 * receiver and sender CSRs of the graph (all four non-NULL, as fu_gather_bwd_lmax takes them)
 * the kernel walks each node's two segments and reads every node row once per side; with all
 * four NULL it runs edge-parallel from idx_i / idx_j.  The outputs are the same either way. */
int fu_gather_fwd_lmax(const float* x, const int64_t* idx_i, const int64_t* idx_j,
                       const float* wigner, const float* wig_ext, const float* rad,
                       const float* csd_emb, const int64_t* batch, const int32_t* recv_ptr,
                       const int32_t* recv_idx, const int32_t* send_ptr, const int32_t* send_idx,
                       float* X_m0, float* X_m1, float* X_m2, int64_t E, int64_t N, int64_t S, int32_t C,
                       int32_t lmax, void* stream);

/* fu_gather_bwd for lmax 2..4 (ops/gather.py:160-405, node-centric, no atomics).  ws is a
 * scratch array of E * (34 + fu_wigner_ext_width(lmax)) floats.  accumulate: bit 0 adds
 * g_wigner and g_wig_ext to the arrays' contents. */
int fu_gather_bwd_lmax(const float* g_X_m0, const float* g_X_m1, const float* g_X_m2,
                       const float* x, const float* wigner, const float* wig_ext, const float* rad,
                       const float* csd_emb, const int64_t* batch, const int32_t* recv_ptr,
                       const int32_t* recv_idx, const int32_t* send_ptr, const int32_t* send_idx,
                       float* g_x, float* g_wigner, float* g_wig_ext, float* g_rad, float* ws,
                       int64_t E, int64_t N, int64_t S, int32_t C, int32_t lmax, int32_t accumulate,
                       void* stream);

/* fu_scatter_fwd for lmax 2..4 (ops/scatter.py:45-140, fp64 CSR accumulation). */
int fu_scatter_fwd_lmax(const int32_t* row_ptr, const int32_t* col_idx, const float* Z_m0,
                        const float* Z_m1, const float* Z_m2, const float* wigner,
                        const float* wig_ext, const float* env, const float* x_res, float* x_out,
                        int64_t N, int64_t E, int32_t C, int32_t lmax, void* stream);

/* fu_scatter_bwd for lmax 2..4 (ops/scatter.py:146-292).  accumulate: bit 0 adds g_wigner
 * and g_wig_ext, bit 1 adds g_env to the arrays' contents. */
int fu_scatter_bwd_lmax(const float* g_out, const int64_t* idx_j, const float* Z_m0,
                        const float* Z_m1, const float* Z_m2, const float* wigner,
                        const float* wig_ext, const float* env, float* g_Z_m0, float* g_Z_m1,
                        float* g_Z_m2, float* g_wigner, float* g_wig_ext, float* g_env, int64_t E,
                        int64_t N, int32_t C, int32_t lmax, int32_t accumulate, void* stream);

/* fu_init_scatter_fwd for lmax 2..4 (ops/scatter.py:360-423): rad (E, (L+1) C). */
int fu_init_scatter_fwd_lmax(const int32_t* row_ptr, const int32_t* col_idx, const float* rad,
                             const float* wigner, const float* wig_ext, const float* env,
                             const int64_t* Z, const int64_t* batch, const float* W_sphere,
                             const float* csd_emb, float* x_out, int64_t N, int64_t E,
                             int64_t num_z, int64_t S, int32_t C, int32_t lmax, void* stream);

/* fu_init_scatter_bwd for lmax 2..4 (ops/scatter.py:426-481); g_wigner / g_wig_ext entries the
 * forward does not read are written as 0 (left as they are when accumulating).  accumulate as
 * in fu_scatter_bwd_lmax. */
int fu_init_scatter_bwd_lmax(const float* g_out, const int64_t* idx_j, const float* rad,
                             const float* wigner, const float* wig_ext, const float* env,
                             float* g_rad, float* g_wigner, float* g_wig_ext, float* g_env,
                             int64_t E, int64_t N, int32_t C, int32_t lmax, int32_t accumulate,
                             void* stream);

/* fu_gating_fwd / fu_gating_bwd (layout 0) for lmax 2..4 (ops/gating.py:32-185). */
int fu_gating_fwd_lmax(const float* Y_m0, const float* Y_m1, const float* Y_m2, float* Z_m0,
                       float* Z_m1, float* Z_m2, int64_t E, int32_t C, int32_t lmax, void* stream);
int fu_gating_bwd_lmax(const float* g_Z_m0, const float* g_Z_m1, const float* g_Z_m2,
                       const float* Y_m0, const float* Y_m1, const float* Y_m2, float* g_Y_m0,
                       float* g_Y_m1, float* g_Y_m2, int64_t E, int32_t C, int32_t lmax,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHUMA_H_ */
