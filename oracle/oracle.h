/*
 * CPU oracle for the MI355X matmul / attention dispatch path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline), never as the thing measured or shipped.
 *
 * Every routine restates the semantics of the reference's CPU path for the
 * dispatch it mirrors; each function cites the reference file:line it follows.
 * Half-precision values are passed as raw IEEE binary16 bit patterns
 * (uint16_t) because gcc 11 has no _Float16 on x86-64.
 *
 * Parity pins (checked in tests/test_oracle.py):
 *   half conversions      exhaustive vs numpy float16
 *   matmul_i8             brute force int64 numpy, closed-form overflow bound
 *   matmul_f16            torch.matmul(a.float(), b.float()) (the reference
 *                         micro model), exact small-integer cases, identity;
 *                         A / B transposed = the plain form of the
 *                         transposed copies, bit for bit
 *   w8a16                 per-element-dequant form, exact power-of-two cases
 *   attention             torch F.scaled_dot_product_attention (the reference
 *                         micro attention model) in f32, causal invariants
 *   attention (general)   SDPA with attn_mask and unequal head dims, a
 *                         float64 closed form with causal + mask + grouped
 *                         heads, brute force at the pipeline test's shapes,
 *                         masked keys = dropped keys (bits), f16 out = f32
 *                         out rounded (bits), fully masked rows = 0
 *   select_hmx_tile_sizes reference lit goldens
 *   choose_static_tiling  brute-force divisor search
 *   batch_matmul_f16      per-batch equality with matmul_f16; bias / ReLU /
 *                         GELU / SiLU against numpy closed forms; epilogue
 *                         order (bias before act, multiplier after)
 *   activation            ReLU / SiLU exact points, GELU-tanh identities
 *                         (odd part, limits, the value at 1)
 *   geglu_f16_ops         hand-computed values at h = 1, -2, 0 and large |h|,
 *                         and within 2e-3 of the f32 epilogue
 *
 * Parity unpinned (no check in this container can fix it):
 *   matmul_f16 / w8a16 / attention summation order: IREE llvm-cpu
 *     (iree-base-compiler 3.11.0) reassociates f32 sums and is not installed,
 *     so its exact order is not known; these routines sum in k order and the
 *     product is held to the 2e-3 relative tolerance, not to bits.
 *   select_hmx_tile_sizes when no candidate fits twice the budget: the
 *     reference then calls hexagon-mlir's determineTileSizes (un-vendored
 *     submodule); this routine returns 0 for that case and does not restate it.
 */
#ifndef IHP_ORACLE_H_
#define IHP_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round-to-nearest-even. */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void oracle_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n);
void oracle_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n);

/* Bits of the `flags` argument, same values as the product ABI. */
#define ORACLE_B_TRANSPOSED 1u /* B stored [N,K] (indexing map (d1,d2)) */
#define ORACLE_ACCUMULATE 2u   /* C_out = C_init + A.B (DPS init is read) */
#define ORACLE_OUT_F32 4u      /* f32 output, else f16 */
#define ORACLE_A_TRANSPOSED 8u /* A stored [K,M] (indexing map (d2,d0)) */

/* linalg.matmul f16 x f16 with f32 accumulation (arith.extf on the inputs),
 * C_out = C_init + sum_k A[m,k]*B[k,n], summed in k order in f32.
 * examples/matmul/matmul.mlir:1-14, UK/hmx.c:328-357 (add into init); the
 * transposed-operand maps of LIT/codegen/transforms/
 * convert_matmul_to_hmx.mlir:60-115 via ORACLE_A/B_TRANSPOSED. */
int oracle_matmul_f16(const uint16_t *a, const uint16_t *b, void *c,
                      int64_t m, int64_t n, int64_t k, int64_t lda,
                      int64_t ldb, int64_t ldc, uint32_t flags, int threads);

/* Activations of the fused epilogue (same values as the product ABI). */
#define ORACLE_ACT_NONE 0u
#define ORACLE_ACT_RELU 1u
#define ORACLE_ACT_GELU_TANH 2u
#define ORACLE_ACT_SILU 3u
float oracle_activation(float v, uint32_t act);

/* linalg.batch_matmul f16 with f32 accumulation and the fused elementwise
 * epilogue the reference fuses after a matmul (bias add, activation, gating
 * multiply; LIT/codegen/pipelines/hexagon_hmx_epilogue_keeps_config.mlir):
 * for each batch z, out = [C_init +] mul * act(A_z.B_z + bias), computed in
 * f32 from the f32 sum and rounded once. bias [N] and mul [M,N] (pitch
 * ld_mul, batch stride s_mul) may be NULL. Strides are in elements. */
int oracle_batch_matmul_f16(const uint16_t *a, const uint16_t *b, void *c,
                            int64_t batch, int64_t m, int64_t n, int64_t k,
                            int64_t lda, int64_t ldb, int64_t ldc, int64_t sa,
                            int64_t sb, int64_t sc, uint32_t flags,
                            const uint16_t *bias, const uint16_t *mul,
                            int64_t ld_mul, int64_t s_mul, uint32_t act,
                            int threads);

/* One element of the reference's GeGLU epilogue with every op rounded to f16,
 * as its IR computes it (LIT/codegen/pipelines/
 * hexagon_hmx_epilogue_keeps_config.mlir:82-101); math.fpowi h^3 is taken as
 * two f16 multiplies. */
uint16_t oracle_geglu_f16_ops(float acc, uint16_t up);

/* i8 x i8 -> i32 exact integer matmul (linalg.matmul / quantized_matmul with
 * zero points 0). */
int oracle_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m,
                     int64_t n, int64_t k, int64_t lda, int64_t ldb,
                     int64_t ldc, uint32_t flags, int threads);

/* W8A16 linear: y[m,n] = f16( (sum_k f32(x[m,k]) * f32(w[k,n])) * f32(s[n]) ),
 * zero point 0, w stored [K,N] (or [N,K] with ORACLE_B_TRANSPOSED). */
int oracle_w8a16(const uint16_t *x, const int8_t *w, const uint16_t *scale,
                 uint16_t *y, int64_t m, int64_t n, int64_t k, int64_t ldx,
                 int64_t ldw, int64_t ldy, uint32_t flags, int threads);

/* softmax(Q K^T * scale + mask) V with f32 scores/softmax, f16 in/out.
 * Layout [B,H,S,D] contiguous. Causal mask is top-left aligned (key j is
 * masked for query i when j > i), as torch's is_causal.
 * IT/models/micro/attention-4x1024x128-f16/model.py (F.sdpa),
 * CG/Pipelines/LoweringPipelines.cpp:561-595 (online attention). */
int oracle_attention_f16(const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, uint16_t *o, int64_t batch,
                         int64_t heads, int64_t seq_q, int64_t seq_kv,
                         int64_t head_dim, float scale, int causal,
                         int threads);

/* The same over strided operands with grouped-query heads: strides holds
 * the (batch, head, row) element strides of q, k, v and o in that order (d
 * contiguous), and query head h reads KV head h / (heads / kv_heads), as the
 * query heads sharing a KV head form one matmul's rows in
 * IT/models/micro/attention-cache-slice-f16/model.py:17-29. */
int oracle_attention_f16_strided(const uint16_t *q, const uint16_t *k,
                                 const uint16_t *v, uint16_t *o,
                                 int64_t batch, int64_t heads,
                                 int64_t kv_heads, int64_t seq_q,
                                 int64_t seq_kv, int64_t head_dim,
                                 const int64_t strides[12], float scale,
                                 int causal, int threads);

/* General form: iree_linalg_ext.attention with head dims head_dim (Q, K)
 * and head_dim_v (V, O), an optional f16 additive mask read through its
 * (batch, head, row, key) element strides (0 broadcasts), added after the
 * scale, and f16 (out_f32 = 0) or f32 output. Keys whose score is -inf weigh
 * 0 and a row with no other key writes 0, as the all-masked-row guard of
 * examples/attention_layer/attention_layer.mlir:80-102 does. The head dims and f32 output follow the online_attention
 * of test/codegen/pipelines/hexagon_lower_executable_target.mlir:195-233
 * (Q/K dim 4, V dim 5, scale 0.5, f32 accumulator); the mask follows the
 * optional mask operand of iree_linalg_ext.attention that
 * CG/Pipelines/LoweringPipelines.cpp:561-595 lowers. */
int oracle_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                     void *o, const uint16_t *mask, int64_t batch,
                     int64_t heads, int64_t kv_heads, int64_t seq_q,
                     int64_t seq_kv, int64_t head_dim, int64_t head_dim_v,
                     const int64_t strides[12], const int64_t mask_strides[4],
                     float scale, int causal, int out_f32, int threads);

/* chooseStaticTilingFactor, CG/Strategy/Planning/Strategies/
 * StrategySupport.cpp:38-69. dynamic bound is passed as INT64_MIN. */
int64_t oracle_choose_static_tiling_factor(int64_t static_bound,
                                           int64_t preferred,
                                           int64_t multiple_of);

/* selectHmxTileSizes restricted to a 2-D matmul root (one M, N, K; no batch),
 * CG/Strategy/Planning/VTCMPlanning.cpp:156-260 with the budget plumbing of
 * CG/Strategy/KernelDispatch.cpp:14-26 (flag budget halved when double
 * buffering, doubled back by the search).
 *   ranges      {M, N, K} static extents or upper bounds
 *   elem_bytes  {A, B, C} element sizes in bytes
 *   b_transposed  B indexed (d1, d2) instead of (d2, d1)
 *   budget_flag_bytes  --iree-hexagon-vtcm-tile-budget-bytes
 * Returns 1 and writes tiles[3] = {m, n, k} if a tile is chosen, 0 if the
 * search finds none (the planner then falls back to hexagon-mlir). */
int oracle_select_hmx_tile_sizes(const int64_t ranges[3],
                                 const int64_t elem_bytes[3], int b_transposed,
                                 int64_t budget_flag_bytes,
                                 int double_buffering, int64_t hmx_m,
                                 int64_t hmx_n, int64_t tiles[3]);

#ifdef __cplusplus
}
#endif
#endif /* IHP_ORACLE_H_ */
