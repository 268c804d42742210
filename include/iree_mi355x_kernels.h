// MI355X (gfx950) matmul / attention dispatch kernels: the C-ABI boundary.
//
// This header replaces the Hexagon HMX micro-kernel ABI
// (plugins/runtime/hexagon/dsp/ukernel/hmx/api.h:16-67) for whole dispatches.
// The reference lowers one linalg.matmul dispatch into a sequence of
// pack / acc_clear / mma / acc_read / unpack calls per 32x32 HMX tile
// (CG/Transforms/HexagonExpandHmxMatmul.cpp:100-343, emitted as calls by
// CG/Conversion/HexagonHmxToLLVM.cpp:22-227). On MI355X the tile loop, the
// staging (the VTCM plan) and the K loop live inside one HIP kernel, so the
// callable unit is the whole matmul: each entry point below computes what one
// matched dispatch region computes.
//
// Conventions (all entry points):
//  * Pointers are device pointers to caller-owned buffers; sizes, leading
//    dimensions (in elements) and counts are int64_t.
//  * `stream` is a hipStream_t (NULL = the legacy default stream). Work is
//    enqueued and the call returns without waiting; calls on different
//    streams are independent unless the caller gives them one workspace.
//  * No entry point allocates, frees or synchronizes device memory: scratch
//    comes from a caller workspace (the workspace queries size it).
//  * Return value is an iree_mi355x_status_t; preconditions are checked on
//    the host before anything is launched, so an error never leaves work
//    behind. The reference ABI has no error channel (its preconditions are
//    proven at compile time by HexagonVerifyHmxRuntimeABI.cpp:84-360); here
//    the same checks return a status instead.
//  * Zero-sized M or N is a no-op; K == 0 writes C_init (or zeros).
#ifndef IREE_MI355X_KERNELS_H_
#define IREE_MI355X_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum iree_mi355x_status_e {
  IREE_MI355X_OK = 0,
  // Null pointer, negative extent, leading dimension smaller than the row,
  // unknown flag bit.
  IREE_MI355X_INVALID_ARGUMENT = 1,
  // A pointer or leading dimension breaks an alignment the kernel needs.
  IREE_MI355X_MISALIGNED = 2,
  // The shape/layout/flag combination has no kernel.
  IREE_MI355X_UNSUPPORTED = 3,
  // hipLaunchKernel (or another HIP call) failed.
  IREE_MI355X_LAUNCH_FAILED = 4,
  // No HIP device is visible.
  IREE_MI355X_NO_DEVICE = 5,
  // The caller-provided workspace is smaller than the query returned.
  IREE_MI355X_WORKSPACE_TOO_SMALL = 6,
} iree_mi355x_status_t;

// Matmul flags: the linalg.matmul indexing-map variants the plugin matcher
// accepts (ContractionStrategy.cpp:152-168 accepts an MxN output with either
// B map; CG/Transforms/HexagonConvertMatmulToHmx.cpp:51-70 packs both).
// B is stored [N, K] (indexing map (d1, d2), "column-major B").
#define IREE_MI355X_MATMUL_B_TRANSPOSED 0x1u
// DPS accumulate: C_out = C_init + A.B, as the HMX unpack adds the tile into
// the init (UK/hmx.c:328-357,426-450). Without it C is overwritten, which is
// the same result for a zero-filled init.
#define IREE_MI355X_MATMUL_ACCUMULATE 0x2u
// f16 matmul only: write f32 C instead of f16.
#define IREE_MI355X_MATMUL_OUT_F32 0x4u
// f16 matmul only: A is stored [K, M] (indexing map (d2, d0), a transposed
// LHS), lda >= M. Combines with B_TRANSPOSED
// (test/codegen/transforms/convert_matmul_to_hmx.mlir:87-115 packs such an A
// along its second dimension).
#define IREE_MI355X_MATMUL_A_TRANSPOSED 0x8u

// Attention flags.
#define IREE_MI355X_ATTENTION_CAUSAL 0x1u
// iree_mi355x_attention only: write f32 o instead of f16.
#define IREE_MI355X_ATTENTION_OUT_F32 0x2u
// iree_mi355x_attention only: an additive mask is given (set exactly when
// the mask pointer is not NULL; in the executable library's attention_f16
// dispatch, the mask is binding 4).
#define IREE_MI355X_ATTENTION_MASK 0x4u

// f16 x f16 matmul with f32 accumulation (inputs widened with arith.extf, as
// in examples/matmul/matmul.mlir:1-14), f16 or f32 output rounded once at the
// end (RNE).
//   a: [M, K] row-major, lda >= K
//   b: [K, N] row-major (ldb >= N) or [N, K] with B_TRANSPOSED (ldb >= K)
//   c: [M, N] row-major, ldc >= N; f16, or f32 with OUT_F32
// M <= 4 with row-major B dispatches to the HBM-streaming GEMV kernel; a
// ragged M or a skinny M the macro-tiles leave idle splits K over the CUs.
// Replaces iree_hexagon_hmx_pack_f16 / pack_transposed_f16 / mma_f16 /
// acc_read_f16 / unpack_acc_f16_to_{f16,f32} (UK/api.h:28-67) as sequenced
// by HexagonExpandHmxMatmul.cpp:286-331.
int iree_mi355x_matmul_f16(const void *a, const void *b, void *c, int64_t m,
                           int64_t n, int64_t k, int64_t lda, int64_t ldb,
                           int64_t ldc, uint32_t flags, void *workspace,
                           size_t workspace_bytes, void *stream);

// Activations of the fused epilogue.
#define IREE_MI355X_ACT_NONE 0u
#define IREE_MI355X_ACT_RELU 1u
// 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))), the GELU form of the
// reference's epilogue-fusion test (plugins/compiler/hexagon/test/codegen/
// pipelines/hexagon_hmx_epilogue_keeps_config.mlir).
#define IREE_MI355X_ACT_GELU_TANH 2u
#define IREE_MI355X_ACT_SILU 3u  // v / (1 + e^-v)

// Elementwise epilogue fused into a matmul's store, computed in f32 on the
// f32 accumulator and rounded once:
//   out[m][n] = [C_init[m][n] +] multiplier[m][n] * act(acc[m][n] + bias[n])
// (the linalg.generic consumers the reference fuses after a matmul: bias add,
// activation, gating multiply, e.g. a GeGLU gate). Every member is optional:
// a NULL pointer drops its term.
typedef struct iree_mi355x_epilogue_t {
  const void *bias;        // f16 [N], shared by every row and batch
  const void *multiplier;  // f16 [M, N] per batch, row pitch ld_multiplier
  int64_t ld_multiplier;
  int64_t batch_stride_multiplier;  // elements between batches (0 = shared)
  uint32_t activation;              // IREE_MI355X_ACT_*
} iree_mi355x_epilogue_t;

// Strided batched f16 matmul with an optional fused epilogue
// (linalg.batch_matmul, e.g. LIT/integration/hmx_batched_matmul.mlir and the
// micro model batch-matmul-4x1024x1024x128): for b in [0, batch),
//   C + b*stride_c = epilogue(A + b*stride_a . B + b*stride_b)
// with the layouts and flags of iree_mi355x_matmul_f16. Strides are in
// elements; stride_a or stride_b 0 shares one operand across the batch
// (broadcast weights), stride_c must separate the outputs. batch <= 65535.
// iree_mi355x_matmul_f16 is this call with batch 1 and no epilogue.
int iree_mi355x_batch_matmul_f16(const void *a, const void *b, void *c,
                                 int64_t batch, int64_t m, int64_t n,
                                 int64_t k, int64_t lda, int64_t ldb,
                                 int64_t ldc, int64_t stride_a,
                                 int64_t stride_b, int64_t stride_c,
                                 uint32_t flags,
                                 const iree_mi355x_epilogue_t *epilogue,
                                 void *workspace, size_t workspace_bytes,
                                 void *stream);

// Workspace a batch_matmul_f16 call of this shape needs (0 if none).
size_t iree_mi355x_batch_matmul_workspace_bytes(int64_t batch, int64_t m,
                                                int64_t n, int64_t k,
                                                uint32_t flags);

// i8 x i8 -> i32 matmul, exact (linalg.matmul i8,i8->i32 or
// linalg.quantized_matmul with zero points 0). Same layouts, flags and
// workspace rules as iree_mi355x_matmul_f16 except OUT_F32 and
// A_TRANSPOSED. The reference has no accelerator kernel for it
// (ContractionStrategy.cpp:138-150, int8 TODO at :141); it runs the generic
// HVX path, whose semantics this keeps bit for bit.
int iree_mi355x_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c,
                          int64_t m, int64_t n, int64_t k, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t flags,
                          void *workspace, size_t workspace_bytes,
                          void *stream);

// W8A16 linear: y[m,n] = f16((sum_k f32(x[m,k]) * f32(w[k,n])) * f32(s[n])),
// zero point 0, dequantization fused into the kernel.
//   x: [M, K] f16 row-major; w: [K, N] int8 (or [N, K] with B_TRANSPOSED);
//   scale: [N] f16; y: [M, N] f16.
// No reference kernel matches a dequant-fused matmul (repo-wide); semantics
// follow the CPU path of the same linalg form.
int iree_mi355x_w8a16_matmul(const void *x, const int8_t *w, const void *scale,
                             void *y, int64_t m, int64_t n, int64_t k,
                             int64_t ldx, int64_t ldw, int64_t ldy,
                             uint32_t flags, void *workspace,
                             size_t workspace_bytes, void *stream);

// Fused attention forward, f16 in/out, f32 scores and softmax:
//   o = softmax(q k^T * scale + mask) v
// q: [B, H, Sq, D], k/v: [B, H, Skv, D], o: [B, H, Sq, D], all contiguous.
// CAUSAL masks key j for query i when j > i (top-left aligned).
// head_dim must be 64 or 128. The reference decomposes attention into
// batch_matmul + softmax generics (examples/attention_layer/
// attention_layer.mlir:48-105) or, for iree_linalg_ext.attention, into an
// online-softmax loop (CG/Pipelines/LoweringPipelines.cpp:561-595); this is
// that online-softmax loop as one kernel.
int iree_mi355x_attention_f16(const void *q, const void *k, const void *v,
                              void *o, int64_t batch, int64_t heads,
                              int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                              float scale, uint32_t flags, void *stream);

// Where each attention operand lives: the element strides of its batch,
// head and row (sequence) dimensions; its head_dim elements are contiguous.
// k and v are indexed by KV head.
typedef struct iree_mi355x_attention_strides_t {
  int64_t q[3];
  int64_t k[3];
  int64_t v[3];
  int64_t o[3];
} iree_mi355x_attention_strides_t;

// iree_mi355x_attention_f16 over strided operands with grouped-query heads:
// query head h (of `heads`) attends with KV head h / (heads / kv_heads).
// K / V may be the first seq_kv rows of a longer KV cache and O may be laid
// out [B, Sq, H, D]: the attention of
// integration_tests/models/micro/attention-cache-slice-f16/model.py:10-29
// (9 query heads over 3 KV heads, the first 64 of 128 cache rows, the
// output permuted to [batch, seq, heads, dim]). heads must be a multiple of
// kv_heads; every stride a multiple of 8 elements and every pointer 16-byte
// aligned; each head's q, k and v rows must lie within 4 GiB of its first
// row. o's row stride must be at least head_dim, and distinct (batch, head,
// row) must not share o elements (not checked beyond the row stride).
// iree_mi355x_attention_f16 is this call with contiguous strides and
// kv_heads == heads.
int iree_mi355x_attention_f16_strided(
    const void *q, const void *k, const void *v, void *o, int64_t batch,
    int64_t heads, int64_t kv_heads, int64_t seq_q, int64_t seq_kv,
    int64_t head_dim, float scale, uint32_t flags,
    const iree_mi355x_attention_strides_t *strides, void *stream);

// Attention in general form: iree_linalg_ext.attention with any head dims,
// an optional additive mask and an f16 or f32 output, as the reference
// lowers it (CG/Pipelines/LoweringPipelines.cpp:561-595; the online_attention
// of its pipeline test test/codegen/pipelines/
// hexagon_lower_executable_target.mlir:195-233 has a Q/K head dim of 4, a V
// head dim of 5, an f16 scale of 0.5 and an f32 accumulator):
//   o = softmax(q k^T * scale + mask [+ causal]) v
// q [B, H, Sq, head_dim], k [B, H_kv, Skv, head_dim], v [B, H_kv, Skv,
// head_dim_v], o [B, H, Sq, head_dim_v] (f32 with OUT_F32), each through its
// (batch, head, row) strides in elements, the head dim contiguous; mask, if
// not NULL, an f16 [B, H, Sq, Skv] view through its (batch, head, row, key)
// strides (0 broadcasts a dimension) added to the scaled scores. A row whose
// keys are all masked (-inf) writes 0, as the all-masked guard of the
// decomposed softmax does (examples/attention_layer/attention_layer.mlir:
// 80-102). head_dim and head_dim_v are 1..256, heads a multiple of
// kv_heads, heads and batch at most 65535. Shapes the MFMA kernel takes
// (equal head dims that are multiples of 16 up to 128, f16 or f32 output,
// the alignment of iree_mi355x_attention_f16_strided, and a mask if any with
// contiguous keys, its other strides and base 8-byte aligned and seq_kv a
// multiple of 4) run there; the rest run a general kernel (32-key blocks in
// LDS, f32 online softmax). _f16 and _f16_strided take head dims 64 and
// 128 only, on the MFMA kernel.
typedef struct iree_mi355x_attention_t {
  const void *q, *k, *v;
  void *o;
  const void *mask;  // f16 additive mask (with ATTENTION_MASK), or NULL
  int64_t batch, heads, kv_heads, seq_q, seq_kv;
  int64_t head_dim, head_dim_v;
  float scale;
  uint32_t flags;  // IREE_MI355X_ATTENTION_CAUSAL | _OUT_F32 | _MASK
  iree_mi355x_attention_strides_t strides;
  int64_t mask_strides[4];  // batch, head, row, key
} iree_mi355x_attention_t;
int iree_mi355x_attention(const iree_mi355x_attention_t *args, void *stream);

// Workspace a matmul_f16 / matmul_i8 / w8a16_matmul call of this shape
// needs (split-K
// partials and arrival counters), 0 if none. Mirrors the scratch query of the
// reference's caller-scratch matmul, hexkl_matmul_f16f16_f32_scratch_bytes
// (CG/Conversion/HexagonRuntimeLinking.h:35-38). The library allocates no
// device memory: a call whose plan needs a workspace and gets none, or a
// smaller one, returns IREE_MI355X_WORKSPACE_TOO_SMALL before anything is
// launched. A workspace must be zero-filled before its first use and is left
// zero-filled in its counter region (its first 256 KiB) after every call, so
// one workspace serves any sequence of calls of any shapes; calls that
// overlap must not share one. The value covers every layout the call may run
// with, the M = 1 transposed-A row included.
size_t iree_mi355x_matmul_workspace_bytes(int64_t m, int64_t n, int64_t k,
                                          uint32_t flags);

// iree_mi355x_matmul_f16 without any allocation: the split-K partials and
// arrival counters live in the library's own device scratch (32 MiB per GPU,
// a static device array held until the process ends) instead of a caller
// workspace, so the caller needs no device memory of its own for them.
// No counterpart in the reference: it is for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc). A shape whose plan needs more scratch than that returns
// IREE_MI355X_WORKSPACE_TOO_SMALL before anything is launched. Every call
// on one GPU shares that GPU's scratch: calls that overlap on a GPU (on
// different streams, or graphs replayed concurrently) race and must be
// ordered by the caller.
int iree_mi355x_matmul_f16_no_alloc(const void *a, const void *b, void *c,
                                    int64_t m, int64_t n, int64_t k,
                                    int64_t lda, int64_t ldb, int64_t ldc,
                                    uint32_t flags, void *stream);

// Last error message recorded on this thread (empty string if none).
const char *iree_mi355x_last_error(void);

// Library version string and the number of visible devices (0 without GPU);
// neither launches work.
const char *iree_mi355x_version(void);
int iree_mi355x_device_count(void);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_KERNELS_H_
