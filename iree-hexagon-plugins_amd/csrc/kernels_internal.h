// Internal interface between the C-ABI layer (abi.cpp), the planner and the
// HIP kernel translation units. Not installed; the public boundary is
// include/iree_mi355x_*.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ihp {

enum ElemKind { kElemF16 = 0, kElemI8 = 1 };

// B operand forms of the fast (LDS-DMA MFMA) kernel.
enum BMode {
  kBTN = 0,    // B [N,K], same type as A
  kBNN16 = 1,  // B [K,N] f16
  kBW8 = 2,    // B [K,N] int8 with per-column f16 scale (W8A16)
  kBNN8 = 3,   // B [K,N] int8, int8 A (row-major int8 weights)
};

// One matmul launch: C[M,N] = [C +] A[M,K] . B (B [K,N] or [N,K]).
struct MatmulArgs {
  const void *a;
  const void *b;
  void *c;
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  int b_transposed;
  int accumulate;
  void *stream;
  const void *scale;  // W8A16 per-column scale (else NULL)
  // split-K configurations: split count, K elements per split, workspace
  // ([counter region][partials, batch x splits x M x N accumulators])
  int splits;
  int k_split;
  void *workspace;
  // Stream-K (split configurations, batch 1): K stages per workgroup run and
  // the workgroup count; `splits` is then the most runs any tile spans (the
  // partial layers). 0 = one tile (split) per workgroup.
  int sk_steps = 0;
  int sk_workgroups = 0;
  // Batch (grid z): element strides between consecutive matrices of A, B, C
  // (0 = one matrix shared by every batch).
  int64_t batch = 1;
  int64_t sa = 0, sb = 0, sc = 0;
  // Fused epilogue (f16 / f32 outputs): out = [C +] mul * act(acc + bias).
  const void *bias = nullptr;  // f16 [N]
  const void *mul = nullptr;   // f16 [M, N] per batch, row pitch ld_mul
  int64_t ld_mul = 0, s_mul = 0;
  int act = 0;                 // kActNone / kActRelu / kActGeluTanh / kActSilu
  int a_transposed = 0;        // A stored [K,M] (lda >= M)
};

enum Activation { kActNone = 0, kActRelu = 1, kActGeluTanh = 2, kActSilu = 3 };

// Device-side view of the fused epilogue; `mul` already points at this
// batch's matrix.
struct Epi {
  const _Float16 *bias;
  const _Float16 *mul;
  int64_t ld_mul;
  int act;
};
inline Epi make_epi(const MatmulArgs &a) {
  return Epi{(const _Float16 *)a.bias, (const _Float16 *)a.mul, a.ld_mul,
             a.act};
}
// Batch stride of the multiplier as the kernels take it: 0 without a
// multiplier, so a kernel offsets `mul` by z * stride with no branch and a
// null multiplier stays null.
inline int64_t epi_batch_stride(const MatmulArgs &a) {
  return a.mul ? a.s_mul : 0;
}

// Every workspace starts with one fixed counter region: one u32 arrival
// counter per tile (split-K GEMM) or column block (GEMV), left at zero by
// every call. Each counter has a 128-byte line of its own (kCounterStride
// u32 apart): counters sharing a line serialized the arrivals of all their
// workgroups (up to 2 us for the last of 256 GEMV workgroups). The region's
// size does not depend on the shape, so no call's partials can overlap
// another call's counters on a shared workspace.
constexpr int kCounterStride = 32;
constexpr size_t kWorkspaceCounterBytes = 256 * 1024;
constexpr int64_t kMaxWorkspaceCounters =
    kWorkspaceCounterBytes / (4 * kCounterStride);
inline size_t split_counter_bytes(int64_t tiles) {
  (void)tiles;
  return kWorkspaceCounterBytes;
}

// An operand the fast (LDS-DMA) kernels can stream: 16-byte aligned base,
// row pitch and batch stride, and a row pitch below 8 MiB, so that a
// macro-tile's lane offsets (at most 256 rows of pitch) fit the 32-bit
// offsets of the copy side. Any other operand takes the general kernel.
constexpr int64_t kMaxFastPitchBytes = (int64_t)1 << 23;
inline bool fast_operand(const void *p, int64_t ld_bytes,
                         int64_t batch_stride_bytes = 0) {
  return (uintptr_t)p % 16 == 0 && ld_bytes % 16 == 0 &&
         ld_bytes < kMaxFastPitchBytes && batch_stride_bytes % 16 == 0;
}

// While set, the C-ABI entry points on this thread validate and plan only:
// no allocation, no launch; the workspace the call needs is written to
// *sink. nullptr ends it.
void set_dry_run(size_t *sink);

typedef hipError_t (*FastLaunchFn)(const MatmulArgs &);

// One compiled kernel: its name, entry (for hipFuncGetAttributes), the
// workgroup size it is launched with, and the executable-library exports
// that may launch it (bit i = export ordinal i; 0 = runtime-internal).
struct KernelEntry {
  const char *name;
  const void *fn;
  int threads;
  uint32_t exports;
};
constexpr uint32_t kExportMatmulF16 = 1u << 0;
constexpr uint32_t kExportMatmulI8 = 1u << 1;
constexpr uint32_t kExportW8A16 = 1u << 2;
constexpr uint32_t kExportAttention = 1u << 3;
constexpr uint32_t kExportBatchMatmulF16 = 1u << 4;
const KernelEntry *gemm_kernels(int *count);
const KernelEntry *gemv_kernels(int *count);
const KernelEntry *attention_kernels(int *count);
const KernelEntry *runtime_kernels(int *count);

// A compiled fast-path (LDS-DMA MFMA) GEMM configuration.
struct FastConfig {
  const char *name;
  int b_mode;    // BMode
  int split_k;   // K split over grid.y, M may be ragged (skinny shapes)
  int a_trans;   // A stored [K,M] (f16 only, exact tiling)
  const void *kernel;  // the instantiated kernel (resource queries)
  int elem;      // ElemKind of A (and of B unless kBW8)
  int out_f32;   // f16 path: f32 output (i8 path: always i32)
  int bm, bn;    // macro-tile
  int bk;        // K elements per LDS stage
  int threads;   // workgroup size
  int stages;    // LDS ring depth
  int lds_bytes; // static LDS per workgroup
  FastLaunchFn launch;
  int mfma;      // MFMA shape: 32 (32x32) or 16 (16x16)
  int table_only;  // chosen only by a measured planner entry, never ranked
  // Column split (unsplit, batch 1): the configuration named `head` runs
  // over columns [0, n_head) in whole rounds of the chip's CUs, then `tail`
  // over [n_head, N) as a second grid on the same stream
  // (column_split_head). Null for a single-grid configuration.
  const char *head = nullptr;
  const char *tail = nullptr;
};

// The CUs a column split's head grid fills in whole rounds (MI355X: 256).
constexpr int64_t kColumnSplitCus = 256;

// Columns [0, n_head) of an M x N output that head tiles (hbm x hbn) cover
// in whole rounds of `cus` workgroups, when the remaining columns fit one
// round of tail tiles (tbm x tbn): 0 where no such split exists (M not
// tiled by either, the head grid not a whole number of rounds, no
// remainder, or a remainder of more than one tail round).
inline int64_t column_split_head(int64_t m, int64_t n, int64_t hbm,
                                 int64_t hbn, int64_t tbm, int64_t tbn,
                                 int64_t cus) {
  if (m <= 0 || m % hbm != 0 || m % tbm != 0 || cus % (m / hbm) != 0)
    return 0;
  const int64_t round_cols = cus / (m / hbm) * hbn;
  const int64_t head = n / round_cols * round_cols;
  if (head == 0 || head == n || (n - head) % tbn != 0 ||
      (m / tbm) * ((n - head) / tbn) > cus)
    return 0;
  return head;
}

const FastConfig *fast_configs(int *count);

enum GeneralKind {
  kGeneralF16F16 = 0,
  kGeneralF16F32 = 1,
  kGeneralI8I32 = 2,
  kGeneralW8A16 = 3,
};
hipError_t launch_general(const MatmulArgs &a, GeneralKind kind,
                          const void *scale);

// Skinny (M <= kGemvMaxRows) matmul with B [K,N] row-major: split-K streaming
// kernel with an in-kernel last-arriver reduction over `splits` partials.
constexpr int kGemvMaxRows = 4;
constexpr int kGemvThreads = 512;
constexpr int kGemvTargetWgs = 256;
struct GemvPlan {
  int splits;          // K split count (grid y)
  int halves;          // 1: a wave streams one row; 2: two 32-lane halves
  int cols_per_wg;     // output columns per workgroup
  int k_chunk;         // rows of W per workgroup
  int rows_per_wave;   // contiguous rows each of the 8 waves streams
  int64_t col_blocks;  // grid x
};
GemvPlan gemv_plan(int64_t m, int64_t n, int64_t k, int w_bytes,
                   int64_t batch = 1);
size_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int w_bytes,
                            int64_t batch = 1);
// w_bytes = 2: f16 weights (scale == NULL); 1: int8 weights with f16 scale.
// With a.b_transposed (W [N,K], K contiguous) the row-dot kernel runs: no K
// split, no workspace.
hipError_t launch_gemv(const MatmulArgs &a, int w_bytes, const void *scale,
                       int out_f32, void *workspace);

// Row-dot form (W [N,K]): x rows staged whole in LDS, at most this many
// bytes of them (m x k x 2), so that a workgroup's LDS (x and the column
// counter) stays under 64 KiB; workgroups per launch (columns dealt in equal
// runs, taken by the waves one at a time).
constexpr int64_t kRowdotMaxXBytes = 60 * 1024;
// W8A16 with W [N,K] and M <= this runs as row-dot launches of at most 8
// rows of x each (each re-reads W): the MFMA tiles take int8 weights only as
// [K,N], and the general kernel is several times slower.
constexpr int kRowdotMaxRowsW8A16 = 16;
// Rows of x per W8A16 row-dot launch: as many as the LDS limit allows (at
// most 8), dealt evenly over the launches M needs; 0 if one row of x does
// not fit.
inline int rowdot_w8a16_rows(int64_t m, int64_t k) {
  int64_t cap = k > 0 ? kRowdotMaxXBytes / (2 * k) : 0;
  if (cap > 8)
    cap = 8;
  if (cap < 1 || m < 1)
    return 0;
  const int64_t launches = (m + cap - 1) / cap;
  return (int)((m + launches - 1) / launches);
}
constexpr int kRowdotMaxWgs = 512;
inline int64_t rowdot_workgroups(int64_t n) {
  const int64_t w = (n + 7) / 8;
  return w < kRowdotMaxWgs ? w : kRowdotMaxWgs;
}

// Where attention's operands live: element strides of the batch, head and
// row dimensions of each (d is contiguous), and the query heads that share
// one K / V head (query head h reads KV head h / group). Checked on the host:
// every stride a multiple of 8 elements, every row of K and V within 4 GiB
// of its head's base (the copies address a head with 32-bit offsets).
struct AttentionLayout {
  int64_t q[3], k[3], v[3], o[3];  // batch, head, row
  int heads, group, seq_q, seq_kv;
  // An additive f16 mask (launches given one): (batch, head, row) element
  // strides, keys contiguous. Checked on the host: strides multiples of 4,
  // the base 8-byte aligned, seq_kv a multiple of 4.
  int64_t m[3];
};

hipError_t launch_attention(const void *q, const void *k, const void *v,
                            void *o, int64_t batch,
                            const AttentionLayout &layout, int64_t head_dim,
                            float scale, int causal, void *stream,
                            const void *mask = nullptr, int out_f32 = 0);

// The general attention kernel's view (attention_general.hip): strides as
// AttentionLayout plus the mask's (batch, head, row, key) element strides
// (0 broadcasts), the two head dims, the scale and the causal flag. Host
// checks: head dims 1..256, heads and batch at most 65535.
struct AttentionGeneralLayout {
  int64_t q[3], k[3], v[3], o[3];
  int64_t mask[4];
  int heads, group, seq_q, seq_kv, dqk, dv;
  float scale;
  int causal;
  // K (V) rows start 16-byte aligned and their head dim is a multiple of 8:
  // the kernel fills LDS 16 bytes at a time.
  int vec_k, vec_v;
};
hipError_t launch_attention_general(const void *q, const void *k,
                                    const void *v, void *o, const void *mask,
                                    int64_t batch,
                                    const AttentionGeneralLayout &layout,
                                    int out_f32, void *stream);
const KernelEntry *attention_general_kernels(int *count);

#ifdef __HIP_DEVICE_COMPILE__
#define IHP_HD __device__
#else
#define IHP_HD __host__ __device__
#endif

template <typename TA, typename TB>
struct MfmaInput {
  typedef _Float16 type;
};
template <>
struct MfmaInput<int8_t, int8_t> {
  typedef int8_t type;
};

// out = mul[row][col] * act(v + bias[col]), in f32 (the accumulator is not
// rounded first). GELU is the tanh form the reference's epilogue fusion test
// computes (plugins/compiler/hexagon/test/codegen/pipelines/
// hexagon_hmx_epilogue_keeps_config.mlir: 0.5 h (1 + tanh(0.7978 (h + 0.0447
// h^3)))); SiLU is v / (1 + e^-v).
//
// Both smooth activations are v * sigmoid(a): SiLU with a = v, and GELU with
// a = 2u, since 0.5 (1 + tanh(u)) = 1 / (1 + e^-2u). The sigmoid is one
// hardware exp2 and one reciprocal (each within ~1 ulp of f32), so the
// epilogue stays a few instructions; e^-a overflowing to +inf gives 0, and
// underflowing to 0 gives 1, the limits of the function.
__device__ __forceinline__ float sigmoid_fast(float a) {
  const float e = __builtin_amdgcn_exp2f(-a * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float epi_apply(float v, int64_t row, int64_t col,
                                           const Epi &e) {
  if (e.bias)
    v += (float)e.bias[col];
  if (e.act == kActRelu) {
    v = v > 0.0f ? v : 0.0f;
  } else if (e.act != kActNone) {
    const float a =
        e.act == kActGeluTanh
            ? 1.5957691216057308f * (v + 0.044715f * v * v * v)
            : v;
    v *= sigmoid_fast(a);
  }
  if (e.mul)
    v *= (float)e.mul[row * e.ld_mul + col];
  return v;
}

__device__ __forceinline__ bool epi_plain(const Epi &e) {
  return !e.bias && !e.mul && e.act == kActNone;
}

// Output store modes (the MFMA kernel's `store_mode` argument): plain store,
// C += result, or (outputs of unsplit tiles only) a store written through
// past this XCD's L2 (sc1). The kernel does not read its output again, and
// written through it leaves no dirty lines for the L2 write-back at the end
// of the kernel: measured 0.7-2.5 % on the int8 4096^3 matmul, whose 64 MiB
// i32 output otherwise sat dirty in the L2s, and 0.6 % on the f16 4096^3
// and 2048 x 4096 x 4096 matmuls. The launcher chooses it for outputs of at
// least kStoreThroughBytes; the kernel tests it once, outside its store loop
// (a per-element three-way test slowed the f16 kernels ~5 %), and paths that
// store element by element treat it as a plain store.
constexpr int kStorePlain = 0;
constexpr int kStoreAccumulate = 1;
constexpr int kStoreThrough = 2;
constexpr int64_t kStoreThroughBytes = 8 << 20;

// Issued as asm: no wait follows a store.
__device__ __forceinline__ void store_through(int32_t *p, int32_t v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v)
               : "memory");
}

// Accumulating store when `mode` is kStoreAccumulate, plain otherwise
// (kStoreThrough included: element stores are not written through).
__device__ __forceinline__ void store_out(float *p, float v, int mode) {
  *p = mode == kStoreAccumulate ? *p + v : v;
}
__device__ __forceinline__ void store_out(_Float16 *p, float v, int mode) {
  *p = (_Float16)(mode == kStoreAccumulate ? (float)*p + v : v);
}
__device__ __forceinline__ void store_out(int32_t *p, int v, int mode) {
  // two's-complement wrap, like the i32 adds of the CPU path
  *p = mode == kStoreAccumulate ? (int32_t)((uint32_t)*p + (uint32_t)v) : v;
}

}  // namespace ihp
