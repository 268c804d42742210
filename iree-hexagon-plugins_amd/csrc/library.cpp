// Executable library table (include/iree_mi355x_executable_library.h): one
// export per matched dispatch kind, each decoding its push constants and
// bindings, checking that every binding covers what the kernel will touch,
// and calling the flat entry point on the dispatch's stream.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/iree_mi355x_executable_library.h"
#include "../../include/iree_mi355x_kernels.h"
#include "kernels_internal.h"

namespace ihp {
int fail(int status, const char *fmt, ...);
}

namespace {

using ihp::fail;
using ihp::set_dry_run;

int64_t u64(const uint32_t *c, int i) {
  return (int64_t)((uint64_t)c[i] | ((uint64_t)c[i + 1] << 32));
}

// Checked int64 arithmetic for binding sizes computed from caller constants:
// any overflow, or a negative operand, yields -1, which check_binding
// rejects. These checks run before the entry points' own extent checks, so
// they must not wrap to a small size that a short binding would pass.
int64_t mul_checked(int64_t a, int64_t b) {
  int64_t r;
  if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r))
    return -1;
  return r;
}
int64_t add_checked(int64_t a, int64_t b) {
  int64_t r;
  if (a < 0 || b < 0 || __builtin_add_overflow(a, b, &r))
    return -1;
  return r;
}

// Bytes a row-major [rows, cols] operand with leading dimension ld occupies
// (-1 if that does not fit in int64 or ld is negative).
int64_t span(int64_t rows, int64_t cols, int64_t ld, int64_t elem) {
  if (rows <= 0 || cols <= 0)
    return 0;
  return mul_checked(add_checked(mul_checked(rows - 1, ld), cols), elem);
}

struct MatmulConsts {
  int64_t m, n, k, lda, ldb, ldc;
  uint32_t flags;
};

int decode_matmul(const iree_mi355x_executable_dispatch_state_t *s,
                  uint32_t bindings, MatmulConsts *out) {
  if (!s || s->constant_count < 13 || !s->constants ||
      s->binding_count < bindings || !s->binding_ptrs || !s->binding_lengths)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "dispatch: constants or bindings missing");
  const uint32_t *c = s->constants;
  out->m = u64(c, 0);
  out->n = u64(c, 2);
  out->k = u64(c, 4);
  out->lda = u64(c, 6);
  out->ldb = u64(c, 8);
  out->ldc = u64(c, 10);
  out->flags = c[12];
  return IREE_MI355X_OK;
}

int check_binding(const iree_mi355x_executable_dispatch_state_t *s, int i,
                  int64_t need, const char *who) {
  if (need < 0 || (size_t)need > s->binding_lengths[i])
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: binding %d holds %zu bytes, dispatch reads %lld", who, i,
                s->binding_lengths[i], (long long)need);
  return IREE_MI355X_OK;
}

int check_matmul_bindings(const iree_mi355x_executable_dispatch_state_t *s,
                          const MatmulConsts &c, int64_t ab, int64_t bb,
                          int64_t cb, int c_index, const char *who) {
  const bool bt = c.flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = c.flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  int st;
  if ((st = check_binding(
           s, 0, at ? span(c.k, c.m, c.lda, ab) : span(c.m, c.k, c.lda, ab),
           who)) ||
      (st = check_binding(
           s, 1, bt ? span(c.n, c.k, c.ldb, bb) : span(c.k, c.n, c.ldb, bb),
           who)) ||
      (st = check_binding(s, c_index, span(c.m, c.n, c.ldc, cb), who)))
    return st;
  return IREE_MI355X_OK;
}

// A dispatch whose state asks for a workspace query only validates and plans
// (see the dispatch-state declaration); the scope ends that mode on return.
struct DryRunScope {
  explicit DryRunScope(const iree_mi355x_executable_dispatch_state_t *s) {
    set_dry_run(s ? s->workspace_query : nullptr);
  }
  ~DryRunScope() { set_dry_run(nullptr); }
};

int dispatch_matmul_f16(const iree_mi355x_executable_environment_t *,
                        const iree_mi355x_executable_dispatch_state_t *s) {
  DryRunScope dry(s);
  MatmulConsts c;
  int st = decode_matmul(s, 3, &c);
  if (st)
    return st;
  const int64_t cb = (c.flags & IREE_MI355X_MATMUL_OUT_F32) ? 4 : 2;
  if ((st = check_matmul_bindings(s, c, 2, 2, cb, 2, "matmul_f16")))
    return st;
  return iree_mi355x_matmul_f16(s->binding_ptrs[0], s->binding_ptrs[1],
                                s->binding_ptrs[2], c.m, c.n, c.k, c.lda,
                                c.ldb, c.ldc, c.flags, s->workspace,
                                s->workspace_bytes, s->stream);
}

int dispatch_matmul_i8(const iree_mi355x_executable_environment_t *,
                       const iree_mi355x_executable_dispatch_state_t *s) {
  DryRunScope dry(s);
  MatmulConsts c;
  int st = decode_matmul(s, 3, &c);
  if (st)
    return st;
  if ((st = check_matmul_bindings(s, c, 1, 1, 4, 2, "matmul_i8")))
    return st;
  return iree_mi355x_matmul_i8((const int8_t *)s->binding_ptrs[0],
                               (const int8_t *)s->binding_ptrs[1],
                               (int32_t *)s->binding_ptrs[2], c.m, c.n, c.k,
                               c.lda, c.ldb, c.ldc, c.flags, s->workspace,
                               s->workspace_bytes, s->stream);
}

int dispatch_w8a16(const iree_mi355x_executable_environment_t *,
                   const iree_mi355x_executable_dispatch_state_t *s) {
  DryRunScope dry(s);
  MatmulConsts c;
  int st = decode_matmul(s, 4, &c);
  if (st)
    return st;
  if ((st = check_matmul_bindings(s, c, 2, 1, 2, 3, "w8a16_matmul")) ||
      (st = check_binding(s, 2, c.n > 0 ? mul_checked(c.n, 2) : 0,
                          "w8a16_matmul")))
    return st;
  return iree_mi355x_w8a16_matmul(
      s->binding_ptrs[0], (const int8_t *)s->binding_ptrs[1],
      s->binding_ptrs[2], s->binding_ptrs[3], c.m, c.n, c.k, c.lda, c.ldb,
      c.ldc, c.flags, s->workspace, s->workspace_bytes, s->stream);
}

// "attention_f16": batch heads seq_q seq_kv head_dim scale_bits flags, then
// optionally kv_heads and the (batch, head, row) element strides of q, k, v
// and o as lo/hi pairs (32 words in all), then optionally head_dim_v and the
// (batch, head, row, key) element strides of the mask as lo/hi pairs (41
// words). Without strides the operands are contiguous [B, H, S, D] with one
// KV head per query head; without the last part head_dim_v is head_dim and
// there is no mask. Bindings: q k v o [mask]; flags take CAUSAL, OUT_F32 and
// (41 words only) MASK.
int dispatch_attention(const iree_mi355x_executable_environment_t *,
                       const iree_mi355x_executable_dispatch_state_t *s) {
  DryRunScope dry(s);
  const char *who = "attention_f16";
  if (!s || s->constant_count < 7 || !s->constants || s->binding_count < 4 ||
      !s->binding_ptrs || !s->binding_lengths)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: constants or bindings missing", who);
  const uint32_t *c = s->constants;
  iree_mi355x_attention_t a = {};
  a.batch = c[0];
  a.heads = c[1];
  a.seq_q = c[2];
  a.seq_kv = c[3];
  a.head_dim = a.head_dim_v = c[4];
  memcpy(&a.scale, &c[5], 4);
  a.flags = c[6];
  a.kv_heads = a.heads;
  const bool strided = s->constant_count >= 32;
  const bool general = s->constant_count >= 41;
  if (general)
    a.head_dim_v = c[32];
  const bool has_mask = a.flags & IREE_MI355X_ATTENTION_MASK;
  if (has_mask && (!general || s->binding_count < 5))
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: a mask needs the 41-word constants and binding 4", who);
  int64_t *dst[4] = {a.strides.q, a.strides.k, a.strides.v, a.strides.o};
  for (int t = 0; t < 4; ++t) {
    const bool kv = t == 1 || t == 2;
    const int64_t rows = kv ? a.seq_kv : a.seq_q;
    const int64_t d = t < 2 ? a.head_dim : a.head_dim_v;
    const int64_t one[3] = {mul_checked(mul_checked(a.heads, rows), d),
                            mul_checked(rows, d), d};
    for (int i = 0; i < 3; ++i)
      dst[t][i] = strided ? u64(c, 8 + 2 * (3 * t + i)) : one[i];
  }
  if (strided)
    a.kv_heads = c[7];
  for (int i = 0; i < 4 && general; ++i)
    a.mask_strides[i] = u64(c, 33 + 2 * i);
  // Bytes from an operand's first element to the end of its last row.
  auto reach = [&](const int64_t *sd, int64_t planes_heads, int64_t rows,
                   int64_t d, int64_t elem) {
    if (a.batch <= 0 || planes_heads <= 0 || rows <= 0 || d <= 0)
      return (int64_t)0;
    const int64_t last = add_checked(
        add_checked(mul_checked(a.batch - 1, sd[0]),
                    mul_checked(planes_heads - 1, sd[1])),
        mul_checked(rows - 1, sd[2]));
    return mul_checked(add_checked(last, d), elem);
  };
  const int64_t ob = (a.flags & IREE_MI355X_ATTENTION_OUT_F32) ? 4 : 2;
  int st_ok;
  if ((st_ok = check_binding(s, 0, reach(a.strides.q, a.heads, a.seq_q,
                                         a.head_dim, 2), who)) ||
      (st_ok = check_binding(s, 1, reach(a.strides.k, a.kv_heads, a.seq_kv,
                                         a.head_dim, 2), who)) ||
      (st_ok = check_binding(s, 2, reach(a.strides.v, a.kv_heads, a.seq_kv,
                                         a.head_dim_v, 2), who)) ||
      (st_ok = check_binding(s, 3, reach(a.strides.o, a.heads, a.seq_q,
                                         a.head_dim_v, ob), who)))
    return st_ok;
  if (has_mask) {
    // The mask's rows are seq_kv long with key stride mask_strides[3].
    int64_t need = 0;
    if (a.batch > 0 && a.heads > 0 && a.seq_q > 0 && a.seq_kv > 0) {
      const int64_t *m = a.mask_strides;
      const int64_t last = add_checked(
          add_checked(mul_checked(a.batch - 1, m[0]),
                      mul_checked(a.heads - 1, m[1])),
          add_checked(mul_checked(a.seq_q - 1, m[2]),
                      mul_checked(a.seq_kv - 1, m[3])));
      need = mul_checked(add_checked(last, 1), 2);
    }
    if ((st_ok = check_binding(s, 4, need, who)))
      return st_ok;
    a.mask = s->binding_ptrs[4];
  }
  a.q = s->binding_ptrs[0];
  a.k = s->binding_ptrs[1];
  a.v = s->binding_ptrs[2];
  a.o = s->binding_ptrs[3];
  return iree_mi355x_attention(&a, s->stream);
}

// "batch_matmul_f16": the matmul_f16 constants, then batch, stride_a,
// stride_b, stride_c (lo/hi pairs), activation, epilogue bindings (bit 0:
// bias, bit 1: multiplier), ld_multiplier, batch_stride_multiplier (lo/hi).
// Bindings: a b c [bias] [multiplier].
int dispatch_batch_matmul(const iree_mi355x_executable_environment_t *,
                          const iree_mi355x_executable_dispatch_state_t *s) {
  DryRunScope dry(s);
  const char *who = "batch_matmul_f16";
  MatmulConsts c;
  int st = decode_matmul(s, 3, &c);
  if (st)
    return st;
  if (s->constant_count < 27)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: constants missing", who);
  const uint32_t *k = s->constants;
  const int64_t batch = u64(k, 13), sa = u64(k, 15), sb = u64(k, 17),
                sc = u64(k, 19);
  const uint32_t act = k[21], epi_bindings = k[22];
  const int64_t ld_mul = u64(k, 23), s_mul = u64(k, 25);
  const bool has_bias = epi_bindings & 1u, has_mul = epi_bindings & 2u;
  const uint32_t need = 3 + (has_bias ? 1 : 0) + (has_mul ? 1 : 0);
  if (s->binding_count < need || batch < 0 || sa < 0 || sb < 0 || sc < 0 ||
      s_mul < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: bindings or strides", who);
  const bool bt = c.flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = c.flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  const int64_t cb = (c.flags & IREE_MI355X_MATMUL_OUT_F32) ? 4 : 2;
  const int64_t last = batch > 0 ? batch - 1 : 0;
  auto batched = [&](int64_t stride, int64_t one, int64_t elem) {
    if (one <= 0)
      return one;  // 0: nothing read; -1: overflow
    return add_checked(mul_checked(mul_checked(last, stride), elem), one);
  };
  if ((st = check_binding(
           s, 0,
           batched(sa, at ? span(c.k, c.m, c.lda, 2) : span(c.m, c.k, c.lda, 2),
                   2),
           who)) ||
      (st = check_binding(
           s, 1,
           batched(sb, bt ? span(c.n, c.k, c.ldb, 2) : span(c.k, c.n, c.ldb, 2),
                   2),
           who)) ||
      (st = check_binding(s, 2, batched(sc, span(c.m, c.n, c.ldc, cb), cb),
                          who)))
    return st;
  iree_mi355x_epilogue_t epi = {};
  epi.activation = act;
  uint32_t next = 3;
  if (has_bias) {
    if ((st = check_binding(s, next, mul_checked(c.n, 2), who)))
      return st;
    epi.bias = s->binding_ptrs[next++];
  }
  if (has_mul) {
    if ((st = check_binding(s, next,
                            batched(s_mul, span(c.m, c.n, ld_mul, 2), 2), who)))
      return st;
    epi.multiplier = s->binding_ptrs[next++];
    epi.ld_multiplier = ld_mul;
    epi.batch_stride_multiplier = s_mul;
  }
  return iree_mi355x_batch_matmul_f16(
      s->binding_ptrs[0], s->binding_ptrs[1], s->binding_ptrs[2], batch, c.m,
      c.n, c.k, c.lda, c.ldb, c.ldc, sa, sb, sc, c.flags, &epi, s->workspace,
      s->workspace_bytes, s->stream);
}

const iree_mi355x_executable_library_header_t kHeader = {
    IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, "iree_mi355x_gfx950"};

const iree_mi355x_executable_dispatch_fn_t kPtrs[] = {
    dispatch_matmul_f16, dispatch_matmul_i8, dispatch_w8a16,
    dispatch_attention, dispatch_batch_matmul};

// Largest static LDS and workgroup of any kernel an export can launch (the
// GPU tests compare them with what the loaded kernels report): the int8
// MFMA rings (up to the row-major-B split-K tiles' 4 x 36 / 3 x 48 KiB,
// 512 threads; split-K tiles use a workspace), the f16 ones
// up to the 64x256 split-K tile's 4 x 40 KiB (all of a CU's LDS), the
// W8A16 256x256 ring (3 x 48 KiB), the GEMV (512 threads, its 8-wave
// reduction buffer at most 128 KiB), the attention K/V rings (two wave
// groups x 4 x 16 KiB) and the merge's (max, sum) exchange (2 KiB), 512
// threads.
constexpr uint64_t kF16Flags = IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
                               IREE_MI355X_DISPATCH_FLAG_USES_MFMA |
                               IREE_MI355X_DISPATCH_FLAG_USES_LDS_DMA |
                               IREE_MI355X_DISPATCH_FLAG_USES_WORKSPACE;
const iree_mi355x_executable_dispatch_attrs_t kAttrs[] = {
    {kF16Flags, 163840, 512},
    {kF16Flags, 147456, 512},
    {kF16Flags, 147456, 512},
    {IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
         IREE_MI355X_DISPATCH_FLAG_USES_MFMA |
         IREE_MI355X_DISPATCH_FLAG_USES_LDS_DMA,
     135168, 512},
    {kF16Flags, 163840, 512},
};

const char *const kNames[] = {"matmul_f16", "matmul_i8", "w8a16_matmul",
                              "attention_f16", "batch_matmul_f16"};

const iree_mi355x_executable_library_t kLibrary = {
    &kHeader,
    {0, nullptr},
    {5, kPtrs, kAttrs, kNames},
};

}  // namespace

extern "C" const iree_mi355x_executable_library_header_t **
iree_mi355x_executable_library_query(
    iree_mi355x_executable_library_version_t max_version,
    const iree_mi355x_executable_environment_t *environment) {
  (void)environment;
  if (max_version != IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST)
    return nullptr;
  // The library struct begins with its header pointer.
  return const_cast<const iree_mi355x_executable_library_header_t **>(
      &kLibrary.header);
}

// ---------------------------------------------------------------- resources

namespace {

// The kernel lists of every translation unit, in one index space.
const ihp::KernelEntry *kernel_at(int index) {
  const ihp::KernelEntry *(*lists[])(int *) = {
      ihp::gemm_kernels, ihp::gemv_kernels, ihp::attention_kernels,
      ihp::attention_general_kernels, ihp::runtime_kernels};
  for (auto list : lists) {
    int n = 0;
    const ihp::KernelEntry *e = list(&n);
    if (index < n)
      return e + index;
    index -= n;
  }
  return nullptr;
}

}  // namespace

extern "C" int iree_mi355x_kernel_count(void) {
  int total = 0, n = 0;
  ihp::gemm_kernels(&n);
  total += n;
  ihp::gemv_kernels(&n);
  total += n;
  ihp::attention_kernels(&n);
  total += n;
  ihp::attention_general_kernels(&n);
  total += n;
  ihp::runtime_kernels(&n);
  return total + n;
}

extern "C" int iree_mi355x_kernel_resources(
    int index, iree_mi355x_kernel_resources_t *out) {
  if (!out || index < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "kernel_resources: bad argument");
  const ihp::KernelEntry *e = kernel_at(index);
  if (!e)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "kernel_resources: index %d of %d", index,
                iree_mi355x_kernel_count());
  memset(out, 0, sizeof(*out));
  out->name = e->name;
  out->exports = e->exports;
  out->threads = e->threads;
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0)
    return fail(IREE_MI355X_NO_DEVICE,
                "kernel_resources: no device to load %s from", e->name);
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, e->fn) != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED,
                "kernel_resources: hipFuncGetAttributes(%s) failed", e->name);
  int resident = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, e->fn,
                                                   e->threads, 0) != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED,
                "kernel_resources: occupancy of %s failed", e->name);
  out->vgprs = attr.numRegs;
  out->lds_bytes = (int32_t)attr.sharedSizeBytes;
  out->scratch_bytes = (int32_t)attr.localSizeBytes;
  out->max_threads = attr.maxThreadsPerBlock;
  out->workgroups_per_cu = resident;
  return IREE_MI355X_OK;
}
