// Executable library table (include/iree_mi355x_executable_library.h): one
// export per matched dispatch kind, each decoding its push constants and
// bindings, checking that every binding covers what the kernel will touch,
// and calling the flat entry point on the dispatch's stream.
#include <cstring>

#include "../../include/iree_mi355x_executable_library.h"
#include "../../include/iree_mi355x_kernels.h"

namespace ihp {
int fail(int status, const char *fmt, ...);
}

namespace {

using ihp::fail;

int64_t u64(const uint32_t *c, int i) {
  return (int64_t)((uint64_t)c[i] | ((uint64_t)c[i + 1] << 32));
}

// Bytes a row-major [rows, cols] operand with leading dimension ld occupies.
int64_t span(int64_t rows, int64_t cols, int64_t ld, int64_t elem) {
  if (rows <= 0 || cols <= 0)
    return 0;
  return ((rows - 1) * ld + cols) * elem;
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
  int st;
  if ((st = check_binding(s, 0, span(c.m, c.k, c.lda, ab), who)) ||
      (st = check_binding(
           s, 1, bt ? span(c.n, c.k, c.ldb, bb) : span(c.k, c.n, c.ldb, bb),
           who)) ||
      (st = check_binding(s, c_index, span(c.m, c.n, c.ldc, cb), who)))
    return st;
  return IREE_MI355X_OK;
}

int dispatch_matmul_f16(const iree_mi355x_executable_environment_t *,
                        const iree_mi355x_executable_dispatch_state_t *s) {
  MatmulConsts c;
  int st = decode_matmul(s, 3, &c);
  if (st)
    return st;
  const int64_t cb = (c.flags & IREE_MI355X_MATMUL_OUT_F32) ? 4 : 2;
  if ((st = check_matmul_bindings(s, c, 2, 2, cb, 2, "matmul_f16")))
    return st;
  return iree_mi355x_matmul_f16(s->binding_ptrs[0], s->binding_ptrs[1],
                                s->binding_ptrs[2], c.m, c.n, c.k, c.lda,
                                c.ldb, c.ldc, c.flags, nullptr, 0, s->stream);
}

int dispatch_matmul_i8(const iree_mi355x_executable_environment_t *,
                       const iree_mi355x_executable_dispatch_state_t *s) {
  MatmulConsts c;
  int st = decode_matmul(s, 3, &c);
  if (st)
    return st;
  if ((st = check_matmul_bindings(s, c, 1, 1, 4, 2, "matmul_i8")))
    return st;
  return iree_mi355x_matmul_i8((const int8_t *)s->binding_ptrs[0],
                               (const int8_t *)s->binding_ptrs[1],
                               (int32_t *)s->binding_ptrs[2], c.m, c.n, c.k,
                               c.lda, c.ldb, c.ldc, c.flags, s->stream);
}

int dispatch_w8a16(const iree_mi355x_executable_environment_t *,
                   const iree_mi355x_executable_dispatch_state_t *s) {
  MatmulConsts c;
  int st = decode_matmul(s, 4, &c);
  if (st)
    return st;
  if ((st = check_matmul_bindings(s, c, 2, 1, 2, 3, "w8a16_matmul")) ||
      (st = check_binding(s, 2, c.n > 0 ? c.n * 2 : 0, "w8a16_matmul")))
    return st;
  return iree_mi355x_w8a16_matmul(
      s->binding_ptrs[0], (const int8_t *)s->binding_ptrs[1],
      s->binding_ptrs[2], s->binding_ptrs[3], c.m, c.n, c.k, c.lda, c.ldb,
      c.ldc, c.flags, nullptr, 0, s->stream);
}

int dispatch_attention(const iree_mi355x_executable_environment_t *,
                       const iree_mi355x_executable_dispatch_state_t *s) {
  if (!s || s->constant_count < 7 || !s->constants || s->binding_count < 4 ||
      !s->binding_ptrs || !s->binding_lengths)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "attention_f16: constants or bindings missing");
  const uint32_t *c = s->constants;
  const int64_t batch = c[0], heads = c[1], sq = c[2], skv = c[3], d = c[4];
  float scale;
  memcpy(&scale, &c[5], 4);
  const int64_t q_bytes = batch * heads * sq * d * 2;
  const int64_t kv_bytes = batch * heads * skv * d * 2;
  int st;
  if ((st = check_binding(s, 0, q_bytes, "attention_f16")) ||
      (st = check_binding(s, 1, kv_bytes, "attention_f16")) ||
      (st = check_binding(s, 2, kv_bytes, "attention_f16")) ||
      (st = check_binding(s, 3, q_bytes, "attention_f16")))
    return st;
  return iree_mi355x_attention_f16(s->binding_ptrs[0], s->binding_ptrs[1],
                                   s->binding_ptrs[2], s->binding_ptrs[3],
                                   batch, heads, sq, skv, d, scale, c[6],
                                   s->stream);
}

const iree_mi355x_executable_library_header_t kHeader = {
    IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, "iree_mi355x_gfx950"};

const iree_mi355x_executable_dispatch_fn_t kPtrs[] = {
    dispatch_matmul_f16, dispatch_matmul_i8, dispatch_w8a16,
    dispatch_attention};

const iree_mi355x_executable_dispatch_attrs_t kAttrs[] = {
    {IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
         IREE_MI355X_DISPATCH_FLAG_USES_MFMA |
         IREE_MI355X_DISPATCH_FLAG_USES_LDS_DMA |
         IREE_MI355X_DISPATCH_FLAG_USES_WORKSPACE,
     163840, 512},
    {IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
         IREE_MI355X_DISPATCH_FLAG_USES_MFMA |
         IREE_MI355X_DISPATCH_FLAG_USES_LDS_DMA,
     163840, 512},
    {IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
         IREE_MI355X_DISPATCH_FLAG_USES_MFMA |
         IREE_MI355X_DISPATCH_FLAG_USES_WORKSPACE,
     49152 + 4, 256},
    {IREE_MI355X_DISPATCH_FLAG_RESOURCES_VALID |
         IREE_MI355X_DISPATCH_FLAG_USES_MFMA,
     16384 + 128 * 68 * 2, 256},
};

const char *const kNames[] = {"matmul_f16", "matmul_i8", "w8a16_matmul",
                              "attention_f16"};

const iree_mi355x_executable_library_t kLibrary = {
    &kHeader,
    {0, nullptr},
    {4, kPtrs, kAttrs, kNames},
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
