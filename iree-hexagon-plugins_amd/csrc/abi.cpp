// C-ABI entry points (include/iree_mi355x_kernels.h): host-side argument
// checks, kernel selection and launch.
//
// The reference proves its kernels' preconditions at compile time
// (CG/Transforms/HexagonVerifyHmxRuntimeABI.cpp:84-360: placement, row-major
// layout, 64/128/2048-byte alignment, extents that fit) and its kernels have
// no error channel (UK/api.h). Here every check runs on the host before
// launch and reports an iree_mi355x_status_t; nothing is launched on error.
#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/iree_mi355x_kernels.h"
#include "../../include/iree_mi355x_planner.h"
#include "kernels_internal.h"

namespace ihp {

static thread_local char g_last_error[512];

int fail(int status, const char *fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

static int ok() {
  g_last_error[0] = 0;
  return IREE_MI355X_OK;
}

// Validate-only calls (an executable-library dispatch whose state carries a
// workspace query): every check and the plan run, nothing is allocated or
// launched, and the workspace the launch would need is written to the sink.
static thread_local size_t *g_dry_run = nullptr;

void set_dry_run(size_t *sink) { g_dry_run = sink; }

static bool dry_run(int64_t workspace_needed) {
  if (!g_dry_run)
    return false;
  *g_dry_run = workspace_needed > 0 ? (size_t)workspace_needed : 0;
  return true;
}

static bool aligned(const void *p, size_t a) {
  return ((uintptr_t)p % a) == 0;
}

static const int64_t kMaxExtent = (int64_t)1 << 31;

// The split-K partials and arrival counters of a call come from the
// caller's workspace: the library allocates no device memory. A call whose
// plan needs `need` bytes and has none, or fewer, is refused before
// anything is launched.
int require_workspace(const char *who, size_t need, const void *workspace,
                      size_t workspace_bytes) {
  if (need == 0 || (workspace && workspace_bytes >= need))
    return IREE_MI355X_OK;
  if (!workspace)
    return fail(IREE_MI355X_WORKSPACE_TOO_SMALL,
                "%s: the plan needs a workspace of %zu bytes (size it with "
                "the workspace query) and none was passed",
                who, need);
  return fail(IREE_MI355X_WORKSPACE_TOO_SMALL, "%s: workspace %zu < %zu", who,
              workspace_bytes, need);
}

// Scratch of the allocation-free entry point: device memory of the
// library's own code object, one copy per GPU that runs the library, held
// until the process ends. It is zero from load, and every kernel that uses
// it leaves its arrival counters at zero again, so no call clears it;
// calls that overlap on one GPU race on it.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device: the host-side name is only a stand-in, not a device address.
static std::mutex g_scratch_mutex;
static std::vector<void *> g_scratch;

static int scratch_address(void **out) {
  *out = nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return fail(IREE_MI355X_NO_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if ((int)g_scratch.size() <= dev)
    g_scratch.resize(dev + 1, nullptr);
  if (!g_scratch[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return fail(IREE_MI355X_LAUNCH_FAILED,
                  "scratch: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(e));
    }
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return IREE_MI355X_OK;
}

static int launch_status(hipError_t e, const char *what) {
  if (e != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// Launch the planned MFMA configuration, with its split-K workspace (the
// caller's if given and large enough, else the library's).
static int launch_mfma(MatmulArgs &args, const iree_mi355x_matmul_plan_t &plan,
                       void *workspace, size_t workspace_bytes,
                       const char *who) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  args.splits = plan.splits > 1 ? plan.splits : 1;
  args.k_split = plan.k_split;
  args.sk_steps = plan.stream_k_steps;
  args.sk_workgroups = plan.stream_k_steps > 0 ? (int)plan.workgroups : 0;
  args.workspace = nullptr;
  if (plan.workspace_bytes > 0) {
    const int st = require_workspace(who, (size_t)plan.workspace_bytes,
                                     workspace, workspace_bytes);
    if (st != IREE_MI355X_OK)
      return st;
    args.workspace = workspace;
  }
  return launch_status(cfgs[plan.config_index].launch(args),
                       cfgs[plan.config_index].name);
}

// Shared shape / stride checks for the three matmul entry points.
static int check_matmul(const char *who, const void *a, const void *b,
                        void *c, int64_t m, int64_t n, int64_t k, int64_t lda,
                        int64_t ldb, int64_t ldc, uint32_t flags,
                        uint32_t allowed_flags, size_t a_elem, size_t b_elem,
                        size_t c_elem) {
  if (flags & ~allowed_flags)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x", who,
                flags & ~allowed_flags);
  if (m < 0 || n < 0 || k < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative extent", who);
  if (m >= kMaxExtent || n >= kMaxExtent || k >= kMaxExtent)
    return fail(IREE_MI355X_UNSUPPORTED, "%s: extent >= 2^31", who);
  if (m == 0 || n == 0)
    return IREE_MI355X_OK;
  const bool bt = flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  const bool at = flags & IREE_MI355X_MATMUL_A_TRANSPOSED;
  if (!c || (k > 0 && (!a || !b)))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null pointer", who);
  if (lda < (at ? m : k) || ldb < (bt ? k : n) || ldc < n || lda < 0 ||
      ldb < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: leading dimension smaller than the row", who);
  if ((a && !aligned(a, a_elem)) || (b && !aligned(b, b_elem)) ||
      !aligned(c, c_elem))
    return fail(IREE_MI355X_MISALIGNED,
                "%s: pointer not aligned to its element size", who);
  return IREE_MI355X_OK;
}

// One row of a transposed A ([K, 1] with unit pitch) is the contiguous row
// [1, K]: the same matmul without the transpose, which lets M = 1 decode
// stream as a GEMV. Returns the flags the call runs with.
uint32_t m1_row_layout(int64_t m, int64_t lda, uint32_t flags) {
  if ((flags & IREE_MI355X_MATMUL_A_TRANSPOSED) && m == 1 && lda == 1)
    return flags & ~IREE_MI355X_MATMUL_A_TRANSPOSED;
  return flags;
}

}  // namespace ihp

using namespace ihp;

extern "C" {

const char *iree_mi355x_last_error(void) { return g_last_error; }

const char *iree_mi355x_version(void) { return "iree-mi355x 0.1 gfx950"; }

int iree_mi355x_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess)
    return 0;
  return n;
}

size_t iree_mi355x_matmul_workspace_bytes(int64_t m, int64_t n, int64_t k,
                                          uint32_t flags) {
  if (m <= 0 || n <= 0 || k <= 0)
    return 0;
  // The largest workspace any f16, int8 or W8A16 plan of this shape uses (plans
  // assume 16-byte aligned operands, the case that can pick split-K), over
  // both layouts a call may take: one row of a transposed A with unit pitch
  // runs as the untransposed row (see m1_row_layout).
  size_t most = 0;
  const int32_t forms[4][3] = {
      {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16},
      {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F32},
      {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_F16},
      {IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I32}};
  for (int layout = 0; layout < 2; ++layout) {
    const uint32_t lf =
        layout == 0 ? flags : m1_row_layout(m, 1, flags);
    if (layout == 1 && lf == flags)
      break;
    for (int f = 0; f < 4; ++f) {
      iree_mi355x_matmul_desc_t d;
      iree_mi355x_matmul_desc_init(&d, forms[f][0], forms[f][1], forms[f][2],
                                   m, n, k, lf & ~IREE_MI355X_MATMUL_OUT_F32);
      d.has_scale = f == 2;
      if (f == 1)
        d.flags |= IREE_MI355X_MATMUL_OUT_F32;
      iree_mi355x_matmul_plan_t p;
      if (iree_mi355x_plan_matmul(&d, &p) == IREE_MI355X_OK &&
          (size_t)p.workspace_bytes > most)
        most = (size_t)p.workspace_bytes;
    }
  }
  return most;
}

}  // extern "C"

namespace ihp {

// f16 matmul of `args` (batch and epilogue included): plan, workspace,
// launch. Shapes and pointers are validated by the caller.
static int matmul_f16_run(const char *who, MatmulArgs &args, uint32_t flags,
                          void *workspace, size_t workspace_bytes) {
  const bool out_f32 = flags & IREE_MI355X_MATMUL_OUT_F32;
  const uint32_t run_flags = m1_row_layout(args.m, args.lda, flags);
  if (run_flags != flags) {
    args.lda = args.k;
    flags = run_flags;
  }
  args.a_transposed = (flags & IREE_MI355X_MATMUL_A_TRANSPOSED) ? 1 : 0;
  iree_mi355x_matmul_desc_t desc;
  iree_mi355x_matmul_desc_init(&desc, IREE_MI355X_ELEM_F16,
                               IREE_MI355X_ELEM_F16,
                               out_f32 ? IREE_MI355X_ELEM_F32
                                       : IREE_MI355X_ELEM_F16,
                               args.m, args.n, args.k, flags);
  desc.a_aligned16 = fast_operand(args.a, args.lda * 2, args.sa * 2);
  desc.b_aligned16 = fast_operand(args.b, args.ldb * 2, args.sb * 2);
  desc.batch = args.batch;
  iree_mi355x_matmul_plan_t plan;
  if (iree_mi355x_plan_matmul(&desc, &plan) != IREE_MI355X_OK)
    return fail(IREE_MI355X_UNSUPPORTED, "%s: no plan", who);
  if (dry_run(plan.workspace_bytes))
    return ok();
  int st;
  switch (plan.family) {
    case IREE_MI355X_FAMILY_GEMV:
      if ((st = require_workspace(who, (size_t)plan.workspace_bytes,
                                  workspace, workspace_bytes)) !=
          IREE_MI355X_OK)
        return st;
      return launch_status(launch_gemv(args, 2, nullptr, out_f32, workspace),
                           "gemv_f16");
    case IREE_MI355X_FAMILY_MFMA:
      return launch_mfma(args, plan, workspace, workspace_bytes, who);
    default:
      return launch_status(
          launch_general(args, out_f32 ? kGeneralF16F32 : kGeneralF16F16,
                         nullptr),
          "gemm_general_f16");
  }
}

}  // namespace ihp

extern "C" {

int iree_mi355x_matmul_f16(const void *a, const void *b, void *c, int64_t m,
                           int64_t n, int64_t k, int64_t lda, int64_t ldb,
                           int64_t ldc, uint32_t flags, void *workspace,
                           size_t workspace_bytes, void *stream) {
  const bool out_f32 = flags & IREE_MI355X_MATMUL_OUT_F32;
  int st = check_matmul("matmul_f16", a, b, c, m, n, k, lda, ldb, ldc, flags,
                        IREE_MI355X_MATMUL_B_TRANSPOSED |
                            IREE_MI355X_MATMUL_ACCUMULATE |
                            IREE_MI355X_MATMUL_OUT_F32 |
                            IREE_MI355X_MATMUL_A_TRANSPOSED,
                        2, 2, out_f32 ? 4 : 2);
  if (st != IREE_MI355X_OK || m == 0 || n == 0)
    return st == IREE_MI355X_OK ? ok() : st;
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc,
                  (flags & IREE_MI355X_MATMUL_B_TRANSPOSED) ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream};
  return matmul_f16_run("matmul_f16", args, flags, workspace,
                        workspace_bytes);
}

int iree_mi355x_matmul_f16_no_alloc(const void *a, const void *b, void *c,
                                    int64_t m, int64_t n, int64_t k,
                                    int64_t lda, int64_t ldb, int64_t ldc,
                                    uint32_t flags, void *stream) {
  const char *who = "matmul_f16_no_alloc";
  const bool out_f32 = flags & IREE_MI355X_MATMUL_OUT_F32;
  int st = check_matmul(who, a, b, c, m, n, k, lda, ldb, ldc, flags,
                        IREE_MI355X_MATMUL_B_TRANSPOSED |
                            IREE_MI355X_MATMUL_ACCUMULATE |
                            IREE_MI355X_MATMUL_OUT_F32 |
                            IREE_MI355X_MATMUL_A_TRANSPOSED,
                        2, 2, out_f32 ? 4 : 2);
  if (st != IREE_MI355X_OK || m == 0 || n == 0)
    return st == IREE_MI355X_OK ? ok() : st;
  void *ws = nullptr;
  if ((st = scratch_address(&ws)) != IREE_MI355X_OK)
    return st;
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc,
                  (flags & IREE_MI355X_MATMUL_B_TRANSPOSED) ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream};
  // A plan needing more than the scratch holds is refused by the workspace
  // check (WORKSPACE_TOO_SMALL) before anything is launched.
  return matmul_f16_run(who, args, flags, ws, kNoAllocScratchBytes);
}

int iree_mi355x_batch_matmul_f16(const void *a, const void *b, void *c,
                                 int64_t batch, int64_t m, int64_t n,
                                 int64_t k, int64_t lda, int64_t ldb,
                                 int64_t ldc, int64_t stride_a,
                                 int64_t stride_b, int64_t stride_c,
                                 uint32_t flags,
                                 const iree_mi355x_epilogue_t *epilogue,
                                 void *workspace, size_t workspace_bytes,
                                 void *stream) {
  const char *who = "batch_matmul_f16";
  const bool out_f32 = flags & IREE_MI355X_MATMUL_OUT_F32;
  if (batch < 0 || stride_a < 0 || stride_b < 0 || stride_c < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative batch or stride",
                who);
  if (batch > 65535)
    return fail(IREE_MI355X_UNSUPPORTED, "%s: batch %lld > 65535", who,
                (long long)batch);
  int st = check_matmul(who, a, b, c, m, n, k, lda, ldb, ldc, flags,
                        IREE_MI355X_MATMUL_B_TRANSPOSED |
                            IREE_MI355X_MATMUL_ACCUMULATE |
                            IREE_MI355X_MATMUL_OUT_F32 |
                            IREE_MI355X_MATMUL_A_TRANSPOSED,
                        2, 2, out_f32 ? 4 : 2);
  if (st != IREE_MI355X_OK || m == 0 || n == 0 || batch == 0)
    return st == IREE_MI355X_OK ? ok() : st;
  if (batch > 1 && stride_c < (m - 1) * ldc + n)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: stride_c %lld overlaps the outputs of consecutive "
                "batches", who, (long long)stride_c);
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc,
                  (flags & IREE_MI355X_MATMUL_B_TRANSPOSED) ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream};
  args.batch = batch;
  args.sa = stride_a;
  args.sb = stride_b;
  args.sc = stride_c;
  if (epilogue) {
    if (epilogue->activation > IREE_MI355X_ACT_SILU)
      return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: unknown activation %u",
                  who, epilogue->activation);
    if ((epilogue->bias && !aligned(epilogue->bias, 2)) ||
        (epilogue->multiplier && !aligned(epilogue->multiplier, 2)))
      return fail(IREE_MI355X_MISALIGNED, "%s: epilogue operand misaligned",
                  who);
    if (epilogue->multiplier && (epilogue->ld_multiplier < n ||
                                 epilogue->batch_stride_multiplier < 0))
      return fail(IREE_MI355X_INVALID_ARGUMENT,
                  "%s: multiplier pitch smaller than the row", who);
    args.bias = epilogue->bias;
    args.mul = epilogue->multiplier;
    args.ld_mul = epilogue->ld_multiplier;
    args.s_mul = epilogue->batch_stride_multiplier;
    args.act = (int)epilogue->activation;
  }
  return matmul_f16_run(who, args, flags, workspace, workspace_bytes);
}

size_t iree_mi355x_batch_matmul_workspace_bytes(int64_t batch, int64_t m,
                                                int64_t n, int64_t k,
                                                uint32_t flags) {
  if (batch <= 0 || m <= 0 || n <= 0 || k <= 0)
    return 0;
  size_t most = 0;
  for (int layout = 0; layout < 2; ++layout) {
    const uint32_t lf = layout == 0 ? flags : m1_row_layout(m, 1, flags);
    if (layout == 1 && lf == flags)
      break;
    iree_mi355x_matmul_desc_t d;
    iree_mi355x_matmul_desc_init(
        &d, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16,
        (lf & IREE_MI355X_MATMUL_OUT_F32) ? IREE_MI355X_ELEM_F32
                                          : IREE_MI355X_ELEM_F16,
        m, n, k, lf);
    d.batch = batch;
    iree_mi355x_matmul_plan_t p;
    if (iree_mi355x_plan_matmul(&d, &p) == IREE_MI355X_OK &&
        (size_t)p.workspace_bytes > most)
      most = (size_t)p.workspace_bytes;
  }
  return most;
}

int iree_mi355x_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c,
                          int64_t m, int64_t n, int64_t k, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t flags,
                          void *workspace, size_t workspace_bytes,
                          void *stream) {
  int st = check_matmul("matmul_i8", a, b, c, m, n, k, lda, ldb, ldc, flags,
                        IREE_MI355X_MATMUL_B_TRANSPOSED |
                            IREE_MI355X_MATMUL_ACCUMULATE,
                        1, 1, 4);
  if (st != IREE_MI355X_OK || m == 0 || n == 0)
    return st == IREE_MI355X_OK ? ok() : st;
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc,
                  (flags & IREE_MI355X_MATMUL_B_TRANSPOSED) ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream};
  iree_mi355x_matmul_desc_t desc;
  iree_mi355x_matmul_desc_init(&desc, IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I8,
                               IREE_MI355X_ELEM_I32, m, n, k, flags);
  desc.a_aligned16 = fast_operand(a, lda);
  desc.b_aligned16 = fast_operand(b, ldb);
  iree_mi355x_matmul_plan_t plan;
  if (iree_mi355x_plan_matmul(&desc, &plan) != IREE_MI355X_OK)
    return fail(IREE_MI355X_UNSUPPORTED, "matmul_i8: no plan");
  if (dry_run(plan.workspace_bytes))
    return ok();
  if (plan.family == IREE_MI355X_FAMILY_MFMA)
    return launch_mfma(args, plan, workspace, workspace_bytes, "matmul_i8");
  return launch_status(launch_general(args, kGeneralI8I32, nullptr),
                       "gemm_general_i8");
}

int iree_mi355x_w8a16_matmul(const void *x, const int8_t *w, const void *scale,
                             void *y, int64_t m, int64_t n, int64_t k,
                             int64_t ldx, int64_t ldw, int64_t ldy,
                             uint32_t flags, void *workspace,
                             size_t workspace_bytes, void *stream) {
  int st = check_matmul("w8a16_matmul", x, w, y, m, n, k, ldx, ldw, ldy, flags,
                        IREE_MI355X_MATMUL_B_TRANSPOSED, 2, 1, 2);
  if (st != IREE_MI355X_OK || m == 0 || n == 0)
    return st == IREE_MI355X_OK ? ok() : st;
  if (!scale)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "w8a16_matmul: null scale");
  if (!aligned(scale, 2))
    return fail(IREE_MI355X_MISALIGNED, "w8a16_matmul: scale misaligned");
  MatmulArgs args{x, w, y, m, n, k, ldx, ldw, ldy,
                  (flags & IREE_MI355X_MATMUL_B_TRANSPOSED) ? 1 : 0, 0, stream,
                  scale};
  iree_mi355x_matmul_desc_t desc;
  iree_mi355x_matmul_desc_init(&desc, IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_I8,
                               IREE_MI355X_ELEM_F16, m, n, k, flags);
  desc.a_aligned16 = fast_operand(x, ldx * 2);
  desc.b_aligned16 = fast_operand(w, ldw);
  desc.has_scale = 1;
  iree_mi355x_matmul_plan_t plan;
  if (iree_mi355x_plan_matmul(&desc, &plan) != IREE_MI355X_OK)
    return fail(IREE_MI355X_UNSUPPORTED, "w8a16_matmul: no plan");
  if (dry_run(plan.workspace_bytes))
    return ok();
  if (plan.family == IREE_MI355X_FAMILY_GEMV) {
    if ((st = require_workspace("w8a16_matmul", (size_t)plan.workspace_bytes,
                                workspace, workspace_bytes)) != IREE_MI355X_OK)
      return st;
    return launch_status(launch_gemv(args, 1, scale, 0, workspace),
                         "gemv_w8a16");
  }
  if (plan.family == IREE_MI355X_FAMILY_MFMA)
    return launch_mfma(args, plan, workspace, workspace_bytes, "w8a16_matmul");
  return launch_status(launch_general(args, kGeneralW8A16, scale),
                       "gemm_general_w8a16");
}

int iree_mi355x_attention_f16_strided(
    const void *q, const void *k, const void *v, void *o, int64_t batch,
    int64_t heads, int64_t kv_heads, int64_t seq_q, int64_t seq_kv,
    int64_t head_dim, float scale, uint32_t flags,
    const iree_mi355x_attention_strides_t *strides, void *stream) {
  const char *who = "attention_f16";
  if (flags & ~IREE_MI355X_ATTENTION_CAUSAL)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x",
                who, flags);
  if (batch < 0 || heads < 0 || kv_heads < 0 || seq_q < 0 || seq_kv < 0 ||
      head_dim < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative extent", who);
  if (!std::isfinite(scale))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: scale not finite", who);
  if (!strides)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null strides", who);
  if (batch == 0 || heads == 0 || seq_q == 0)
    return ok();
  if (kv_heads == 0 || heads % kv_heads != 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: %lld query heads are not a multiple of %lld KV heads",
                who, (long long)heads, (long long)kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return fail(IREE_MI355X_UNSUPPORTED,
                "%s: head_dim %lld (64 or 128 supported)", who,
                (long long)head_dim);
  if (!q || !o || (seq_kv > 0 && (!k || !v)))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null pointer", who);
  const int64_t *st[4] = {strides->q, strides->k, strides->v, strides->o};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      if (st[t][i] < 0)
        return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative stride", who);
  if (strides->o[2] < head_dim)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: o row stride %lld overlaps its rows", who,
                (long long)strides->o[2]);
  // The copies and stores move 16-byte chunks of rows: every base, and
  // every stride (in bytes), must keep them aligned.
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      if (st[t][i] % 8 != 0)
        return fail(IREE_MI355X_MISALIGNED,
                    "%s: strides must be multiples of 8 elements", who);
  if (!aligned(q, 16) || !aligned(o, 16) || (k && !aligned(k, 16)) ||
      (v && !aligned(v, 16)))
    return fail(IREE_MI355X_MISALIGNED,
                "%s: q/k/v/o must be 16-byte aligned", who);
  const int64_t q_blocks = (seq_q + 127) / 128;
  if (batch >= kMaxExtent || heads >= kMaxExtent || seq_q >= kMaxExtent ||
      seq_kv >= kMaxExtent || batch * heads * q_blocks >= kMaxExtent)
    return fail(IREE_MI355X_UNSUPPORTED, "%s: problem too large", who);
  // Q, K and V rows are copied with a 32-bit byte offset from their head's
  // first row.
  const int64_t row_bytes = head_dim * 2;
  auto head_span = [&](const int64_t *s, int64_t rows) -> int64_t {
    if (rows <= 1)
      return rows == 1 ? row_bytes : 0;
    const uint64_t pitch = (uint64_t)s[2] * 2;
    if (s[2] > (int64_t)UINT32_MAX ||
        (pitch > 0 &&
         (uint64_t)(rows - 1) > (UINT32_MAX - (uint64_t)row_bytes) / pitch))
      return INT64_MAX;
    return (int64_t)((uint64_t)(rows - 1) * pitch) + row_bytes;
  };
  if (head_span(strides->q, seq_q) > (int64_t)UINT32_MAX ||
      head_span(strides->k, seq_kv) > (int64_t)UINT32_MAX ||
      head_span(strides->v, seq_kv) > (int64_t)UINT32_MAX)
    return fail(IREE_MI355X_UNSUPPORTED,
                "%s: a head's rows span more than 4 GiB", who);
  if (dry_run(0))
    return ok();
  AttentionLayout layout;
  for (int i = 0; i < 3; ++i) {
    layout.q[i] = strides->q[i];
    layout.k[i] = strides->k[i];
    layout.v[i] = strides->v[i];
    layout.o[i] = strides->o[i];
    layout.m[i] = 0;
  }
  layout.heads = (int)heads;
  layout.group = (int)(heads / kv_heads);
  layout.seq_q = (int)seq_q;
  layout.seq_kv = (int)seq_kv;
  return launch_status(
      launch_attention(q, k, v, o, batch, layout, head_dim, scale,
                       (flags & IREE_MI355X_ATTENTION_CAUSAL) ? 1 : 0, stream),
      "attention_fwd");
}

int iree_mi355x_attention(const iree_mi355x_attention_t *a, void *stream) {
  const char *who = "attention";
  if (!a)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null arguments", who);
  if (a->flags & ~(IREE_MI355X_ATTENTION_CAUSAL | IREE_MI355X_ATTENTION_OUT_F32 |
                   IREE_MI355X_ATTENTION_MASK))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x",
                who, a->flags);
  if (!(a->flags & IREE_MI355X_ATTENTION_MASK) != !a->mask)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: the MASK flag and the mask pointer disagree", who);
  if (a->batch < 0 || a->heads < 0 || a->kv_heads < 0 || a->seq_q < 0 ||
      a->seq_kv < 0 || a->head_dim < 0 || a->head_dim_v < 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative extent", who);
  if (!std::isfinite(a->scale))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: scale not finite", who);
  if (a->batch == 0 || a->heads == 0 || a->seq_q == 0 || a->head_dim_v == 0)
    return ok();
  if (a->kv_heads == 0 || a->heads % a->kv_heads != 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: %lld query heads are not a multiple of %lld KV heads",
                who, (long long)a->heads, (long long)a->kv_heads);
  if (a->head_dim < 1 || a->head_dim > 256 || a->head_dim_v > 256)
    return fail(IREE_MI355X_UNSUPPORTED,
                "%s: head dims %lld / %lld (1..256 supported)", who,
                (long long)a->head_dim, (long long)a->head_dim_v);
  // Grid (query blocks, heads, batch) and 32-bit row and key counters.
  if (a->batch > 65535 || a->heads > 65535 || a->seq_q >= kMaxExtent / 2 ||
      a->seq_kv >= kMaxExtent / 2)
    return fail(IREE_MI355X_UNSUPPORTED, "%s: problem too large", who);
  if (!a->q || !a->o || (a->seq_kv > 0 && (!a->k || !a->v)))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: null pointer", who);
  const iree_mi355x_attention_strides_t &st = a->strides;
  // Mask strides are read only with a mask.
  const int64_t *all[5] = {st.q, st.k, st.v, st.o, a->mask_strides};
  for (int t = 0; t < (a->mask ? 5 : 4); ++t)
    for (int i = 0; i < (t == 4 ? 4 : 3); ++i)
      if (all[t][i] < 0)
        return fail(IREE_MI355X_INVALID_ARGUMENT, "%s: negative stride", who);
  if (st.o[2] < a->head_dim_v)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "%s: o row stride %lld overlaps its rows", who,
                (long long)st.o[2]);
  const bool out_f32 = a->flags & IREE_MI355X_ATTENTION_OUT_F32;
  if (!aligned(a->q, 2) || !aligned(a->o, out_f32 ? 4 : 2) ||
      (a->k && !aligned(a->k, 2)) || (a->v && !aligned(a->v, 2)) ||
      (a->mask && !aligned(a->mask, 2)))
    return fail(IREE_MI355X_MISALIGNED,
                "%s: operands must be aligned to their element size", who);
  const bool causal = a->flags & IREE_MI355X_ATTENTION_CAUSAL;

  // The MFMA kernel: equal head dims that are multiples of 16 up to 128,
  // 16-byte rows and strides, each head's rows within 4 GiB (32-bit copy
  // offsets), and a grid of pairs of 128-row query blocks; a mask with
  // contiguous keys read 4 keys (8 bytes) at a time: strides and base
  // 8-byte aligned, seq_kv a multiple of 4.
  bool fast = a->head_dim == a->head_dim_v && a->head_dim % 16 == 0 &&
              a->head_dim <= 128 &&
              aligned(a->q, 16) && aligned(a->o, 16) &&
              (!a->k || aligned(a->k, 16)) && (!a->v || aligned(a->v, 16));
  if (fast && a->mask)
    fast = a->mask_strides[3] == 1 && a->mask_strides[0] % 4 == 0 &&
           a->mask_strides[1] % 4 == 0 && a->mask_strides[2] % 4 == 0 &&
           aligned(a->mask, 8) && a->seq_kv % 4 == 0;
  for (int t = 0; t < 4 && fast; ++t)
    for (int i = 0; i < 3; ++i)
      if (all[t][i] % 8 != 0)
        fast = false;
  const int64_t row_bytes = a->head_dim * 2;
  auto head_span = [&](const int64_t *s, int64_t rows) -> int64_t {
    if (rows <= 1)
      return rows == 1 ? row_bytes : 0;
    const uint64_t pitch = (uint64_t)s[2] * 2;
    if (s[2] > (int64_t)UINT32_MAX ||
        (pitch > 0 &&
         (uint64_t)(rows - 1) > (UINT32_MAX - (uint64_t)row_bytes) / pitch))
      return INT64_MAX;
    return (int64_t)((uint64_t)(rows - 1) * pitch) + row_bytes;
  };
  if (fast && (head_span(st.q, a->seq_q) > (int64_t)UINT32_MAX ||
               head_span(st.k, a->seq_kv) > (int64_t)UINT32_MAX ||
               head_span(st.v, a->seq_kv) > (int64_t)UINT32_MAX ||
               a->batch * a->heads * ((a->seq_q + 127) / 128) >= kMaxExtent))
    fast = false;
  if (fast && !a->mask && !out_f32 &&
      (a->head_dim == 64 || a->head_dim == 128))
    return iree_mi355x_attention_f16_strided(
        a->q, a->k, a->v, a->o, a->batch, a->heads, a->kv_heads, a->seq_q,
        a->seq_kv, a->head_dim, a->scale, a->flags & IREE_MI355X_ATTENTION_CAUSAL,
        &a->strides, stream);
  if (dry_run(0))
    return ok();
  if (fast) {
    AttentionLayout layout;
    for (int i = 0; i < 3; ++i) {
      layout.q[i] = st.q[i];
      layout.k[i] = st.k[i];
      layout.v[i] = st.v[i];
      layout.o[i] = st.o[i];
      layout.m[i] = a->mask_strides[i];
    }
    layout.heads = (int)a->heads;
    layout.group = (int)(a->heads / a->kv_heads);
    layout.seq_q = (int)a->seq_q;
    layout.seq_kv = (int)a->seq_kv;
    return launch_status(
        launch_attention(a->q, a->k, a->v, a->o, a->batch, layout,
                         a->head_dim, a->scale, causal ? 1 : 0, stream,
                         a->mask, out_f32 ? 1 : 0),
        a->mask ? "attention_fwd_mask" : "attention_fwd");
  }
  AttentionGeneralLayout g;
  for (int i = 0; i < 3; ++i) {
    g.q[i] = st.q[i];
    g.k[i] = st.k[i];
    g.v[i] = st.v[i];
    g.o[i] = st.o[i];
  }
  for (int i = 0; i < 4; ++i)
    g.mask[i] = a->mask_strides[i];
  g.heads = (int)a->heads;
  g.group = (int)(a->heads / a->kv_heads);
  g.seq_q = (int)a->seq_q;
  g.seq_kv = (int)a->seq_kv;
  g.dqk = (int)a->head_dim;
  g.dv = (int)a->head_dim_v;
  g.scale = a->scale;
  g.causal = causal ? 1 : 0;
  g.vec_k = a->head_dim % 8 == 0 && st.k[0] % 8 == 0 && st.k[1] % 8 == 0 &&
            st.k[2] % 8 == 0 && aligned(a->k, 16);
  g.vec_v = a->head_dim_v % 8 == 0 && st.v[0] % 8 == 0 &&
            st.v[1] % 8 == 0 && st.v[2] % 8 == 0 && aligned(a->v, 16);
  return launch_status(
      launch_attention_general(a->q, a->k, a->v, a->o, a->mask, a->batch, g,
                               out_f32 ? 1 : 0, stream),
      "attention_general");
}


int iree_mi355x_attention_f16(const void *q, const void *k, const void *v,
                              void *o, int64_t batch, int64_t heads,
                              int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                              float scale, uint32_t flags, void *stream) {
  // Contiguous [B, H, S, D] operands, one KV head per query head.
  if (heads >= kMaxExtent || seq_q >= kMaxExtent || seq_kv >= kMaxExtent ||
      head_dim >= kMaxExtent)
    return fail(IREE_MI355X_UNSUPPORTED, "attention_f16: problem too large");
  iree_mi355x_attention_strides_t s;
  const int64_t qs[3] = {heads * seq_q * head_dim, seq_q * head_dim, head_dim};
  const int64_t ks[3] = {heads * seq_kv * head_dim, seq_kv * head_dim,
                         head_dim};
  for (int i = 0; i < 3; ++i) {
    s.q[i] = s.o[i] = qs[i];
    s.k[i] = s.v[i] = ks[i];
  }
  return iree_mi355x_attention_f16_strided(q, k, v, o, batch, heads, heads,
                                           seq_q, seq_kv, head_dim, scale,
                                           flags, &s, stream);
}

}  // extern "C"
