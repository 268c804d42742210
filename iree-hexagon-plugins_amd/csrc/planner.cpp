// Dispatch classification and gfx950 macro-tile planning (host only).
// See include/iree_mi355x_planner.h for the reference functions each entry
// point replaces.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <tuple>

#include "../../include/iree_mi355x_kernels.h"
#include "../../include/iree_mi355x_planner.h"
#include "kernels_internal.h"

namespace ihp {

int fail(int status, const char *fmt, ...);

namespace {

constexpr int64_t kDefaultLdsBudget = 160 * 1024;
constexpr int32_t kDefaultCus = 256;

// Measured choices (bench.py --tune writes the candidates' timings; the
// winners are recorded here). Keyed by element types, exact shape and flags.
struct TunedEntry {
  int32_t a_elem, c_elem;
  int64_t m, n, k;
  uint32_t flags;
  const char *config;
};
// Measured on MI355X with random inputs (bench.py --tune): the 4-wave
// 256x256 tile wins for int8 (the 8-wave one draws more power for the same
// work), the 8-wave one for f16.
const TunedEntry kTuned[] = {
    {IREE_MI355X_ELEM_I8, IREE_MI355X_ELEM_I32, 4096, 4096, 4096,
     IREE_MI355X_MATMUL_B_TRANSPOSED, "i8_tn_256x256x128_w2x2_s2"},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F16, 4096, 4096, 4096,
     IREE_MI355X_MATMUL_B_TRANSPOSED, "f16_tn_256x256x64_w2x4_s2"},
    {IREE_MI355X_ELEM_F16, IREE_MI355X_ELEM_F32, 4096, 4096, 4096,
     IREE_MI355X_MATMUL_B_TRANSPOSED, "f16f32_tn_256x256x64_w2x4_s2"},
    {0, 0, 0, 0, 0, 0, nullptr},  // sentinel
};

int elem_bytes(int32_t e) {
  switch (e) {
    case IREE_MI355X_ELEM_I8:
      return 1;
    case IREE_MI355X_ELEM_F16:
      return 2;
    default:
      return 4;
  }
}

bool types_supported(const iree_mi355x_matmul_desc_t &d) {
  const bool f16 = d.a_elem == IREE_MI355X_ELEM_F16 &&
                   d.b_elem == IREE_MI355X_ELEM_F16 &&
                   (d.c_elem == IREE_MI355X_ELEM_F16 ||
                    d.c_elem == IREE_MI355X_ELEM_F32) &&
                   !d.has_scale;
  const bool i8 = d.a_elem == IREE_MI355X_ELEM_I8 &&
                  d.b_elem == IREE_MI355X_ELEM_I8 &&
                  d.c_elem == IREE_MI355X_ELEM_I32 && !d.has_scale;
  const bool w8a16 = d.a_elem == IREE_MI355X_ELEM_F16 &&
                     d.b_elem == IREE_MI355X_ELEM_I8 &&
                     d.c_elem == IREE_MI355X_ELEM_F16 && d.has_scale;
  return f16 || i8 || w8a16;
}

bool gemv_eligible(const iree_mi355x_matmul_desc_t &d) {
  if (d.m < 1 || d.m > kGemvMaxRows || d.k < 1 ||
      (d.flags & IREE_MI355X_MATMUL_B_TRANSPOSED) || !d.b_aligned16)
    return false;
  const int cols = 16 / elem_bytes(d.b_elem);
  if (d.n % cols != 0)
    return false;
  // int8 weights only in the W8A16 form; f16 with f16 or f32 output.
  if (d.b_elem == IREE_MI355X_ELEM_I8)
    return d.has_scale;
  return true;
}

// The B form a dispatch needs, or -1 if no fast kernel computes it.
int wanted_b_mode(const iree_mi355x_matmul_desc_t &d) {
  const bool bt = d.flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  if (d.has_scale)
    return (!bt && d.a_elem == IREE_MI355X_ELEM_F16 &&
            d.b_elem == IREE_MI355X_ELEM_I8 &&
            d.c_elem == IREE_MI355X_ELEM_F16 &&
            !(d.flags & IREE_MI355X_MATMUL_ACCUMULATE))
               ? kBW8
               : -1;
  if (d.a_elem != d.b_elem)
    return -1;
  if (bt)
    return kBTN;
  return d.a_elem == IREE_MI355X_ELEM_F16 ? kBNN16 : -1;
}

// Fast-kernel candidates that tile the shape exactly.
bool fast_fits(const iree_mi355x_matmul_desc_t &d, const FastConfig &c) {
  if (!d.a_aligned16 || !d.b_aligned16 || d.k <= 0)
    return false;
  if (c.b_mode != wanted_b_mode(d))
    return false;
  const int want_elem = d.a_elem == IREE_MI355X_ELEM_I8 ? kElemI8 : kElemF16;
  if (c.elem != want_elem)
    return false;
  if (want_elem == kElemF16 && c.out_f32 != (d.c_elem == IREE_MI355X_ELEM_F32))
    return false;
  return d.m % c.bm == 0 && d.n % c.bn == 0 && d.k % c.bk == 0;
}

}  // namespace
}  // namespace ihp

using namespace ihp;

extern "C" {

void iree_mi355x_matmul_desc_init(iree_mi355x_matmul_desc_t *desc,
                                  int32_t a_elem, int32_t b_elem,
                                  int32_t c_elem, int64_t m, int64_t n,
                                  int64_t k, uint32_t flags) {
  memset(desc, 0, sizeof(*desc));
  desc->a_elem = a_elem;
  desc->b_elem = b_elem;
  desc->c_elem = c_elem;
  desc->m = m;
  desc->n = n;
  desc->k = k;
  desc->flags = flags;
  desc->a_aligned16 = 1;
  desc->b_aligned16 = 1;
  desc->lds_budget_bytes = kDefaultLdsBudget;
  desc->num_cus = kDefaultCus;
}

int32_t iree_mi355x_classify_matmul(const iree_mi355x_matmul_desc_t *d) {
  if (!d || !types_supported(*d) || d->m < 0 || d->n < 0 || d->k < 0)
    return IREE_MI355X_FAMILY_NONE;
  if (gemv_eligible(*d))
    return IREE_MI355X_FAMILY_GEMV;
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  for (int i = 0; i < count; ++i)
    if (fast_fits(*d, cfgs[i]) && cfgs[i].lds_bytes <= d->lds_budget_bytes)
      return IREE_MI355X_FAMILY_MFMA;
  return IREE_MI355X_FAMILY_GENERAL;
}

int iree_mi355x_plan_matmul(const iree_mi355x_matmul_desc_t *d,
                            iree_mi355x_matmul_plan_t *plan) {
  if (!d || !plan)
    return IREE_MI355X_INVALID_ARGUMENT;
  memset(plan, 0, sizeof(*plan));
  plan->config_index = -1;
  const int32_t family = iree_mi355x_classify_matmul(d);
  plan->family = family;
  if (family == IREE_MI355X_FAMILY_NONE)
    return IREE_MI355X_UNSUPPORTED;
  const int64_t budget =
      d->lds_budget_bytes > 0 ? d->lds_budget_bytes : kDefaultLdsBudget;
  const int64_t cus = d->num_cus > 0 ? d->num_cus : kDefaultCus;

  if (family == IREE_MI355X_FAMILY_GEMV) {
    const int wb = elem_bytes(d->b_elem);
    GemvPlan g = gemv_plan(d->m, d->n, d->k, wb);
    snprintf(plan->config_name, sizeof(plan->config_name), "gemv_%s_r%lld",
             wb == 1 ? "w8a16" : "f16", (long long)d->m);
    plan->tile_m = d->m;
    plan->tile_n = g.cols_per_wg;
    plan->tile_k = g.k_chunk;
    plan->workgroups = g.col_blocks * g.splits;
    plan->threads = 256;
    plan->splits = g.splits;
    plan->workspace_bytes = (int64_t)gemv_workspace_bytes(d->m, d->n, d->k, wb);
    plan->traffic_bytes = d->n * d->k * wb + d->m * d->k * 2;
    return IREE_MI355X_OK;
  }

  if (family == IREE_MI355X_FAMILY_MFMA) {
    int count = 0;
    const FastConfig *cfgs = fast_configs(&count);
    int best = -1;
    // A measured entry wins when it fits.
    for (const TunedEntry &t : kTuned) {
      if (!t.config || t.a_elem != d->a_elem || t.c_elem != d->c_elem || t.m != d->m ||
          t.n != d->n || t.k != d->k || t.flags != d->flags)
        continue;
      for (int i = 0; i < count; ++i)
        if (strcmp(cfgs[i].name, t.config) == 0 && fast_fits(*d, cfgs[i]) &&
            cfgs[i].lds_bytes <= budget) {
          best = i;
          plan->from_tuned_table = 1;
        }
    }
    // Otherwise rank: (over budget, per-CU critical work, traffic, tiles, -N).
    std::tuple<int, int64_t, int64_t, int64_t, int64_t> best_rank;
    const int64_t ab = elem_bytes(d->a_elem), bb = elem_bytes(d->b_elem);
    if (best < 0) {
      for (int i = 0; i < count; ++i) {
        const FastConfig &c = cfgs[i];
        if (!fast_fits(*d, c) || c.lds_bytes > budget)
          continue;
        const int64_t tiles = (d->m / c.bm) * (d->n / c.bn);
        const int64_t critical = ((tiles + cus - 1) / cus) * c.bm * c.bn;
        const int64_t traffic = ab * d->m * d->k * (d->n / c.bn) +
                                bb * d->n * d->k * (d->m / c.bm);
        auto rank = std::make_tuple(0, critical, traffic, tiles,
                                    -(int64_t)c.bn);
        if (best < 0 || rank < best_rank) {
          best = i;
          best_rank = rank;
        }
      }
    }
    if (best < 0)
      return IREE_MI355X_UNSUPPORTED;
    const FastConfig &c = cfgs[best];
    plan->config_index = best;
    snprintf(plan->config_name, sizeof(plan->config_name), "%s", c.name);
    plan->tile_m = c.bm;
    plan->tile_n = c.bn;
    plan->tile_k = c.bk;
    plan->lds_bytes = c.lds_bytes;
    plan->workgroups = (d->m / c.bm) * (d->n / c.bn);
    plan->threads = c.threads;
    plan->traffic_bytes = ab * d->m * d->k * (d->n / c.bn) +
                          bb * d->n * d->k * (d->m / c.bm);
    return IREE_MI355X_OK;
  }

  // General kernel: 64x64 tiles, 256 threads, 10 KiB LDS.
  snprintf(plan->config_name, sizeof(plan->config_name), "general_64x64");
  plan->tile_m = 64;
  plan->tile_n = 64;
  plan->tile_k = 64 / (d->a_elem == IREE_MI355X_ELEM_I8 &&
                               d->b_elem == IREE_MI355X_ELEM_I8
                           ? 1
                           : 2);
  plan->lds_bytes = 2 * 64 * 80;
  plan->workgroups = ((d->m + 63) / 64) * ((d->n + 63) / 64);
  plan->threads = 256;
  const int64_t ab = elem_bytes(d->a_elem), bb = elem_bytes(d->b_elem);
  plan->traffic_bytes = ab * d->m * d->k * ((d->n + 63) / 64) +
                        bb * d->n * d->k * ((d->m + 63) / 64);
  return IREE_MI355X_OK;
}

int iree_mi355x_mfma_config_count(void) {
  int count = 0;
  fast_configs(&count);
  return count;
}

int iree_mi355x_mfma_config_info(int index, const char **name,
                                 int32_t *b_form, int32_t *a_elem,
                                 int32_t *c_elem, int64_t *tile_m,
                                 int64_t *tile_n, int64_t *tile_k,
                                 int64_t *lds_bytes, int32_t *threads) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  if (index < 0 || index >= count)
    return IREE_MI355X_INVALID_ARGUMENT;
  const FastConfig &c = cfgs[index];
  if (name)
    *name = c.name;
  if (b_form)
    *b_form = c.b_mode;
  if (a_elem)
    *a_elem = c.elem == kElemI8 ? IREE_MI355X_ELEM_I8 : IREE_MI355X_ELEM_F16;
  if (c_elem)
    *c_elem = c.elem == kElemI8 ? IREE_MI355X_ELEM_I32
                                : (c.out_f32 ? IREE_MI355X_ELEM_F32
                                             : IREE_MI355X_ELEM_F16);
  if (tile_m)
    *tile_m = c.bm;
  if (tile_n)
    *tile_n = c.bn;
  if (tile_k)
    *tile_k = c.bk;
  if (lds_bytes)
    *lds_bytes = c.lds_bytes;
  if (threads)
    *threads = c.threads;
  return IREE_MI355X_OK;
}

int iree_mi355x_matmul_mfma_config(int index, const void *a, const void *b,
                                   const void *scale, void *c, int64_t m,
                                   int64_t n, int64_t k, int64_t lda,
                                   int64_t ldb, int64_t ldc, uint32_t flags,
                                   void *stream) {
  int count = 0;
  const FastConfig *cfgs = fast_configs(&count);
  if (index < 0 || index >= count)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: bad index %d",
                index);
  const FastConfig &cfg = cfgs[index];
  const int32_t ae = cfg.elem == kElemI8 ? IREE_MI355X_ELEM_I8
                                         : IREE_MI355X_ELEM_F16;
  const int32_t be = cfg.b_mode == kBW8 ? IREE_MI355X_ELEM_I8 : ae;
  const int32_t ce = cfg.elem == kElemI8
                         ? IREE_MI355X_ELEM_I32
                         : (cfg.out_f32 ? IREE_MI355X_ELEM_F32
                                        : IREE_MI355X_ELEM_F16);
  iree_mi355x_matmul_desc_t d;
  iree_mi355x_matmul_desc_init(&d, ae, be, ce, m, n, k, flags);
  d.has_scale = cfg.b_mode == kBW8;
  const int64_t aeb = elem_bytes(ae), beb = elem_bytes(be);
  d.a_aligned16 = a && ((uintptr_t)a % 16 == 0) && (lda * aeb) % 16 == 0;
  d.b_aligned16 = b && ((uintptr_t)b % 16 == 0) && (ldb * beb) % 16 == 0;
  const bool bt = flags & IREE_MI355X_MATMUL_B_TRANSPOSED;
  if (flags & ~(IREE_MI355X_MATMUL_B_TRANSPOSED | IREE_MI355X_MATMUL_ACCUMULATE |
                IREE_MI355X_MATMUL_OUT_F32))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: unknown flags");
  if (!c || (uintptr_t)c % elem_bytes(ce) != 0 || lda < k ||
      ldb < (bt ? k : n) || ldc < n || m >= ((int64_t)1 << 31) ||
      n >= ((int64_t)1 << 31) || k >= ((int64_t)1 << 31) ||
      (d.has_scale && (!scale || (uintptr_t)scale % 2 != 0)))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "mfma_config: bad arguments");
  if (!fast_fits(d, cfg))
    return fail(IREE_MI355X_UNSUPPORTED,
                "mfma_config %s: shape or layout does not fit", cfg.name);
  MatmulArgs args{a, b, c, m, n, k, lda, ldb, ldc, bt ? 1 : 0,
                  (flags & IREE_MI355X_MATMUL_ACCUMULATE) ? 1 : 0, stream,
                  scale};
  hipError_t e = cfg.launch(args);
  if (e != hipSuccess)
    return fail(IREE_MI355X_LAUNCH_FAILED, "%s: %s", cfg.name,
                hipGetErrorString(e));
  return IREE_MI355X_OK;
}

}  // extern "C"
