// Dispatch matcher (include/iree_mi355x_matcher.h): which library export
// computes a linalg op or a dispatch region, decided from the op's loops,
// indexing maps, element types and body. Host-only.
//
// Contraction analysis follows the reference's rules:
//  * loop roles as linalg::inferContractionDims assigns them, restricted to
//    one M, N and K loop and at most one batch loop
//    (ContractionStrategy.cpp:27-53, analyzeSupportedContraction);
//  * the output keeps M before N (isHmxLowerableMatmul, :152-168; a
//    transposed output is rejected, specialize_hmx_contractions.mlir
//    @transposed_output_is_kept);
//  * a generic's body must be the multiply-accumulate of its two inputs,
//    possibly through extensions (the f16 -> f32 mixed-precision body the
//    specialization keeps, HexagonSpecializeHmxContractions.cpp:32-35);
//  * element types: f16 inputs into f16 or f32 (hasHmxElementTypes,
//    :138-150), plus the int8 and W8A16 forms this library adds.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <utility>

#include "../../include/iree_mi355x_kernels.h"
#include "../../include/iree_mi355x_matcher.h"

namespace {

constexpr int kMaxOps = IREE_MI355X_LINALG_MAX_OPERANDS;
constexpr int kMaxBody = IREE_MI355X_LINALG_MAX_BODY;
constexpr int kMaxLoops = IREE_MI355X_LINALG_MAX_LOOPS;
constexpr uint32_t kArg = 1000;  // expression leaf: a block argument

typedef iree_mi355x_linalg_op_t Op;
typedef iree_mi355x_match_t Match;

void reject(Match *out, const char *fmt, ...) {
  out->taken = 0;
  out->export_name[0] = 0;
  out->init_fill = 0;
  out->init_value = 0.0;
  va_list args;
  va_start(args, fmt);
  vsnprintf(out->reason, sizeof(out->reason), fmt, args);
  va_end(args);
}

void accept(Match *out, const char *export_name, uint32_t flags) {
  out->taken = 1;
  snprintf(out->export_name, sizeof(out->export_name), "%s", export_name);
  out->flags = flags;
  out->reason[0] = 0;
}

void clear(Match *out) {
  memset(out, 0, sizeof(*out));
  out->batch_loop = out->m_loop = out->n_loop = out->k_loop = -1;
  out->head_loop = out->head_dim_loop = -1;
  out->root = -1;
  out->scale = 1.0f;
}

int operands(const Op &op) { return (int)(op.num_inputs + op.num_outputs); }

// ------------------------------------------------------------------ body --

// Expression tree of one body value.
struct Expr {
  uint32_t op;  // IREE_MI355X_BODY_* or kArg
  int32_t type;
  int arg;       // kArg: block argument
  double value;  // CONST value, INDEX loop, CMP predicate
  const Expr *a[3];
};

struct Body {
  Expr nodes[kMaxOps + kMaxBody];
  const Expr *yields[kMaxOps];
  int num_yields = 0;

  // Builds the trees; false if the body is malformed.
  bool build(const Op &op) {
    const int nargs = operands(op);
    for (int i = 0; i < nargs; ++i)
      nodes[i] = Expr{kArg, op.elem_type[i], i, 0.0, {nullptr, nullptr, nullptr}};
    int defined = nargs;
    num_yields = 0;
    if (op.num_body_ops > (uint32_t)kMaxBody)
      return false;
    for (uint32_t b = 0; b < op.num_body_ops; ++b) {
      const iree_mi355x_body_op_t &bo = op.body[b];
      if (bo.opcode == IREE_MI355X_BODY_YIELD) {
        for (int j = 0; j < 3 && bo.operands[j] >= 0; ++j) {
          if (bo.operands[j] >= defined || num_yields >= kMaxOps)
            return false;
          yields[num_yields++] = &nodes[bo.operands[j]];
        }
        return b + 1 == op.num_body_ops;  // the yield ends the body
      }
      Expr &e = nodes[defined];
      e = Expr{bo.opcode, bo.type, -1, bo.constant, {nullptr, nullptr, nullptr}};
      for (int j = 0; j < 3; ++j) {
        if (bo.operands[j] < 0)
          continue;
        if (bo.operands[j] >= defined)
          return false;
        e.a[j] = &nodes[bo.operands[j]];
      }
      ++defined;
    }
    return false;  // no yield
  }
};

bool is_ext(const Expr *e) {
  return e->op == IREE_MI355X_BODY_EXTF || e->op == IREE_MI355X_BODY_EXTSI;
}

const Expr *strip_ext(const Expr *e) {
  while (e && is_ext(e))
    e = e->a[0];
  return e;
}

bool is_arg(const Expr *e, int arg) {
  e = strip_ext(e);
  return e && e->op == kArg && e->arg == arg;
}

bool is_const(const Expr *e, double *value) {
  e = strip_ext(e);
  if (!e || e->op != IREE_MI355X_BODY_CONST)
    return false;
  if (value)
    *value = e->value;
  return true;
}

// A binary op `code` with operands (x, y) in either order.
bool binary(const Expr *e, uint32_t code, const Expr **x, const Expr **y) {
  if (!e || e->op != code || !e->a[0] || !e->a[1])
    return false;
  *x = e->a[0];
  *y = e->a[1];
  return true;
}

// One factor of a contraction product: the block argument it reads, and
// the zero point subtracted from it (arith.subi of a constant), if any.
struct Factor {
  int arg = -1;
  bool converted = false;  // through sitofp (int8 weights in a float body)
  double zero_point = 0.0;
  bool zero_point_known = true;
};

bool factor_of(const Expr *e, Factor *f) {
  e = strip_ext(e);
  if (!e)
    return false;
  const Expr *x, *y;
  if (binary(e, IREE_MI355X_BODY_SUBI, &x, &y)) {
    double zp;
    if (!is_const(y, &zp)) {
      f->zero_point_known = false;
      return false;
    }
    f->zero_point = zp;
    e = strip_ext(x);
  }
  if (e && e->op == IREE_MI355X_BODY_SITOFP) {
    f->converted = true;
    e = strip_ext(e->a[0]);
  }
  if (!e || e->op != kArg)
    return false;
  f->arg = e->arg;
  return true;
}

// Flattens a product tree (MULF / MULI) into at most 3 factors.
bool product_factors(const Expr *e, uint32_t mul, Factor *f, int *count) {
  e = strip_ext(e);
  const Expr *x, *y;
  if (binary(e, mul, &x, &y))
    return product_factors(x, mul, f, count) &&
           product_factors(y, mul, f, count);
  if (*count >= 3)
    return false;
  return factor_of(e, &f[(*count)++]);
}

// The body of a contraction of inputs `a`, `b` (and an optional per-column
// `scale` input, the W8A16 dequantization) into output argument `out`:
// out + a * b [* scale], up to extensions and operand order. Returns false
// with `why` set otherwise. Zero points found are returned.
bool contraction_body(const Op &op, int a, int b, int scale, int out,
                      bool integer, double zp[2], char *why, size_t n) {
  Body body;
  if (!body.build(op) || body.num_yields != 1) {
    snprintf(why, n, "body is not one yielded value");
    return false;
  }
  const uint32_t add = integer ? IREE_MI355X_BODY_ADDI : IREE_MI355X_BODY_ADDF;
  const uint32_t mul = integer ? IREE_MI355X_BODY_MULI : IREE_MI355X_BODY_MULF;
  const Expr *x, *y;
  if (!binary(strip_ext(body.yields[0]), add, &x, &y)) {
    snprintf(why, n, "body does not yield an accumulation (%s)",
             integer ? "arith.addi" : "arith.addf");
    return false;
  }
  if (!is_arg(x, out))
    std::swap(x, y);
  if (!is_arg(x, out)) {
    snprintf(why, n, "body does not add into the output");
    return false;
  }
  Factor f[3];
  int count = 0;
  if (!product_factors(y, mul, f, &count) || count != (scale >= 0 ? 3 : 2)) {
    snprintf(why, n, "body is not a product of the inputs%s",
             scale >= 0 ? " and the scale" : "");
    return false;
  }
  bool seen_a = false, seen_b = false, seen_s = false;
  zp[0] = zp[1] = 0.0;
  for (int i = 0; i < count; ++i) {
    if (!f[i].zero_point_known) {
      snprintf(why, n, "zero point is not a constant");
      return false;
    }
    if (f[i].arg == a && !seen_a) {
      seen_a = true;
      zp[0] = f[i].zero_point;
    } else if (f[i].arg == b && !seen_b) {
      seen_b = true;
      zp[1] = f[i].zero_point;
    } else if (f[i].arg == scale && scale >= 0 && !seen_s) {
      seen_s = true;
    } else {
      snprintf(why, n, "body multiplies an operand other than the inputs");
      return false;
    }
  }
  return true;
}

// -------------------------------------------------------------- contraction --

struct Roles {
  int batch = -1, m = -1, n = -1, k = -1;
  bool a_t = false, b_t = false;
};

bool map_valid(const Op &op, int i) {
  if (op.map_rank[i] > (uint32_t)kMaxLoops)
    return false;
  for (uint32_t r = 0; r < op.map_rank[i]; ++r)
    if (op.map[i][r] != IREE_MI355X_MAP_ZERO &&
        (op.map[i][r] < 0 || op.map[i][r] >= (int)op.num_loops))
      return false;
  return true;
}

bool map_has(const Op &op, int i, int loop) {
  for (uint32_t r = 0; r < op.map_rank[i]; ++r)
    if (op.map[i][r] == loop)
      return true;
  return false;
}

bool map_is(const Op &op, int i, int l0, int l1, int l2 = -2) {
  const int want = l2 == -2 ? 2 : 3;
  if ((int)op.map_rank[i] != want)
    return false;
  return op.map[i][0] == l0 && op.map[i][1] == l1 &&
         (want == 2 || op.map[i][2] == l2);
}

bool projected_permutation(const Op &op, int i) {
  for (uint32_t r = 0; r < op.map_rank[i]; ++r) {
    if (op.map[i][r] < 0)
      return false;
    for (uint32_t s = 0; s < r; ++s)
      if (op.map[i][s] == op.map[i][r])
        return false;
  }
  return true;
}

bool is_reduction(const Op &op, int loop) {
  return (op.reduction_loops >> loop) & 1u;
}

// Loop roles of A . B -> C (operands a, b, c), and the operand layouts.
bool contraction_roles(const Op &op, int a, int b, int c, Roles *r,
                       char *why, size_t n) {
  for (int i : {a, b, c})
    if (!projected_permutation(op, i)) {
      snprintf(why, n, "operand %d map is not a projected permutation", i);
      return false;
    }
  int nb = 0, nm = 0, nn = 0, nk = 0;
  for (int d = 0; d < (int)op.num_loops; ++d) {
    const bool ia = map_has(op, a, d), ib = map_has(op, b, d),
               ic = map_has(op, c, d), red = is_reduction(op, d);
    if (red && ia && ib && !ic) {
      r->k = d;
      ++nk;
    } else if (!red && ia && ib && ic) {
      r->batch = d;
      ++nb;
    } else if (!red && ia && !ib && ic) {
      r->m = d;
      ++nm;
    } else if (!red && !ia && ib && ic) {
      r->n = d;
      ++nn;
    } else {
      snprintf(why, n, "loop d%d has no matmul role", d);
      return false;
    }
  }
  if (nk != 1 || nm != 1 || nn != 1 || nb > 1) {
    snprintf(why, n,
             "not matmul-shaped: %d batch, %d M, %d N, %d K loops (one M, N "
             "and K and at most one batch are taken)",
             nb, nm, nn, nk);
    return false;
  }
  const int bt = r->batch;
  const bool has_b = bt >= 0;
  // Output: [batch,] M, N.
  const bool c_mn = has_b ? map_is(op, c, bt, r->m, r->n) : map_is(op, c, r->m, r->n);
  const bool c_nm = has_b ? map_is(op, c, bt, r->n, r->m) : map_is(op, c, r->n, r->m);
  if (c_nm) {
    snprintf(why, n, "transposed output (N before M)");
    return false;
  }
  if (!c_mn) {
    snprintf(why, n, "output map is not [batch,] M, N");
    return false;
  }
  if (has_b ? map_is(op, a, bt, r->m, r->k) : map_is(op, a, r->m, r->k)) {
    r->a_t = false;
  } else if (has_b ? map_is(op, a, bt, r->k, r->m) : map_is(op, a, r->k, r->m)) {
    r->a_t = true;
  } else {
    snprintf(why, n, "A map is not [batch,] M, K or [batch,] K, M");
    return false;
  }
  if (has_b ? map_is(op, b, bt, r->k, r->n) : map_is(op, b, r->k, r->n)) {
    r->b_t = false;
  } else if (has_b ? map_is(op, b, bt, r->n, r->k) : map_is(op, b, r->n, r->k)) {
    r->b_t = true;
  } else {
    snprintf(why, n, "B map is not [batch,] K, N or [batch,] N, K");
    return false;
  }
  return true;
}

const char *type_name(int t) {
  switch (t) {
    case IREE_MI355X_TYPE_F16: return "f16";
    case IREE_MI355X_TYPE_BF16: return "bf16";
    case IREE_MI355X_TYPE_F32: return "f32";
    case IREE_MI355X_TYPE_F64: return "f64";
    case IREE_MI355X_TYPE_I1: return "i1";
    case IREE_MI355X_TYPE_I8: return "i8";
    case IREE_MI355X_TYPE_I32: return "i32";
    case IREE_MI355X_TYPE_I64: return "i64";
    case IREE_MI355X_TYPE_INDEX: return "index";
  }
  return "none";
}

// Element types a contraction's operands carry once extension generics in
// front of it are looked through (region matching), else their own.
struct Types {
  int a, b, c;
};

struct Region {
  const Op *ops;
  int count;
};

// What a destination operand (a contraction's init, a reduction's start
// value) holds before the op runs. A linalg contraction computes
// init + A.B (examples/matmul/matmul.mlir; the HMX unpack adds every tile
// into the init, UK/hmx.c:328-357,426-450), so the init decides between an
// overwriting and an accumulating dispatch.
enum InitKind { kInitConstant, kInitArgument, kInitOther };
struct Init {
  InitKind kind = kInitOther;
  double value = 0.0;  // kInitConstant
  char why[96] = {0};  // kInitOther
};

// The init of operand `operand` of op `index` (of region `rg`, or of a lone
// op when rg is null): a region argument, a splat constant, a linalg.fill
// of a constant in the region, or something else.
Init init_of(const Region *rg, const Op &op, int index, int operand) {
  Init init;
  const int producer = op.producer[operand];
  if (producer == IREE_MI355X_FROM_ARGUMENT) {
    init.kind = kInitArgument;
    return init;
  }
  if (producer == IREE_MI355X_FROM_CONSTANT) {
    init.kind = kInitConstant;
    init.value = op.scalar[operand];
    return init;
  }
  if (!rg || producer < 0 || producer >= index) {
    snprintf(init.why, sizeof(init.why),
             "the init is produced by an op outside the description");
    return init;
  }
  const Op &p = rg->ops[producer];
  if (p.kind == IREE_MI355X_LINALG_FILL && p.num_inputs == 1) {
    if (p.producer[0] == IREE_MI355X_FROM_CONSTANT) {
      init.kind = kInitConstant;
      init.value = p.scalar[0];
      return init;
    }
    snprintf(init.why, sizeof(init.why),
             "the init is a fill of a value that is not a constant");
    return init;
  }
  snprintf(init.why, sizeof(init.why),
           "the init is produced by op %d, which is not a fill", producer);
  return init;
}

bool init_is(const Init &init, double value) {
  return init.kind == kInitConstant && init.value == value;
}

// Applies the output init to an accepted contraction: a zero init keeps the
// overwriting export; a region argument, or a fill of another constant,
// adds ACCUMULATE (C_out = C_init + A.B) where the export has that form
// (the constant is returned for the caller to fill first); anything else
// is not taken. `truncated`: the contraction accumulates in f32 and a
// truncation after it writes the result, so an init would have to be read
// in f32.
void apply_init(const Init &init, bool truncated, Match *out) {
  if (!out->taken)
    return;
  if (init_is(init, 0.0))
    return;
  if (init.kind == kInitOther) {
    reject(out, "%s", init.why);
    return;
  }
  const char *what = init.kind == kInitConstant ? "a nonzero fill"
                                                : "a region argument";
  if (truncated) {
    reject(out, "the init is %s, accumulated in f32 before a truncation: "
           "no kernel (the accumulating exports read the init in the "
           "output type)", what);
    return;
  }
  if (strcmp(out->export_name, "w8a16_matmul") == 0) {
    reject(out, "the init is %s, and w8a16_matmul has no accumulating form",
           what);
    return;
  }
  out->flags |= IREE_MI355X_MATMUL_ACCUMULATE;
  if (init.kind == kInitConstant) {
    out->init_fill = 1;
    out->init_value = init.value;
  }
}

// A (possibly batched) contraction with two inputs, optionally a per-column
// scale (W8A16), or linalg.quantized_matmul's zero points.
void match_contraction(const Op &op, uint32_t options, Types t, Match *out) {
  const bool generic = op.kind == IREE_MI355X_LINALG_GENERIC;
  if (op.num_outputs != 1) {
    reject(out, "contraction with %u outputs", op.num_outputs);
    return;
  }
  const int c = (int)op.num_inputs;
  int scale = -1;
  double zp[2] = {0.0, 0.0};
  bool zp_known = true;
  if (op.kind == IREE_MI355X_LINALG_QUANTIZED_MATMUL) {
    if (op.num_inputs != 4) {
      reject(out, "quantized_matmul needs A, B and two zero points");
      return;
    }
    for (int i = 0; i < 2; ++i) {
      if (op.producer[2 + i] != IREE_MI355X_FROM_CONSTANT)
        zp_known = false;
      else
        zp[i] = op.scalar[2 + i];
    }
  } else if (op.num_inputs == 3 && generic) {
    scale = 2;
  } else if (op.num_inputs != 2) {
    reject(out, "contraction with %u inputs", op.num_inputs);
    return;
  }
  Roles r;
  if (!contraction_roles(op, 0, 1, c, &r, out->reason, sizeof(out->reason))) {
    out->taken = 0;
    return;
  }
  out->batch_loop = r.batch;
  out->m_loop = r.m;
  out->n_loop = r.n;
  out->k_loop = r.k;
  if (scale >= 0 &&
      !((op.map_rank[scale] == 1 && op.map[scale][0] == r.n) ||
        (op.map_rank[scale] == 2 && op.map[scale][0] == IREE_MI355X_MAP_ZERO &&
         op.map[scale][1] == r.n))) {
    reject(out, "third input is not a per-column (N) scale");
    return;
  }
  const bool integer = t.a == IREE_MI355X_TYPE_I8 && t.b == IREE_MI355X_TYPE_I8;
  if (generic) {
    if (options & IREE_MI355X_MATCH_NAMED_ONLY) {
      reject(out,
             "matmul-like 'linalg.generic' is not lowered: only named "
             "linalg.matmul and linalg.batch_matmul with an MxN output are");
      return;
    }
    char why[120];
    if (!contraction_body(op, 0, 1, scale, c, integer, zp, why, sizeof(why))) {
      reject(out, "%s", why);
      return;
    }
  }
  if (!zp_known) {
    reject(out, "zero points are not constants");
    return;
  }
  if (zp[0] != 0.0 || zp[1] != 0.0) {
    reject(out, "nonzero zero point (%g, %g): only zero point 0 is taken",
           zp[0], zp[1]);
    return;
  }
  uint32_t flags = (r.b_t ? IREE_MI355X_MATMUL_B_TRANSPOSED : 0u) |
                   (r.a_t ? IREE_MI355X_MATMUL_A_TRANSPOSED : 0u);
  const bool batched = r.batch >= 0;
  if (scale >= 0) {
    if (!(t.a == IREE_MI355X_TYPE_F16 && t.b == IREE_MI355X_TYPE_I8 &&
          op.elem_type[2] == IREE_MI355X_TYPE_F16 && t.c == IREE_MI355X_TYPE_F16)) {
      reject(out, "dequantized contraction (%s, %s, scale %s) -> %s has no "
             "kernel (f16 x int8 with an f16 scale into f16 is taken)",
             type_name(t.a), type_name(t.b), type_name(op.elem_type[2]),
             type_name(t.c));
      return;
    }
    if (batched || r.a_t) {
      reject(out, "W8A16 with a batch loop or a transposed A has no kernel");
      return;
    }
    accept(out, "w8a16_matmul", flags);
    return;
  }
  if (t.a == IREE_MI355X_TYPE_F16 && t.b == IREE_MI355X_TYPE_F16 &&
      (t.c == IREE_MI355X_TYPE_F16 || t.c == IREE_MI355X_TYPE_F32)) {
    if (t.c == IREE_MI355X_TYPE_F32)
      flags |= IREE_MI355X_MATMUL_OUT_F32;
    accept(out, batched ? "batch_matmul_f16" : "matmul_f16", flags);
    return;
  }
  if (integer && t.c == IREE_MI355X_TYPE_I32) {
    if (batched || r.a_t) {
      reject(out, "int8 with a batch loop or a transposed A has no kernel");
      return;
    }
    accept(out, "matmul_i8", flags);
    return;
  }
  reject(out, "element types (%s, %s) -> %s have no kernel (f16 x f16 -> "
         "f16 / f32 and i8 x i8 -> i32 are taken)",
         type_name(t.a), type_name(t.b), type_name(t.c));
}

// iree_linalg_ext.attention: Q [.., M, K1], K [.., K2, K1], V [.., K2, N],
// a scale, an optional mask, O [.., M, N]; K1 and K2 are reductions. At
// most two batch loops (batch, head). Q, K, V are f16 and O f16 or f32
// (*flags gains OUT_F32); head dims K1 and N are 1..256.
bool attention_shape(const Op &op, Match *out, uint32_t *flags) {
  const int q = 0, k = 1, v = 2, o = (int)op.num_inputs;
  const uint32_t rank = op.map_rank[q];
  if (rank < 2 || op.map_rank[k] != rank || op.map_rank[v] != rank ||
      op.map_rank[o] != rank) {
    reject(out, "attention operands of different ranks");
    return false;
  }
  const int nb = (int)rank - 2;
  if (nb > 2) {
    reject(out, "attention with %d batch loops (batch and head are taken)",
           nb);
    return false;
  }
  for (int i = 0; i < nb; ++i) {
    const int l = op.map[q][i];
    if (l < 0 || is_reduction(op, l) || op.map[k][i] != l ||
        op.map[v][i] != l || op.map[o][i] != l) {
      reject(out, "attention batch loops are not the same outermost loops");
      return false;
    }
  }
  const int m = op.map[q][nb], k1 = op.map[q][nb + 1];
  const int k2 = op.map[k][nb], n = op.map[v][nb + 1];
  if (m < 0 || k1 < 0 || k2 < 0 || n < 0 || op.map[k][nb + 1] != k1 ||
      op.map[v][nb] != k2 || op.map[o][nb] != m || op.map[o][nb + 1] != n ||
      !is_reduction(op, k1) || !is_reduction(op, k2) || is_reduction(op, m) ||
      is_reduction(op, n)) {
    reject(out, "attention maps are not Q[.., M, K1] K[.., K2, K1] "
           "V[.., K2, N] O[.., M, N]");
    return false;
  }
  for (int i : {q, k, v})
    if (op.elem_type[i] != IREE_MI355X_TYPE_F16) {
      reject(out, "attention operand %d is %s (f16 is taken)", i,
             type_name(op.elem_type[i]));
      return false;
    }
  if (op.elem_type[o] == IREE_MI355X_TYPE_F32) {
    *flags |= IREE_MI355X_ATTENTION_OUT_F32;
  } else if (op.elem_type[o] != IREE_MI355X_TYPE_F16) {
    reject(out, "attention output is %s (f16 and f32 are taken)",
           type_name(op.elem_type[o]));
    return false;
  }
  const int64_t d1 = op.loop_extent[k1], dn = op.loop_extent[n];
  if (d1 < 1 || d1 > 256 || dn < 1 || dn > 256) {
    reject(out, "head dims %lld / %lld (static 1..256 are taken)",
           (long long)d1, (long long)dn);
    return false;
  }
  out->batch_loop = nb > 0 ? op.map[q][0] : -1;
  out->head_loop = nb > 1 ? op.map[q][1] : -1;
  out->m_loop = m;
  out->n_loop = n;
  out->k_loop = k2;
  out->head_dim_loop = k1;
  return true;
}

// An attention mask read from a region argument: f16 (added to the scaled
// scores), its map an ordered selection of (batch loops, M, K2), the
// dimensions it leaves out broadcast.
bool attention_mask(const Op &op, int index, const Match &shape, Match *out) {
  if (op.elem_type[index] != IREE_MI355X_TYPE_F16) {
    reject(out, "attention mask is %s (an f16 additive mask is taken)",
           type_name(op.elem_type[index]));
    return false;
  }
  const int order[4] = {shape.batch_loop, shape.head_loop, shape.m_loop,
                        shape.k_loop};
  int next = 0;
  for (uint32_t r = 0; r < op.map_rank[index]; ++r) {
    const int l = op.map[index][r];
    while (next < 4 && order[next] != l)
      ++next;
    if (l < 0 || next == 4) {
      reject(out, "attention mask map is not a selection of (batch, head, "
             "M, K2) in order");
      return false;
    }
    ++next;
  }
  return true;
}

bool valid_op(const Op &op) {
  if (op.num_loops > (uint32_t)kMaxLoops || op.num_inputs > (uint32_t)kMaxOps ||
      op.num_outputs > (uint32_t)kMaxOps || operands(op) > kMaxOps ||
      op.num_body_ops > (uint32_t)kMaxBody)
    return false;
  for (int i = 0; i < operands(op); ++i)
    if (!map_valid(op, i))
      return false;
  return true;
}

// `init` is what the op's output holds before it runs (contractions only);
// `truncated` as for apply_init.
int match_one(const Op &op, uint32_t options, Types t, const Init &init,
              bool truncated, Match *out) {
  switch (op.kind) {
    case IREE_MI355X_LINALG_MATMUL:
    case IREE_MI355X_LINALG_BATCH_MATMUL:
    case IREE_MI355X_LINALG_QUANTIZED_MATMUL:
      match_contraction(op, options, t, out);
      apply_init(init, truncated, out);
      return IREE_MI355X_OK;
    case IREE_MI355X_LINALG_GENERIC: {
      if (op.reduction_loops == 0) {
        reject(out, "elementwise generic (no reduction loop): not a "
               "contraction");
        return IREE_MI355X_OK;
      }
      match_contraction(op, options, t, out);
      apply_init(init, truncated, out);
      return IREE_MI355X_OK;
    }
    case IREE_MI355X_LINALG_ATTENTION: {
      if (op.num_inputs < 4 || op.num_inputs > 5 || op.num_outputs != 1) {
        reject(out, "attention needs Q, K, V, a scale [, a mask] and O");
        return IREE_MI355X_OK;
      }
      if (op.producer[3] != IREE_MI355X_FROM_CONSTANT) {
        reject(out, "attention scale is not a constant");
        return IREE_MI355X_OK;
      }
      uint32_t flags = 0;
      if (!attention_shape(op, out, &flags))
        return IREE_MI355X_OK;
      if (op.num_inputs == 5) {
        if (op.producer[4] != IREE_MI355X_FROM_ARGUMENT) {
          reject(out, "attention mask of unknown content (a region argument "
                 "or a causal mask generic is taken)");
          return IREE_MI355X_OK;
        }
        if (!attention_mask(op, 4, *out, out))
          return IREE_MI355X_OK;
        flags |= IREE_MI355X_ATTENTION_MASK;
      }
      out->scale = (float)op.scalar[3];
      accept(out, "attention_f16", flags);
      return IREE_MI355X_OK;
    }
    default:
      reject(out, "op kind %u is not a contraction", op.kind);
      return IREE_MI355X_OK;
  }
}

// --------------------------------------------------------------- regions --

bool identity_map(const Op &op, int i) {
  const int rank = (int)op.map_rank[i];
  if (rank != (int)op.num_loops)
    return false;
  for (int r = 0; r < rank; ++r)
    if (op.map[i][r] != r)
      return false;
  return true;
}

// An elementwise generic of one input (identity maps, no reduction) whose
// body yields f(input): the single body op code, with its constant operand
// when f is a multiplication by a constant.
bool unary_elementwise(const Op &op, uint32_t *code, double *constant) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.reduction_loops != 0 ||
      op.num_inputs != 1 || op.num_outputs != 1 || !identity_map(op, 0) ||
      !identity_map(op, 1))
    return false;
  Body body;
  if (!body.build(op) || body.num_yields != 1)
    return false;
  const Expr *e = body.yields[0];
  *constant = 1.0;
  const Expr *x, *y;
  if (binary(e, IREE_MI355X_BODY_MULF, &x, &y)) {
    double c;
    if (!is_arg(x, 0))
      std::swap(x, y);
    const Expr *cy = y;
    while (cy && (cy->op == IREE_MI355X_BODY_TRUNCF || is_ext(cy)))
      cy = cy->a[0];
    if (!is_arg(x, 0) || !cy || cy->op != IREE_MI355X_BODY_CONST)
      return false;
    c = cy->value;
    *code = IREE_MI355X_BODY_MULF;
    *constant = c;
    return true;
  }
  if ((e->op == IREE_MI355X_BODY_EXTF || e->op == IREE_MI355X_BODY_TRUNCF ||
       e->op == IREE_MI355X_BODY_EXP || e->op == IREE_MI355X_BODY_EXTSI) &&
      e->a[0] && e->a[0]->op == kArg && e->a[0]->arg == 0) {
    *code = e->op;
    return true;
  }
  return false;
}

// A transpose of the last two dimensions: one map the identity, the other
// the identity with its last two results swapped.
bool swaps_last_two(const Op &op) {
  if (op.num_outputs != 1 || op.map_rank[0] != op.num_loops ||
      op.map_rank[1] != op.num_loops || op.num_loops < 2)
    return false;
  const int last = (int)op.num_loops - 1;
  for (int i = 0; i < 2; ++i) {
    if (!identity_map(op, i))
      continue;
    const int o = 1 - i;
    for (int r = 0; r < last - 1; ++r)
      if (op.map[o][r] != r)
        return false;
    return op.map[o][last - 1] == last && op.map[o][last] == last - 1;
  }
  return false;
}

// Where an operand's values come from once elementwise extensions,
// multiplications by constants and transposes in front of it are looked
// through: a region argument (`arg` = true) or an op, the element type at
// the source, the constant factor gathered, and the permutation of the
// last two dimensions.
struct Source {
  bool arg = false;
  int op = -1;      // producing op (when !arg)
  int result = 0;
  int type = IREE_MI355X_TYPE_NONE;
  double factor = 1.0;
  bool transposed = false;
};

Source trace(const Region &rg, int op_index, int operand) {
  Source s;
  const Op *op = &rg.ops[op_index];
  int producer = op->producer[operand];
  int result = op->producer_result[operand];
  s.type = op->elem_type[operand];
  while (true) {
    if (producer == IREE_MI355X_FROM_ARGUMENT) {
      s.arg = true;
      return s;
    }
    if (producer < 0 || producer >= op_index) {
      s.op = -1;
      return s;
    }
    const Op &p = rg.ops[producer];
    uint32_t code;
    double c;
    if (p.kind == IREE_MI355X_LINALG_TRANSPOSE && p.num_inputs == 1 &&
        swaps_last_two(p)) {
      s.transposed = !s.transposed;
      s.type = p.elem_type[0];
      op_index = producer;
      result = p.producer_result[0];
      producer = p.producer[0];
      continue;
    }
    if (unary_elementwise(p, &code, &c) &&
        (code == IREE_MI355X_BODY_EXTF || code == IREE_MI355X_BODY_MULF ||
         code == IREE_MI355X_BODY_EXTSI)) {
      s.factor *= c;
      s.type = p.elem_type[0];
      op_index = producer;
      result = p.producer_result[0];
      producer = p.producer[0];
      continue;
    }
    s.op = producer;
    s.result = result;
    return s;
  }
}

// A row reduction over the last loop into [.., 1] or [..]: body yields
// code(input, output) for output 0 (more outputs, e.g. an argmax index,
// are allowed for MAXF).
bool row_reduction(const Op &op, uint32_t code) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.num_inputs != 1 ||
      op.num_outputs < 1 || op.num_loops < 1)
    return false;
  const int last = (int)op.num_loops - 1;
  if (op.reduction_loops != (1u << last) || !identity_map(op, 0))
    return false;
  const int o = 1;
  const uint32_t rank = op.map_rank[o];
  bool drops = rank == (uint32_t)last;
  bool zeroes = rank == (uint32_t)op.num_loops &&
                op.map[o][last] == IREE_MI355X_MAP_ZERO;
  for (int r = 0; r < last && (drops || zeroes); ++r)
    if (op.map[o][r] != r)
      drops = zeroes = false;
  if (!drops && !zeroes)
    return false;
  Body body;
  if (!body.build(op) || body.num_yields < 1)
    return false;
  const Expr *x, *y;
  if (!binary(body.yields[0], code, &x, &y))
    return false;
  return (is_arg(x, 0) && is_arg(y, 1)) || (is_arg(x, 1) && is_arg(y, 0));
}

// An elementwise generic of two inputs, the second broadcast along the last
// loop (a row vector), yielding code(in0, in1).
bool row_broadcast_binary(const Op &op, uint32_t code) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.reduction_loops != 0 ||
      op.num_inputs != 2 || op.num_outputs != 1 || !identity_map(op, 0) ||
      !identity_map(op, 2))
    return false;
  const int last = (int)op.num_loops - 1;
  const uint32_t rank = op.map_rank[1];
  bool ok = rank == (uint32_t)op.num_loops &&
            op.map[1][last] == IREE_MI355X_MAP_ZERO;
  if (!ok && rank == (uint32_t)last)
    ok = true;
  for (int r = 0; r < last && ok; ++r)
    if (op.map[1][r] != r)
      ok = false;
  if (!ok)
    return false;
  Body body;
  if (!body.build(op) || body.num_yields != 1)
    return false;
  const Expr *e = body.yields[0];
  return e->op == code && is_arg(e->a[0], 0) && is_arg(e->a[1], 1);
}

// The causal mask: an elementwise generic over the scores [.., M, K2]
// yielding select(index(K2) > index(M), -inf, s) (or cmpi sgt / ugt).
bool causal_mask(const Op &op) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.reduction_loops != 0 ||
      op.num_inputs != 1 || op.num_outputs != 1 || !identity_map(op, 0) ||
      op.num_loops < 2)
    return false;
  Body body;
  if (!body.build(op) || body.num_yields != 1)
    return false;
  const Expr *e = body.yields[0];
  if (e->op != IREE_MI355X_BODY_SELECT || !e->a[0] || !e->a[1] || !e->a[2])
    return false;
  double v;
  if (!is_const(e->a[1], &v) || !(std::isinf(v) && v < 0) ||
      !is_arg(e->a[2], 0))
    return false;
  const Expr *cmp = e->a[0];
  if (cmp->op != IREE_MI355X_BODY_CMPI ||
      (cmp->value != IREE_MI355X_PRED_GT && cmp->value != IREE_MI355X_PRED_UGT))
    return false;
  auto index_of = [](const Expr *x) -> int {
    while (x && x->op == IREE_MI355X_BODY_INDEX_CAST)
      x = x->a[0];
    return x && x->op == IREE_MI355X_BODY_INDEX ? (int)x->value : -1;
  };
  const int last = (int)op.num_loops - 1;
  return index_of(cmp->a[0]) == last && index_of(cmp->a[1]) == last - 1;
}

// The all-masked-row guard of the decomposed softmax: select(all(s ==
// -inf) over the row, 0, p). Returns the index of the op producing p.
int guard_input(const Region &rg, int index) {
  const Op &op = rg.ops[index];
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.reduction_loops != 0 ||
      op.num_inputs != 3 || op.num_outputs != 1 || !identity_map(op, 2) ||
      !identity_map(op, 3))
    return -1;
  Body body;
  if (!body.build(op) || body.num_yields != 1)
    return -1;
  const Expr *e = body.yields[0];
  if (e->op != IREE_MI355X_BODY_SELECT || !is_arg(e->a[0], 0) ||
      !is_arg(e->a[1], 1) || !is_arg(e->a[2], 2))
    return -1;
  if (op.producer[1] != IREE_MI355X_FROM_CONSTANT || op.scalar[1] != 0.0)
    return -1;
  // condition: a row AND-reduction of (x == -inf), starting from true
  const int cond = op.producer[0];
  if (cond < 0 || cond >= index ||
      !row_reduction(rg.ops[cond], IREE_MI355X_BODY_ANDI) ||
      !init_is(init_of(&rg, rg.ops[cond], cond, 1), 1.0))
    return -1;
  const int eq = rg.ops[cond].producer[0];
  if (eq < 0 || eq >= cond)
    return -1;
  const Op &cmp = rg.ops[eq];
  Body cb;
  if (cmp.kind != IREE_MI355X_LINALG_GENERIC || cmp.num_inputs != 1 ||
      !cb.build(cmp) || cb.num_yields != 1)
    return -1;
  const Expr *c = cb.yields[0];
  double v;
  if (c->op != IREE_MI355X_BODY_CMPF || c->value != IREE_MI355X_PRED_EQ ||
      !is_arg(c->a[0], 0) || !is_const(c->a[1], &v) ||
      !(std::isinf(v) && v < 0))
    return -1;
  return op.producer[2];
}

// A batch_matmul of the attention chain written as a linalg.generic must
// have the multiply-accumulate body, as a single contraction must.
bool chain_contraction_body(const Op &op) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC)
    return true;
  double zp[2];
  char why[120];
  return contraction_body(op, 0, 1, -1, 2, false, zp, why, sizeof(why));
}

// The decomposed attention of examples/attention_layer/attention_layer.mlir:
// S = (Q.a) . (K.b)^T [masked]; P = exp(S - rowmax S) / rowsum(...) [guarded];
// O = P . V [truncated to f16]. The two batch_matmuls start from zero
// fills, the row max from -inf and the row sum from 0
// (attention_layer.mlir:47,52,80,102).
bool match_attention_chain(const Region &rg, int root, uint32_t options,
                           Match *out) {
  int pv = root;
  bool truncated = false;
  {
    uint32_t code;
    double c;
    if (unary_elementwise(rg.ops[root], &code, &c) &&
        code == IREE_MI355X_BODY_TRUNCF) {
      pv = rg.ops[root].producer[0];
      truncated = true;
      if (pv < 0 || pv >= root)
        return false;
    }
  }
  const Op &bmm2 = rg.ops[pv];
  if (bmm2.kind != IREE_MI355X_LINALG_BATCH_MATMUL &&
      bmm2.kind != IREE_MI355X_LINALG_GENERIC)
    return false;
  if (bmm2.num_inputs != 2 || bmm2.num_outputs != 1)
    return false;
  Roles r2;
  char why[120];
  if (!contraction_roles(bmm2, 0, 1, 2, &r2, why, sizeof(why)) ||
      r2.a_t || r2.b_t || !chain_contraction_body(bmm2))
    return false;
  // V: an f16 region argument (through extensions)
  const Source v = trace(rg, pv, 1);
  if (!v.arg || v.type != IREE_MI355X_TYPE_F16 || v.factor != 1.0 ||
      v.transposed)
    return false;
  // P: [guard] divide(exp(sub(S, max)), sum)
  int p = bmm2.producer[0];
  if (p < 0 || p >= pv)
    return false;
  const int guarded = guard_input(rg, p);
  if (guarded >= 0)
    p = guarded;
  if (p < 0 || !row_broadcast_binary(rg.ops[p], IREE_MI355X_BODY_DIVF))
    return false;
  const int ex = rg.ops[p].producer[0], sum = rg.ops[p].producer[1];
  if (ex < 0 || sum < 0 || !row_reduction(rg.ops[sum], IREE_MI355X_BODY_ADDF) ||
      rg.ops[sum].producer[0] != ex)
    return false;
  const Init sum_init = init_of(&rg, rg.ops[sum], sum, 1);
  uint32_t code;
  double c;
  if (!unary_elementwise(rg.ops[ex], &code, &c) || code != IREE_MI355X_BODY_EXP)
    return false;
  const int sub = rg.ops[ex].producer[0];
  if (sub < 0 || !row_broadcast_binary(rg.ops[sub], IREE_MI355X_BODY_SUBF))
    return false;
  int s = rg.ops[sub].producer[0];
  const int mx = rg.ops[sub].producer[1];
  if (mx < 0 || !row_reduction(rg.ops[mx], IREE_MI355X_BODY_MAXF) ||
      rg.ops[mx].producer[0] != s)
    return false;
  const Init max_init = init_of(&rg, rg.ops[mx], mx, 1);
  // S: [causal mask] [scale] bmm1
  bool causal = false;
  double score_factor = 1.0;
  while (s >= 0) {
    if (causal_mask(rg.ops[s])) {
      if (causal)
        return false;
      causal = true;
      s = rg.ops[s].producer[0];
      continue;
    }
    if (unary_elementwise(rg.ops[s], &code, &c) && code == IREE_MI355X_BODY_MULF) {
      score_factor *= c;
      s = rg.ops[s].producer[0];
      continue;
    }
    break;
  }
  if (s < 0)
    return false;
  const Op &bmm1 = rg.ops[s];
  if ((bmm1.kind != IREE_MI355X_LINALG_BATCH_MATMUL &&
       bmm1.kind != IREE_MI355X_LINALG_GENERIC) ||
      bmm1.num_inputs != 2 || bmm1.num_outputs != 1)
    return false;
  Roles r1;
  if (!contraction_roles(bmm1, 0, 1, 2, &r1, why, sizeof(why)) || r1.a_t ||
      !chain_contraction_body(bmm1))
    return false;
  const Source q = trace(rg, s, 0), k = trace(rg, s, 1);
  if (!q.arg || !k.arg || q.transposed || q.type != IREE_MI355X_TYPE_F16 ||
      k.type != IREE_MI355X_TYPE_F16)
    return false;
  // K reaches bmm1 as [K1, K2]: through a transpose of K [K2, K1], or read
  // transposed by the map.
  if (k.transposed == r1.b_t)
    return false;
  // The chain is attention's; what follows decides whether the kernel
  // computes it.
  out->root = root;
  if ((options & IREE_MI355X_MATCH_NAMED_ONLY) &&
      (bmm1.kind == IREE_MI355X_LINALG_GENERIC ||
       bmm2.kind == IREE_MI355X_LINALG_GENERIC)) {
    reject(out, "matmul-like 'linalg.generic' in the attention chain is not "
           "lowered: only named batch_matmuls are");
    return true;
  }
  if (!init_is(init_of(&rg, bmm1, s, 2), 0.0) ||
      !init_is(init_of(&rg, bmm2, pv, 2), 0.0)) {
    reject(out, "an attention batch_matmul does not start from a zero fill");
    return true;
  }
  if (!init_is(sum_init, 0.0)) {
    reject(out, "the softmax row sum does not start from 0");
    return true;
  }
  if (max_init.kind != kInitConstant || !(max_init.value <= -3.4028234663852886e38)) {
    reject(out, "the softmax row max does not start from -inf");
    return true;
  }
  // The match reports bmm2's loops, so Q.K's head dim must be V's.
  const int64_t head = bmm1.loop_extent[r1.k];
  if (head != bmm2.loop_extent[r2.n] || head < 1 || head > 256) {
    reject(out, "attention head dims %lld / %lld (equal, static, 1..256 are "
           "taken)", (long long)head, (long long)bmm2.loop_extent[r2.n]);
    out->root = root;
    return true;
  }
  const int out_type = truncated ? rg.ops[root].elem_type[1]
                                 : bmm2.elem_type[2];
  if (out_type != IREE_MI355X_TYPE_F16 && out_type != IREE_MI355X_TYPE_F32) {
    reject(out, "attention output is %s (f16 and f32 are taken)",
           type_name(out_type));
    out->root = root;
    return true;
  }
  out->root = root;
  out->batch_loop = r2.batch;
  out->m_loop = r2.m;
  out->n_loop = r2.n;
  out->k_loop = r2.k;
  out->head_dim_loop = r2.n;
  out->scale = (float)(q.factor * k.factor * score_factor);
  accept(out, "attention_f16",
         (causal ? IREE_MI355X_ATTENTION_CAUSAL : 0u) |
             (out_type == IREE_MI355X_TYPE_F32 ? IREE_MI355X_ATTENTION_OUT_F32
                                               : 0u));
  return true;
}

// A dequantization generic feeding B of a matmul: w_f16 = sitofp(w_i8) *
// scale[n]. Returns the index of the int8 weight's producer chain start
// (the op itself) or -1.
bool dequant_generic(const Op &op) {
  if (op.kind != IREE_MI355X_LINALG_GENERIC || op.reduction_loops != 0 ||
      op.num_inputs != 2 || op.num_outputs != 1 || !identity_map(op, 0) ||
      !identity_map(op, 2) || op.num_loops != 2)
    return false;
  if (op.elem_type[0] != IREE_MI355X_TYPE_I8 ||
      op.elem_type[1] != IREE_MI355X_TYPE_F16 ||
      op.elem_type[2] != IREE_MI355X_TYPE_F16)
    return false;
  // scale per output column of W [K, N]: map (d1)
  if (!(op.map_rank[1] == 1 && op.map[1][0] == 1))
    return false;
  Body body;
  if (!body.build(op) || body.num_yields != 1)
    return false;
  Factor f[3];
  int count = 0;
  if (!product_factors(body.yields[0], IREE_MI355X_BODY_MULF, f, &count) ||
      count != 2)
    return false;
  const bool a = f[0].arg == 0 && f[0].converted && f[1].arg == 1;
  const bool b = f[1].arg == 0 && f[1].converted && f[0].arg == 1;
  return (a || b) && f[0].zero_point == 0.0 && f[1].zero_point == 0.0;
}

}  // namespace

extern "C" {

int iree_mi355x_match_linalg_op(const iree_mi355x_linalg_op_t *op,
                                uint32_t options, iree_mi355x_match_t *out) {
  if (!op || !out)
    return IREE_MI355X_INVALID_ARGUMENT;
  clear(out);
  if (!valid_op(*op)) {
    reject(out, "malformed op description");
    return IREE_MI355X_INVALID_ARGUMENT;
  }
  Body probe;
  if (op->num_body_ops > 0 && !probe.build(*op)) {
    reject(out, "malformed body");
    return IREE_MI355X_INVALID_ARGUMENT;
  }
  const int c = (int)op->num_inputs;
  Types t{op->elem_type[0], op->num_inputs > 1 ? op->elem_type[1] : 0,
          op->num_outputs > 0 ? op->elem_type[c] : 0};
  out->root = 0;
  return match_one(*op, options, t,
                   op->num_outputs > 0 ? init_of(nullptr, *op, 0, c) : Init(),
                   false, out);
}

int iree_mi355x_match_dispatch_region(const iree_mi355x_linalg_op_t *ops,
                                      uint32_t count, uint32_t options,
                                      iree_mi355x_match_t *out) {
  if (!ops || !out || count == 0 || count > 256)
    return IREE_MI355X_INVALID_ARGUMENT;
  clear(out);
  for (uint32_t i = 0; i < count; ++i) {
    Body probe;
    if (!valid_op(ops[i]) || (ops[i].num_body_ops > 0 && !probe.build(ops[i]))) {
      reject(out, "malformed op %u", i);
      return IREE_MI355X_INVALID_ARGUMENT;
    }
    for (int j = 0; j < operands(ops[i]); ++j)
      if (ops[i].producer[j] >= (int)i) {
        reject(out, "op %u reads op %d, which does not precede it", i,
               ops[i].producer[j]);
        return IREE_MI355X_INVALID_ARGUMENT;
      }
  }
  const Region rg{ops, (int)count};
  const int root = (int)count - 1;
  // The attention chain, or an attention op (possibly behind a causal mask).
  if (match_attention_chain(rg, root, options, out))
    return IREE_MI355X_OK;
  clear(out);
  const Op &r = ops[root];
  if (r.kind == IREE_MI355X_LINALG_ATTENTION) {
    if (r.num_inputs == 5 && r.producer[4] >= 0 &&
        causal_mask(ops[r.producer[4]])) {
      // An additive causal mask: the mask generic selects -inf above the
      // diagonal of a zero tensor.
      Op plain = r;
      plain.num_inputs = 4;
      for (int i = 4; i < kMaxOps - 1; ++i) {
        plain.elem_type[i] = r.elem_type[i + 1];
        plain.map_rank[i] = r.map_rank[i + 1];
        memcpy(plain.map[i], r.map[i + 1], sizeof(plain.map[i]));
        plain.producer[i] = r.producer[i + 1];
      }
      Types t{r.elem_type[0], r.elem_type[1], r.elem_type[5]};
      match_one(plain, options, t, Init(), false, out);
      if (out->taken)
        out->flags |= IREE_MI355X_ATTENTION_CAUSAL;
      out->root = root;
      return IREE_MI355X_OK;
    }
    Types t{r.elem_type[0], r.elem_type[1], r.elem_type[r.num_inputs]};
    match_one(r, options, t, Init(), false, out);
    out->root = root;
    return IREE_MI355X_OK;
  }
  // A contraction, with a truncation after an f32 accumulation, extension
  // generics before its inputs, or a dequantization generic before B.
  int mm = root;
  int out_type = -1;
  {
    uint32_t code;
    double cst;
    if (unary_elementwise(r, &code, &cst) && code == IREE_MI355X_BODY_TRUNCF &&
        r.producer[0] >= 0) {
      mm = r.producer[0];
      out_type = r.elem_type[1];
    }
  }
  const Op &m = ops[mm];
  const int c = (int)m.num_inputs;
  if (m.num_outputs != 1 || m.num_inputs < 2) {
    match_one(m, options,
              Types{m.elem_type[0], m.num_inputs > 1 ? m.elem_type[1] : 0,
                    m.num_outputs ? m.elem_type[c] : 0},
              m.num_outputs ? init_of(&rg, m, mm, c) : Init(), out_type >= 0,
              out);
    out->root = root;
    return IREE_MI355X_OK;
  }
  Source a = trace(rg, mm, 0), b = trace(rg, mm, 1);
  if (a.factor != 1.0 || b.factor != 1.0 || a.transposed || b.transposed) {
    reject(out, "matmul inputs scaled or transposed by other ops of the region");
    out->root = root;
    return IREE_MI355X_OK;
  }
  const bool accum_f32 = m.elem_type[c] == IREE_MI355X_TYPE_F32;
  Types t{a.type, b.type, out_type >= 0 ? out_type : m.elem_type[c]};
  if (out_type >= 0 && !accum_f32) {
    reject(out, "truncation after a %s contraction", type_name(m.elem_type[c]));
    out->root = root;
    return IREE_MI355X_OK;
  }
  const Init init = init_of(&rg, m, mm, c);
  // A matmul whose B is the output of a dequantization generic: W8A16.
  if (!b.arg && b.op >= 0 && dequant_generic(ops[b.op]) &&
      ops[b.op].producer[0] == IREE_MI355X_FROM_ARGUMENT) {
    Roles rr;
    char why[120];
    double zp[2];
    if (!a.arg) {
      // Only extensions fold into the kernel's A read; any other producer
      // (an activation, a second matmul) would be dropped.
      reject(out, "matmul input produced by an op the region cannot fold");
    } else if (m.kind != IREE_MI355X_LINALG_MATMUL &&
               m.kind != IREE_MI355X_LINALG_GENERIC) {
      reject(out, "dequantized B feeds a %s, not a matmul",
             m.kind == IREE_MI355X_LINALG_BATCH_MATMUL ? "batch_matmul"
                                                       : "non-contraction");
    } else if (m.kind == IREE_MI355X_LINALG_GENERIC &&
               (options & IREE_MI355X_MATCH_NAMED_ONLY)) {
      reject(out,
             "matmul-like 'linalg.generic' is not lowered: only named "
             "linalg.matmul and linalg.batch_matmul with an MxN output are");
    } else if (m.num_inputs != 2) {
      reject(out, "contraction with %u inputs", m.num_inputs);
    } else if (!contraction_roles(m, 0, 1, c, &rr, why, sizeof(why))) {
      reject(out, "%s", why);
    } else if (m.kind == IREE_MI355X_LINALG_GENERIC &&
               !contraction_body(m, 0, 1, -1, c, false, zp, why,
                                 sizeof(why))) {
      reject(out, "%s", why);
    } else if (rr.b_t || rr.a_t || rr.batch >= 0) {
      reject(out, "dequantized B must be [K, N] of a plain matmul");
    } else if (a.type != IREE_MI355X_TYPE_F16 ||
               (t.c != IREE_MI355X_TYPE_F16)) {
      reject(out, "dequantized matmul (%s, int8) -> %s has no kernel",
             type_name(a.type), type_name(t.c));
    } else {
      out->m_loop = rr.m;
      out->n_loop = rr.n;
      out->k_loop = rr.k;
      accept(out, "w8a16_matmul", 0);
      apply_init(init, out_type >= 0, out);
    }
    out->root = root;
    return IREE_MI355X_OK;
  }
  if (!a.arg || !b.arg) {
    reject(out, "matmul input produced by an op the region cannot fold");
    out->root = root;
    return IREE_MI355X_OK;
  }
  // The extensions looked through are exactly what a mixed-precision body
  // does inside a contraction, so the contraction's own body and types are
  // judged with the source types.
  match_one(m, options, t, init, out_type >= 0, out);
  out->root = root;
  return IREE_MI355X_OK;
}

}  // extern "C"
