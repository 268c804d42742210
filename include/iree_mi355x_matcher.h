// Dispatch matcher: decides, from a linalg op's structure, whether (and how)
// this library computes it. Host-only: no HIP call, usable without a GPU.
//
// This is the plugin-side half of the reference's matmul path: what its
// configuration pipeline does before any kernel is chosen.
//  * HexagonSpecializeHmxContractionsPass
//    (CG/Transforms/HexagonSpecializeHmxContractions.cpp:29-59) rewrites an
//    f16 linalg.generic contraction into a named linalg.matmul /
//    batch_matmul when HMX can lower it;
//  * isHmxCandidateContraction / hasHmxElementTypes / isHmxLowerableMatmul
//    and analyzeSupportedContraction
//    (CG/Strategy/Planning/Strategies/ContractionStrategy.cpp:27-168): one M,
//    N and K loop, at most one batch loop, f16 inputs into f16 / f32, and an
//    output with M before N (a transposed output is rejected);
//  * the attention of examples/attention_layer/attention_layer.mlir:48-105
//    (batch_matmul, softmax generics, batch_matmul), and the
//    iree_linalg_ext.attention op lowered by
//    CG/Pipelines/LoweringPipelines.cpp:561-595.
// Here one call returns the export of the executable library that computes
// the op (include/iree_mi355x_executable_library.h names), its flags and
// loop roles, or "not taken" with the reason. The int8 (linalg.matmul
// i8 x i8 -> i32 and linalg.quantized_matmul with zero points 0) and W8A16
// (int8 weights dequantized by a per-column scale inside the contraction)
// forms, which HMX does not take (ContractionStrategy.cpp:141), are taken
// here by their own exports.
//
// An op is described as data, the way a compiler plugin sees it after
// walking the IR: loops and iterator types, one indexing map per operand
// (the loop each result dimension reads, or IREE_MI355X_MAP_ZERO for the
// constant 0 of a broadcast), element types, where each operand comes from
// (another op of the dispatch region, a region argument, or a constant), and
// the body as a list of scalar ops in SSA form.
#ifndef IREE_MI355X_MATCHER_H_
#define IREE_MI355X_MATCHER_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IREE_MI355X_LINALG_MAX_LOOPS 8
#define IREE_MI355X_LINALG_MAX_OPERANDS 6
#define IREE_MI355X_LINALG_MAX_BODY 24

// Op kinds.
#define IREE_MI355X_LINALG_GENERIC 0u
#define IREE_MI355X_LINALG_MATMUL 1u            // linalg.matmul (maps given)
#define IREE_MI355X_LINALG_BATCH_MATMUL 2u      // linalg.batch_matmul
#define IREE_MI355X_LINALG_QUANTIZED_MATMUL 3u  // A, B, zero point A, zero point B
#define IREE_MI355X_LINALG_FILL 4u
#define IREE_MI355X_LINALG_TRANSPOSE 5u         // output map permutes the input's
#define IREE_MI355X_LINALG_ATTENTION 6u         // iree_linalg_ext.attention

// Element types.
#define IREE_MI355X_TYPE_NONE 0
#define IREE_MI355X_TYPE_F16 1
#define IREE_MI355X_TYPE_BF16 2
#define IREE_MI355X_TYPE_F32 3
#define IREE_MI355X_TYPE_F64 4
#define IREE_MI355X_TYPE_I1 5
#define IREE_MI355X_TYPE_I8 6
#define IREE_MI355X_TYPE_I32 7
#define IREE_MI355X_TYPE_I64 8
#define IREE_MI355X_TYPE_INDEX 9

// An indexing-map result that is the constant 0 (a broadcast dimension).
#define IREE_MI355X_MAP_ZERO (-1)
// Producers of an operand other than an op of the region.
#define IREE_MI355X_FROM_ARGUMENT (-1)  // a region (dispatch) argument
#define IREE_MI355X_FROM_CONSTANT (-2)  // a splat constant: `scalar` holds it

// Body ops. Value ids: 0 .. inputs+outputs-1 are the block arguments
// (inputs, then outputs); body op i defines value inputs+outputs+i.
#define IREE_MI355X_BODY_YIELD 0u     // operands: the yielded values
#define IREE_MI355X_BODY_CONST 1u     // `constant`
#define IREE_MI355X_BODY_EXTF 2u
#define IREE_MI355X_BODY_TRUNCF 3u
#define IREE_MI355X_BODY_EXTSI 4u
#define IREE_MI355X_BODY_SITOFP 5u
#define IREE_MI355X_BODY_MULF 6u
#define IREE_MI355X_BODY_ADDF 7u
#define IREE_MI355X_BODY_SUBF 8u
#define IREE_MI355X_BODY_DIVF 9u
#define IREE_MI355X_BODY_MAXF 10u     // arith.maximumf
#define IREE_MI355X_BODY_EXP 11u      // math.exp
#define IREE_MI355X_BODY_MULI 12u
#define IREE_MI355X_BODY_ADDI 13u
#define IREE_MI355X_BODY_SUBI 14u
#define IREE_MI355X_BODY_INDEX 15u    // linalg.index `constant` (a loop)
#define IREE_MI355X_BODY_INDEX_CAST 16u
#define IREE_MI355X_BODY_CMPF 17u     // predicate in `constant`: 1 oeq, 2 ogt
#define IREE_MI355X_BODY_CMPI 18u     // predicate in `constant`: 1 eq, 2 sgt, 3 ugt
#define IREE_MI355X_BODY_SELECT 19u   // operands: condition, true, false
#define IREE_MI355X_BODY_ANDI 20u

#define IREE_MI355X_PRED_EQ 1
#define IREE_MI355X_PRED_GT 2
#define IREE_MI355X_PRED_UGT 3

typedef struct iree_mi355x_body_op_t {
  uint32_t opcode;      // IREE_MI355X_BODY_*
  int32_t operands[3];  // value ids, -1 where unused
  int32_t type;         // result element type (IREE_MI355X_TYPE_*)
  double constant;      // CONST value, INDEX loop, CMP predicate
} iree_mi355x_body_op_t;

typedef struct iree_mi355x_linalg_op_t {
  uint32_t kind;                // IREE_MI355X_LINALG_*
  uint32_t num_loops;           // <= IREE_MI355X_LINALG_MAX_LOOPS
  uint32_t reduction_loops;     // bit d set: loop d is a reduction
  int64_t loop_extent[IREE_MI355X_LINALG_MAX_LOOPS];  // -1: dynamic
  uint32_t num_inputs;
  uint32_t num_outputs;
  // Per operand (inputs, then outputs):
  int32_t elem_type[IREE_MI355X_LINALG_MAX_OPERANDS];
  uint32_t map_rank[IREE_MI355X_LINALG_MAX_OPERANDS];
  int32_t map[IREE_MI355X_LINALG_MAX_OPERANDS][IREE_MI355X_LINALG_MAX_LOOPS];
  int32_t producer[IREE_MI355X_LINALG_MAX_OPERANDS];  // op index or FROM_*
  int32_t producer_result[IREE_MI355X_LINALG_MAX_OPERANDS];
  double scalar[IREE_MI355X_LINALG_MAX_OPERANDS];  // FROM_CONSTANT value
  uint32_t num_body_ops;
  iree_mi355x_body_op_t body[IREE_MI355X_LINALG_MAX_BODY];
} iree_mi355x_linalg_op_t;

typedef struct iree_mi355x_match_t {
  int32_t taken;           // 1: `export_name` computes the op (or region)
  char export_name[32];    // executable-library export
  uint32_t flags;          // IREE_MI355X_MATMUL_* / IREE_MI355X_ATTENTION_*
  int32_t batch_loop;      // loop roles (-1: none)
  int32_t m_loop, n_loop, k_loop;
  int32_t root;            // region: index of the op whose result it writes
  // Attention: the scale applied to q.k (the product of every constant
  // factor on Q, K or the scores) and the head loop (-1: none).
  float scale;
  int32_t head_loop;
  char reason[160];        // why not taken (empty when taken)
  // Contractions compute init + A.B. A zero init (a splat 0 or a
  // linalg.fill of 0) gives the overwriting export; a region argument gives
  // IREE_MI355X_MATMUL_ACCUMULATE, reading the output buffer as the init. A
  // fill of another constant also gives ACCUMULATE with init_fill = 1: the
  // caller first fills the output with init_value (a command-buffer fill),
  // as the reference unpacks HMX tiles into the filled init
  // (test/codegen/transforms/convert_matmul_to_hmx.mlir:40-55).
  int32_t init_fill;
  double init_value;
  // Attention: the loop of Q's and K's head dim (n_loop is V's and O's); in
  // the decomposed chain, whose loops are those of P.V, the two are equal
  // and this is n_loop. With IREE_MI355X_ATTENTION_MASK the op's mask input
  // is a region argument whose map selects, in order, some of (batch_loop,
  // head_loop, m_loop, k_loop); the dimensions it leaves out broadcast.
  int32_t head_dim_loop;
} iree_mi355x_match_t;

// Options.
// Strategy selection alone, without the specialization pass before it: a
// matmul-shaped linalg.generic is then not taken (the reference warns and
// plans it without HMX, test/codegen/strategy/
// hexagon_strategy_hmx_generic_contraction.mlir); only named ops are.
#define IREE_MI355X_MATCH_NAMED_ONLY 0x1u

// One op. Returns IREE_MI355X_OK (with out->taken 0 or 1) or
// IREE_MI355X_INVALID_ARGUMENT for a malformed description (a map naming a
// loop past num_loops, a body value used before it is defined, ...).
int iree_mi355x_match_linalg_op(const iree_mi355x_linalg_op_t *op,
                                uint32_t options, iree_mi355x_match_t *out);

// A dispatch region: ops in program order, producers referring to earlier
// ops; the last op's first result is the region's result. Takes what one op
// takes, a dequantization generic feeding a matmul (W8A16), elementwise
// extensions of matmul inputs, and the attention chain (scaled Q.K^T,
// row max, exp, row sum, divide, optional all-masked-row guard and causal
// mask, P.V, truncation) or an iree_linalg_ext.attention op.
int iree_mi355x_match_dispatch_region(const iree_mi355x_linalg_op_t *ops,
                                      uint32_t count, uint32_t options,
                                      iree_mi355x_match_t *out);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_MATCHER_H_
