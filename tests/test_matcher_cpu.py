"""The dispatch matcher (include/iree_mi355x_matcher.h) on the reference's own
fixtures, without a GPU.

Each case transcribes, as data (loops, maps, element types, body), one
function of the reference's lit tests, and asserts what the reference's
pipeline decides for it, restated for this library's exports:

  * plugins/compiler/hexagon/test/codegen/transforms/
    specialize_hmx_contractions.mlir (all six functions);
  * .../test/codegen/strategy/hexagon_strategy_hmx_generic_contraction.mlir
    (all four functions: a generic is planned without HMX when strategy
    selection runs alone, named_only=True here);
  * .../test/codegen/transforms/convert_matmul_to_hmx.mlir (the maps and
    element types of its converted matmuls) and convert_matmul_to_hmx_invalid
    .mlir (dynamic and empty extents, taken here on purpose: this library's
    extents are launch arguments, not the static HMX packing grid);
  * examples/attention_layer/attention_layer.mlir:48-105, the decomposed
    attention, and variants of it.
"""
import functools
import math

import pytest

MIXED_BODY = [("a32", "extf", ["a"], "f32"), ("b32", "extf", ["b"], "f32"),
              ("m", "mulf", ["a32", "b32"], "f32"),
              ("s", "addf", ["c", "m"], "f32"), ("yield", ["s"])]
F16_BODY = [("m", "mulf", ["a", "b"], "f16"), ("s", "addf", ["c", "m"], "f16"),
            ("yield", ["s"])]
F32_BODY = [("m", "mulf", ["a", "b"], "f32"), ("s", "addf", ["c", "m"], "f32"),
            ("yield", ["s"])]
ABC = ["a", "b", "c"]


def generic(pkg, loops, red, maps, types, body, extents=None, inputs=2,
            args=ABC, producers=None):
    return pkg.linalg_op(pkg.OP_GENERIC, loops, maps, types, inputs=inputs,
                         reductions=red, body=body, args=args,
                         extents=extents, producers=producers)


def named(pkg, kind, loops, red, maps, types, extents=None, producers=None):
    return pkg.linalg_op(kind, loops, maps, types, inputs=len(maps) - 1,
                         reductions=red, extents=extents, producers=producers)


def fill(pkg, loops, typ, value):
    """linalg.fill ins(%value) outs(%empty) over all of `loops`."""
    return pkg.linalg_op(pkg.OP_FILL, loops, ["", loops], [typ, typ],
                         inputs=1, producers=[("const", value)])


# The init of a contraction's output as a zero splat constant, what a
# linalg.fill of 0 amounts to. Cases that transcribe a lit function with a
# fill op describe the fill as an op of a region instead.
ZERO_INIT = ("const", 0.0)


# ----------------------------------------- specialize_hmx_contractions.mlir --

def test_f16_mixed_precision_transposed_rhs(pkg):
    op = generic(pkg, "d0 d1 d2", ["d2"], ["d0 d2", "d1 d2", "d0 d1"],
                 ["f16", "f16", "f32"], MIXED_BODY,
                 {"d0": 64, "d1": 128, "d2": 96})
    m = pkg.match(op)
    assert m.taken and m.export == "matmul_f16", m.reason
    # outs(%init), a function argument: the contraction adds into it
    assert m.flags == pkg.B_TRANSPOSED | pkg.OUT_F32 | pkg.ACCUMULATE
    assert not m.init_fill
    assert (m.m_loop, m.n_loop, m.k_loop, m.batch_loop) == (0, 1, 2, -1)


def test_f16_batch_contraction(pkg):
    op = generic(pkg, "d0 d1 d2 d3", ["d3"],
                 ["d0 d1 d3", "d0 d3 d2", "d0 d1 d2"], ["f16"] * 3, F16_BODY)
    m = pkg.match(op)
    assert m.taken and m.export == "batch_matmul_f16", m.reason
    assert m.flags == pkg.ACCUMULATE  # outs(%init), an argument
    assert (m.batch_loop, m.m_loop, m.n_loop, m.k_loop) == (0, 1, 2, 3)


def test_f32_contraction_is_kept(pkg):
    op = generic(pkg, "d0 d1 d2", ["d2"], ["d0 d2", "d2 d1", "d0 d1"],
                 ["f32"] * 3, F32_BODY)
    m = pkg.match(op)
    assert not m.taken and "element types" in m.reason


def test_transposed_output_is_kept(pkg):
    op = generic(pkg, "d0 d1 d2", ["d2"], ["d0 d2", "d2 d1", "d1 d0"],
                 ["f16", "f16", "f32"], MIXED_BODY)
    m = pkg.match(op)
    assert not m.taken and "transposed output" in m.reason


def test_two_reduction_dims_are_kept(pkg):
    op = generic(pkg, "d0 d1 d2 d3", ["d2", "d3"],
                 ["d0 d2 d3", "d3 d2 d1", "d0 d1"], ["f16"] * 3, F16_BODY)
    m = pkg.match(op)
    assert not m.taken and "not matmul-shaped" in m.reason
    assert "2 K" in m.reason


def test_elementwise_is_kept(pkg):
    op = generic(pkg, "d0 d1", [], ["d0 d1"] * 3, ["f16"] * 3,
                 [("s", "addf", ["a", "b"], "f16"), ("yield", ["s"])])
    m = pkg.match(op)
    assert not m.taken and "elementwise" in m.reason


# ------------------------- hexagon_strategy_hmx_generic_contraction.mlir --

def test_strategy_generic_contraction_planned_without_mfma(pkg):
    # %init = linalg.fill ins(%zero : f32) outs(%empty), then the generic
    init = fill(pkg, "d0 d1", "f32", 0.0)
    op = generic(pkg, "d0 d1 d2", ["d2"], ["d0 d2", "d1 d2", "d0 d1"],
                 ["f16", "f16", "f32"], MIXED_BODY,
                 {"d0": 256, "d1": 1024, "d2": 1536},
                 producers=["arg", "arg", 0])
    alone = pkg.match_region([init, op], named_only=True)
    assert not alone.taken and "only named" in alone.reason
    # the configuration pipeline specializes it first: then it is taken
    full = pkg.match_region([init, op])
    assert full.taken and full.flags == pkg.B_TRANSPOSED | pkg.OUT_F32
    assert full.root == 1 and not full.init_fill


def test_strategy_named_contraction(pkg):
    init = fill(pkg, "d0 d1", "f32", 0.0)
    op = named(pkg, pkg.OP_MATMUL, "d0 d1 d2", ["d2"],
               ["d0 d2", "d1 d2", "d0 d1"], ["f16", "f16", "f32"],
               producers=["arg", "arg", 0])
    m = pkg.match_region([init, op], named_only=True)
    assert m.taken and m.export == "matmul_f16", m.reason
    assert m.flags == pkg.B_TRANSPOSED | pkg.OUT_F32


def test_strategy_named_transposed_output(pkg):
    op = named(pkg, pkg.OP_MATMUL, "d0 d1 d2", ["d2"],
               ["d0 d2", "d1 d2", "d1 d0"], ["f16", "f16", "f32"])
    m = pkg.match(op, named_only=True)
    assert not m.taken and "transposed output" in m.reason


def test_strategy_named_unsupported_output_type(pkg):
    op = named(pkg, pkg.OP_MATMUL, "d0 d1 d2", ["d2"],
               ["d0 d2", "d2 d1", "d0 d1"], ["f16", "f16", "bf16"])
    m = pkg.match(op, named_only=True)
    assert not m.taken and "bf16" in m.reason


# ------------------------------------------------ convert_matmul_to_hmx.mlir --

@pytest.mark.parametrize("maps,out,init,flags", [
    # @convert_f32_output / @convert_ragged: a fill of 0
    (["m k", "k n", "m n"], "f32", 0.0, "OUT_F32"),
    # @convert_f16_output: a fill of 5.0 kept as the accumulation's init
    (["m k", "k n", "m n"], "f16", 5.0, "ACCUMULATE"),
    # @convert_both_inputs_transposed
    (["k m", "n k", "m n"], "f32", 0.0, "A_TRANSPOSED B_TRANSPOSED OUT_F32"),
])
def test_convert_matmul_layouts(pkg, maps, out, init, flags):
    filled = fill(pkg, "m n", out, init)
    op = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], maps, ["f16", "f16", out],
               {"m": 1537, "n": 1539, "k": 257}, producers=["arg", "arg", 0])
    m = pkg.match_region([filled, op])
    want = 0
    for f in flags.split():
        want |= getattr(pkg, f)
    assert m.taken and m.export == "matmul_f16" and m.flags == want, m.reason
    # the caller fills the output with the constant before an accumulating
    # dispatch; a zero fill needs none
    assert m.init_fill == (init != 0.0) and m.init_value == init


def test_convert_unit_batch_transpose_b(pkg):
    filled = fill(pkg, "b m n", "f32", 0.0)
    op = named(pkg, pkg.OP_BATCH_MATMUL, "b m n k", ["k"],
               ["b m k", "b n k", "b m n"], ["f16", "f16", "f32"],
               {"b": 1, "m": 32, "n": 32, "k": 64}, producers=["arg", "arg", 0])
    m = pkg.match_region([filled, op])
    assert m.taken and m.export == "batch_matmul_f16", m.reason
    assert m.flags == pkg.B_TRANSPOSED | pkg.OUT_F32 and m.batch_loop == 0


@pytest.mark.parametrize("extents", [
    {"m": -1, "n": -1, "k": 64},   # reject_unbounded_dynamic_shape
    {"m": 0, "n": 32, "k": 64},    # reject_zero_logical_extent
    {"m": 1537, "n": -1, "k": 257},  # convert_bounded_dynamic_boundary
])
def test_dynamic_and_empty_extents_are_taken(pkg, extents):
    op = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
               ["f16", "f16", "f32"], extents)
    m = pkg.match(op)
    assert m.taken and m.export == "matmul_f16", m.reason


# ---------------------------------------------- int8, zero points, W8A16 ----

I8_BODY = [("a32", "extsi", ["a"], "i32"), ("b32", "extsi", ["b"], "i32"),
           ("m", "muli", ["a32", "b32"], "i32"),
           ("s", "addi", ["c", "m"], "i32"), ("yield", ["s"])]


def test_int8_generic_and_named(pkg):
    op = generic(pkg, "m n k", ["k"], ["m k", "n k", "m n"],
                 ["i8", "i8", "i32"], I8_BODY)
    m = pkg.match(op)
    assert m.taken and m.export == "matmul_i8", m.reason
    assert m.flags == pkg.B_TRANSPOSED | pkg.ACCUMULATE
    op = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
               ["i8", "i8", "i32"], producers=["arg", "arg", ZERO_INIT])
    m = pkg.match(op)
    assert m.taken and m.export == "matmul_i8" and m.flags == 0
    # int8 kernels have no transposed-A or batched form
    op = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["k m", "k n", "m n"],
               ["i8", "i8", "i32"])
    assert not pkg.match(op).taken
    # an f32 body over int8 inputs is not the integer contraction
    op = generic(pkg, "m n k", ["k"], ["m k", "n k", "m n"],
                 ["i8", "i8", "i32"], F32_BODY)
    assert not pkg.match(op).taken


@pytest.mark.parametrize("zp,taken", [((0, 0), True), ((3, 0), False),
                                      ((0, -1), False)])
def test_quantized_matmul_zero_points(pkg, zp, taken):
    op = pkg.linalg_op(pkg.OP_QUANTIZED_MATMUL, "m n k",
                       ["m k", "k n", "", "", "m n"],
                       ["i8", "i8", "i32", "i32", "i32"], inputs=4,
                       reductions=["k"],
                       producers=["arg", "arg", ("const", zp[0]),
                                  ("const", zp[1])])
    m = pkg.match(op)
    assert m.taken == taken, m.reason
    if taken:
        assert m.export == "matmul_i8"
    else:
        assert "zero point" in m.reason


def test_quantized_matmul_runtime_zero_point_not_taken(pkg):
    op = pkg.linalg_op(pkg.OP_QUANTIZED_MATMUL, "m n k",
                       ["m k", "k n", "", "", "m n"],
                       ["i8", "i8", "i32", "i32", "i32"], inputs=4,
                       reductions=["k"])
    m = pkg.match(op)
    assert not m.taken and "not constants" in m.reason


def test_generic_zero_point_subtraction(pkg):
    def body(zp):
        return [("a32", "extsi", ["a"], "i32"), ("z", "const", [], "i32", zp),
                ("az", "subi", ["a32", "z"], "i32"),
                ("b32", "extsi", ["b"], "i32"),
                ("m", "muli", ["az", "b32"], "i32"),
                ("s", "addi", ["c", "m"], "i32"), ("yield", ["s"])]
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["i8", "i8", "i32"], body(0))
    assert pkg.match(op).taken
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["i8", "i8", "i32"], body(5))
    m = pkg.match(op)
    assert not m.taken and "zero point" in m.reason


W8_ARGS = ["x", "w", "s", "y"]


@pytest.mark.parametrize("order", ["dequant_then_mul", "scale_after"])
def test_w8a16_fused_dequant_generic(pkg, order):
    if order == "dequant_then_mul":
        body = [("wf", "sitofp", ["w"], "f16"), ("wd", "mulf", ["wf", "s"], "f16"),
                ("x32", "extf", ["x"], "f32"), ("w32", "extf", ["wd"], "f32"),
                ("p", "mulf", ["x32", "w32"], "f32"),
                ("y32", "extf", ["y"], "f32"),
                ("r", "addf", ["y32", "p"], "f32"),
                ("t", "truncf", ["r"], "f16"), ("yield", ["t"])]
    else:
        body = [("wf", "sitofp", ["w"], "f16"), ("p", "mulf", ["x", "wf"], "f16"),
                ("q", "mulf", ["p", "s"], "f16"),
                ("r", "addf", ["y", "q"], "f16"), ("yield", ["r"])]
    prods = ["arg", "arg", "arg", ZERO_INIT]
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "n", "m n"],
                 ["f16", "i8", "f16", "f16"], body, inputs=3, args=W8_ARGS,
                 producers=prods)
    m = pkg.match(op)
    if order == "dequant_then_mul":
        # a truncation of the accumulation inside the body is not the
        # accumulate-in-the-output form: not taken as one op
        assert not m.taken
    else:
        assert m.taken and m.export == "w8a16_matmul", m.reason
        # accumulating into an argument: the W8A16 export has no such form
        op = generic(pkg, "m n k", ["k"], ["m k", "k n", "n", "m n"],
                     ["f16", "i8", "f16", "f16"], body, inputs=3,
                     args=W8_ARGS)
        m = pkg.match(op)
        assert not m.taken and "no accumulating form" in m.reason
    # a per-row (K) scale is not the per-output-channel dequantization
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "k", "m n"],
                 ["f16", "i8", "f16", "f16"], body, inputs=3, args=W8_ARGS,
                 producers=prods)
    assert not pkg.match(op).taken


def dequant(pkg):
    return generic(pkg, "k n", [], ["k n", "n", "k n"], ["i8", "f16", "f16"],
                   [("wf", "sitofp", ["w"], "f16"),
                    ("d", "mulf", ["wf", "s"], "f16"), ("yield", ["d"])],
                   args=["w", "s", "o"])


def test_w8a16_dequant_generic_feeding_matmul(pkg):
    dq = dequant(pkg)
    mm = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
               ["f16", "f16", "f16"], {"m": 1, "n": 11008, "k": 4096},
               producers=["arg", 0, ZERO_INIT])
    m = pkg.match_region([dq, mm])
    assert m.taken and m.export == "w8a16_matmul" and m.root == 1, m.reason
    assert (m.m_loop, m.n_loop, m.k_loop) == (0, 1, 2) and m.flags == 0
    # the same with the init a fill op of the region
    filled = fill(pkg, "m n", "f16", 0.0)
    mm_f = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["f16", "f16", "f16"], producers=["arg", 0, 1])
    m = pkg.match_region([dq, filled, mm_f])
    assert m.taken and m.export == "w8a16_matmul" and m.root == 2, m.reason
    # the weight transposed by the matmul's map: no kernel
    mm2 = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "n k", "m n"],
                ["f16", "f16", "f16"], producers=["arg", 0, ZERO_INIT])
    assert not pkg.match_region([dq, mm2]).taken


def test_w8a16_region_keeps_every_producer_of_a(pkg):
    # relu(x) feeding the matmul's A: the kernel reads x itself, so the
    # region is not taken (without the dequantization it is not either)
    relu = generic(pkg, "m k", [], ["m k", "m k"], ["f16", "f16"],
                   [("z", "const", [], "f16", 0.0),
                    ("r", "maximumf", ["i", "z"], "f16"), ("yield", ["r"])],
                   inputs=1, args=["i", "o"])
    dq = dequant(pkg)
    mm = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
               ["f16", "f16", "f16"], producers=[0, 1, ZERO_INIT])
    m = pkg.match_region([relu, dq, mm])
    assert not m.taken and "cannot fold" in m.reason
    plain = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
                  ["f16", "f16", "f16"], producers=[0, "arg", ZERO_INIT])
    assert not pkg.match_region([relu, plain]).taken


def test_w8a16_region_generic_matmul_rules(pkg):
    dq = dequant(pkg)
    gm = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["f16", "f16", "f16"], F16_BODY,
                 producers=["arg", 0, ZERO_INIT])
    m = pkg.match_region([dq, gm])
    assert m.taken and m.export == "w8a16_matmul", m.reason
    # strategy selection alone takes named matmuls only
    m = pkg.match_region([dq, gm], named_only=True)
    assert not m.taken and "only named" in m.reason
    # a generic whose body is not the multiply-accumulate
    wrong = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                    ["f16", "f16", "f16"],
                    [("m", "addf", ["a", "b"], "f16"),
                     ("s", "addf", ["c", "m"], "f16"), ("yield", ["s"])],
                    producers=["arg", 0, ZERO_INIT])
    m = pkg.match_region([dq, wrong])
    assert not m.taken and "product" in m.reason


# ------------------------------------------------------------ output init ----

def test_output_init_forms(pkg):
    maps = ["m k", "k n", "m n"]

    def mm(init_producer, out="f16"):
        return named(pkg, pkg.OP_MATMUL, "m n k", ["k"], maps,
                     ["f16", "f16", out], producers=["arg", "arg",
                                                     init_producer])
    # outs from a region argument: C_out = C_init + A.B
    m = pkg.match_region([mm("arg")])
    assert m.taken and m.flags == pkg.ACCUMULATE and not m.init_fill
    # a fill of 0 (an op, or a splat): overwrite
    m = pkg.match_region([fill(pkg, "m n", "f16", 0.0), mm(0)])
    assert m.taken and m.flags == 0 and not m.init_fill
    m = pkg.match(mm(ZERO_INIT))
    assert m.taken and m.flags == 0
    # a fill of 1.0: accumulate into the filled output
    m = pkg.match_region([fill(pkg, "m n", "f16", 1.0), mm(0)])
    assert m.taken and m.flags == pkg.ACCUMULATE
    assert m.init_fill and m.init_value == 1.0
    m = pkg.match(mm(("const", -2.5)))
    assert m.taken and m.init_fill and m.init_value == -2.5
    # a fill of a value that is not a constant
    dyn = pkg.linalg_op(pkg.OP_FILL, "m n", ["", "m n"], ["f16", "f16"],
                        inputs=1)
    m = pkg.match_region([dyn, mm(0)])
    assert not m.taken and "not a constant" in m.reason
    # an init computed by another op (an elementwise generic)
    neg = generic(pkg, "m n", [], ["m n", "m n"], ["f16", "f16"],
                  [("z", "const", [], "f16", -1.0),
                   ("r", "mulf", ["i", "z"], "f16"), ("yield", ["r"])],
                  inputs=1, args=["i", "o"])
    m = pkg.match_region([neg, mm(0)])
    assert not m.taken and "not a fill" in m.reason
    # a lone op whose init an undescribed op produces
    m = pkg.match(mm(3))
    assert not m.taken and "outside the description" in m.reason


def test_output_init_with_truncation(pkg):
    # f32 accumulation, then truncf to f16: a zero init is taken, an init
    # accumulated in f32 is not (the exports read an init in the output type)
    def region(init_producer):
        mm = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
                   ["f16", "f16", "f32"],
                   producers=["arg", "arg", init_producer])
        tr = generic(pkg, "m n", [], ["m n", "m n"], ["f32", "f16"],
                     [("t", "truncf", ["i"], "f16"), ("yield", ["t"])],
                     inputs=1, args=["i", "o"], producers=[0])
        return [mm, tr]
    m = pkg.match_region(region(ZERO_INIT))
    assert m.taken and m.export == "matmul_f16" and m.flags == 0, m.reason
    m = pkg.match_region(region("arg"))
    assert not m.taken and "truncation" in m.reason
    m = pkg.match_region(region(("const", 2.0)))
    assert not m.taken and "truncation" in m.reason


# ------------------------------------------------------------- attention ----

INF = float("inf")
SCALE = 0.29730177875068026  # attention_layer.mlir: 128^-1/4 on Q and on K


def ew(pkg, types, body, producers, args=("i", "o"), loops="d0 d1 d2",
       maps=None):
    n = len(types)
    return pkg.linalg_op(pkg.OP_GENERIC, loops,
                         maps or ["d0 d1 d2"] * n, types, inputs=n - 1,
                         body=body, args=list(args), producers=producers)


def attention_chain(pkg, *, head=128, causal=False, guard=True, exp=True,
                    out="f16", q_scale=SCALE, bmm_init=("const", 0.0),
                    max_init=-INF, sum_init=0.0, bmm1_body=None, batch=4,
                    seq=1024):
    """The ops of attention_layer.mlir:48-105 in program order (reshapes are
    views and so not ops: a consumer of an expand_shape names the op whose
    result it reshapes)."""
    ops = []

    def add(op):
        ops.append(op)
        return len(ops) - 1
    ext = [("e", "extf", ["i"], "f32"), ("yield", ["e"])]
    q32 = add(ew(pkg, ["f16", "f32"], ext, ["arg"]))
    k32 = add(ew(pkg, ["f16", "f32"], ext, ["arg"]))
    v32 = add(ew(pkg, ["f16", "f32"], ext, ["arg"]))

    def scale_body(c):
        return [("c", "const", [], "f64", c), ("t", "truncf", ["c"], "f32"),
                ("r", "mulf", ["i", "t"], "f32"), ("yield", ["r"])]
    qs = add(ew(pkg, ["f32", "f32"], scale_body(q_scale), [q32]))
    kt = add(pkg.linalg_op(pkg.OP_TRANSPOSE, "d0 d1 d2",
                           ["d0 d2 d1", "d0 d1 d2"], ["f32", "f32"], inputs=1,
                           producers=[k32]))
    ks = add(ew(pkg, ["f32", "f32"], scale_body(SCALE), [kt]))
    if bmm1_body is None:
        s = add(pkg.linalg_op(pkg.OP_BATCH_MATMUL, "b m n k",
                              ["b m k", "b k n", "b m n"], ["f32"] * 3,
                              inputs=2, reductions=["k"],
                              extents={"b": batch, "m": seq, "n": seq,
                                       "k": head},
                              producers=[qs, ks, bmm_init]))
    else:
        s = add(pkg.linalg_op(pkg.OP_GENERIC, "b m n k",
                              ["b m k", "b k n", "b m n"], ["f32"] * 3,
                              inputs=2, reductions=["k"], body=bmm1_body,
                              args=ABC,
                              extents={"b": batch, "m": seq, "n": seq,
                                       "k": head},
                              producers=[qs, ks, bmm_init]))
    if causal:
        s = add(ew(pkg, ["f32", "f32"], [
            ("q", "index", [], "index", "d1"), ("k", "index", [], "index", "d2"),
            ("gt", "cmpi", ["k", "q"], "i1", "sgt"),
            ("ninf", "const", [], "f32", -INF),
            ("r", "select", ["gt", "ninf", "i"], "f32"), ("yield", ["r"])],
            [s]))
    red = ["d2"]
    mx = add(pkg.linalg_op(pkg.OP_GENERIC, "d0 d1 d2",
                           ["d0 d1 d2", "d0 d1", "d0 d1"],
                           ["f32", "f32", "i64"], inputs=1, reductions=red,
                           args=["i", "o", "idx"],
                           producers=[s, ("const", max_init),
                                      ("const", 0.0)],
                           body=[("j", "index", [], "index", "d2"),
                                 ("ji", "index_cast", ["j"], "i64"),
                                 ("mx", "maximumf", ["i", "o"], "f32"),
                                 ("gt", "cmpf", ["i", "o"], "i1", "ogt"),
                                 ("ix", "select", ["gt", "ji", "idx"], "i64"),
                                 ("yield", ["mx", "ix"])]))
    sub = add(ew(pkg, ["f32", "f32", "f32"],
                 [("d", "subf", ["i", "j"], "f32"), ("yield", ["d"])],
                 [s, mx], args=("i", "j", "o"),
                 maps=["d0 d1 d2", "d0 d1 0", "d0 d1 d2"]))
    e = add(ew(pkg, ["f32", "f32"],
               [("x", "exp" if exp else "extf", ["i"], "f32"), ("yield", ["x"])],
               [sub]))
    total = add(pkg.linalg_op(pkg.OP_GENERIC, "d0 d1 d2",
                              ["d0 d1 d2", "d0 d1 0"], ["f32", "f32"],
                              inputs=1, reductions=red,
                              producers=[e, ("const", sum_init)],
                              args=["i", "o"],
                              body=[("a", "addf", ["i", "o"], "f32"),
                                    ("yield", ["a"])]))
    p = add(ew(pkg, ["f32", "f32", "f32"],
               [("q", "divf", ["i", "j"], "f32"), ("yield", ["q"])],
               [e, total], args=("i", "j", "o"),
               maps=["d0 d1 d2", "d0 d1 0", "d0 d1 d2"]))
    if guard:
        isinf = add(ew(pkg, ["f32", "i1"], [
            ("w", "extf", ["i"], "f64"), ("n", "const", [], "f64", -INF),
            ("c", "cmpf", ["w", "n"], "i1", "oeq"), ("yield", ["c"])], [s]))
        allinf = add(pkg.linalg_op(pkg.OP_GENERIC, "d0 d1 d2",
                                   ["d0 d1 d2", "d0 d1 0"], ["i1", "i1"],
                                   inputs=1, reductions=red,
                                   producers=[isinf, ("const", 1.0)],
                                   args=["i", "o"],
                                   body=[("a", "andi", ["i", "o"], "i1"),
                                         ("yield", ["a"])]))
        p = add(pkg.linalg_op(pkg.OP_GENERIC, "d0 d1 d2",
                              ["d0 d1 0", "d0 d1 d2", "d0 d1 d2", "d0 d1 d2"],
                              ["i1", "f32", "f32", "f32"], inputs=3,
                              producers=[allinf, ("const", 0.0), p],
                              args=["c", "z", "p", "o"],
                              body=[("r", "select", ["c", "z", "p"], "f32"),
                                    ("yield", ["r"])]))
    o = add(pkg.linalg_op(pkg.OP_BATCH_MATMUL, "b m n k",
                          ["b m k", "b k n", "b m n"], ["f32"] * 3, inputs=2,
                          reductions=["k"],
                          extents={"b": batch, "m": seq, "n": head, "k": seq},
                          producers=[p, v32, ("const", 0.0)]))
    if out == "f16":
        add(ew(pkg, ["f32", "f16"], [("t", "truncf", ["i"], "f16"),
                                     ("yield", ["t"])], [o]))
    return ops


def test_attention_layer_chain(pkg):
    ops = attention_chain(pkg)
    m = pkg.match_region(ops)
    assert m.taken and m.export == "attention_f16", m.reason
    assert m.flags == 0 and m.root == len(ops) - 1
    # the two 128^-1/4 factors make the 1/sqrt(128) of SDPA
    assert math.isclose(m.scale, 1 / math.sqrt(128), rel_tol=1e-6)
    assert (m.batch_loop, m.m_loop, m.n_loop, m.k_loop) == (0, 1, 2, 3)


def test_attention_chain_variants(pkg):
    m = pkg.match_region(attention_chain(pkg, causal=True))
    assert m.taken and m.flags == pkg.CAUSAL, m.reason
    m = pkg.match_region(attention_chain(pkg, guard=False))
    assert m.taken, m.reason
    m = pkg.match_region(attention_chain(pkg, q_scale=1.0))
    assert m.taken and math.isclose(m.scale, SCALE, rel_tol=1e-6)
    m = pkg.match_region(attention_chain(pkg, head=64))
    assert m.taken
    # not attention, or not a kernel of this library
    m = pkg.match_region(attention_chain(pkg, exp=False))
    assert not m.taken
    # other head dims and an f32 result take the general kernel
    m = pkg.match_region(attention_chain(pkg, head=96))
    assert m.taken and m.flags == 0, m.reason
    assert m.head_dim_loop == m.n_loop
    m = pkg.match_region(attention_chain(pkg, out="f32"))
    assert m.taken and m.flags == pkg.ATTENTION_OUT_F32, m.reason
    m = pkg.match_region(attention_chain(pkg, head=300))
    assert not m.taken and "head dims" in m.reason


def test_attention_chain_inits(pkg):
    # attention_layer.mlir starts both batch_matmuls from a zero fill, the
    # row max from -inf (0xFF800000) and the row sum from 0
    m = pkg.match_region(attention_chain(pkg, bmm_init="arg"))
    assert not m.taken and "zero fill" in m.reason
    m = pkg.match_region(attention_chain(pkg, bmm_init=("const", 1.0)))
    assert not m.taken and "zero fill" in m.reason
    m = pkg.match_region(attention_chain(pkg, sum_init=1.0))
    assert not m.taken and "row sum" in m.reason
    m = pkg.match_region(attention_chain(pkg, max_init=0.0))
    assert not m.taken and "row max" in m.reason
    # the lowest finite f32 is as good a start as -inf
    m = pkg.match_region(attention_chain(pkg, max_init=-3.4028234663852886e38))
    assert m.taken, m.reason


def test_attention_chain_generic_contraction_bodies(pkg):
    # Q.K^T written as a linalg.generic with the multiply-accumulate body
    m = pkg.match_region(attention_chain(pkg, bmm1_body=F32_BODY))
    assert m.taken and m.export == "attention_f16", m.reason
    # strategy selection alone takes named batch_matmuls only
    m = pkg.match_region(attention_chain(pkg, bmm1_body=F32_BODY),
                         named_only=True)
    assert not m.taken and "only named" in m.reason
    # a reduction body other than the multiply-accumulate is not attention
    maxbody = [("m", "mulf", ["a", "b"], "f32"),
               ("s", "maximumf", ["c", "m"], "f32"), ("yield", ["s"])]
    assert not pkg.match_region(attention_chain(pkg, bmm1_body=maxbody)).taken


def att_op(pkg, head, scale_const=True, mask=None, head_v=None, out="f16",
           mask_type="f16", mask_from="arg", batch_dims="b h", sizes=None,
           scale=0.125):
    """iree_linalg_ext.attention over (batch dims) M K1 K2 N; `mask` is the
    mask's map (None: no mask); `sizes` overrides loop extents."""
    bd = batch_dims.split()
    pre = " ".join(bd)
    maps = [f"{pre} m k1", f"{pre} k2 k1", f"{pre} k2 n", ""]
    types = ["f16", "f16", "f16", "f16"]
    prods = ["arg", "arg", "arg", ("const", scale) if scale_const else "arg"]
    if mask is not None:
        maps.append(mask)
        types.append(mask_type)
        prods.append(mask_from)
    ext = {"b": 1, "h": 32, "g": 2, "m": 2048, "n": head_v or head, "k1": head,
           "k2": 2048}
    ext.update(sizes or {})
    return pkg.linalg_op(pkg.OP_ATTENTION, f"{pre} m n k1 k2",
                         maps + [f"{pre} m n"], types + [out],
                         inputs=len(maps), reductions=["k1", "k2"],
                         extents={d: ext[d] for d in bd + ["m", "n", "k1",
                                                           "k2"]},
                         producers=prods)


def test_linalg_ext_attention_op(pkg):
    att = functools.partial(att_op, pkg)
    m = pkg.match(att(128))
    assert m.taken and m.export == "attention_f16" and m.scale == 0.125
    assert (m.batch_loop, m.head_loop, m.m_loop, m.n_loop, m.k_loop,
            m.head_dim_loop) == (0, 1, 2, 3, 5, 4)
    assert m.flags == 0
    assert not pkg.match(att(128, scale_const=False)).taken
    # head dims 1..256, Q/K and V apart, f16 or f32 output
    m = pkg.match(att(80))
    assert m.taken and m.flags == 0, m.reason
    m = pkg.match(att(4, head_v=5, out="f32"))
    assert m.taken and m.flags == pkg.ATTENTION_OUT_F32, m.reason
    assert m.head_dim_loop == 4 and m.n_loop == 3
    m = pkg.match(att(257))
    assert not m.taken and "head dims" in m.reason
    m = pkg.match(att(64, out="bf16"))
    assert not m.taken and "output" in m.reason
    m = pkg.match(att(64, batch_dims="b g h"))
    assert not m.taken and "batch loops" in m.reason


@pytest.mark.parametrize("mask_map", ["b h m k2", "m k2", "b m k2", "h k2",
                                      "k2", "b h m"])
def test_linalg_ext_attention_argument_mask(pkg, mask_map):
    # an f16 mask from a region argument, full or broadcast along the
    # dimensions its map leaves out
    m = pkg.match(att_op(pkg, 64, mask=mask_map))
    assert m.taken, m.reason
    assert m.flags == pkg.ATTENTION_MASK


@pytest.mark.parametrize("mask_map,mask_type,mask_from,why", [
    ("b h m k2", "i1", "arg", "f16 additive"),
    ("b h m k2", "f32", "arg", "f16 additive"),
    ("b h m k2", "f16", ("const", 0.0), "unknown content"),
    ("b h k2 m", "f16", "arg", "selection"),
    ("b h m k1", "f16", "arg", "selection"),
    ("m b k2", "f16", "arg", "selection"),
])
def test_linalg_ext_attention_mask_rejects(pkg, mask_map, mask_type,
                                           mask_from, why):
    m = pkg.match(att_op(pkg, 64, mask=mask_map, mask_type=mask_type,
                         mask_from=mask_from))
    assert not m.taken and why in m.reason, m.reason


def test_malformed_descriptions_are_errors(pkg):
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["f16"] * 3, F16_BODY)
    op.map[0][1] = 7  # a loop past num_loops
    with pytest.raises(pkg.MI355XError):
        pkg.match(op)
    op = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"],
                 ["f16"] * 3, F16_BODY)
    op.body[0].operands[0] = 9  # a value not yet defined
    with pytest.raises(pkg.MI355XError):
        pkg.match(op)
    a = generic(pkg, "m n k", ["k"], ["m k", "k n", "m n"], ["f16"] * 3,
                F16_BODY)
    a.producer[0] = 0  # reads itself
    with pytest.raises(pkg.MI355XError):
        pkg.match_region([a])
