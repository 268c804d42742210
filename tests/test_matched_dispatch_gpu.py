"""Matched regions run end to end: a dispatch region described as the
plugin sees it goes through the matcher, and what the match returns (the
export, its flags, its scale, the loops whose extents give the shape, an
init to fill) is all the dispatch through the executable-library table
uses. The result is checked against the oracle.

Regions (each as the reference writes it):
  * the decomposed attention of examples/attention_layer/
    attention_layer.mlir:48-105 (extensions, the two 128^-1/4 factors, a
    transpose of K, batch_matmul, row max, exp, row sum, divide, the
    all-masked guard, batch_matmul, truncation), with and without a causal
    mask generic;
  * a dequantization generic feeding a matmul (W8A16);
  * the transposed-B mixed-precision linalg.generic of
    plugins/compiler/hexagon/test/codegen/transforms/
    specialize_hmx_contractions.mlir:20-32 over a zero fill, over its
    argument init, and over a fill of 5.0 as in convert_matmul_to_hmx.mlir:
    40-55;
  * linalg.quantized_matmul with zero points 0;
  * iree_linalg_ext.attention ops the general kernel takes: the shapes of
    test/codegen/pipelines/hexagon_lower_executable_target.mlir:195-233 (Q
    1x2x4, K 1x3x4, V 1x3x5, scale 0.5, f32 result), unequal head dims with
    an f16 mask from a region argument broadcast over batch and heads, and
    the decomposed chain at head dim 96 with an f32 result.
"""
import numpy as np
import pytest
import torch

from test_matcher_cpu import (MIXED_BODY, ZERO_INIT, att_op, attention_chain,
                              dequant, fill, generic, named)

pytestmark = pytest.mark.gpu


def extent(op, loop):
    return int(op.loop_extent[loop])


def dispatch(pkg, name, constants, tensors, stream=None):
    """A plugin's dispatch: validate and size the workspace with a query,
    then run with a zeroed workspace of that size."""
    s = torch.cuda.current_stream().cuda_stream if stream is None else stream
    ptrs = [t.data_ptr() for t in tensors]
    lens = [t.numel() * t.element_size() for t in tensors]
    st, need = pkg.call_export(name, constants, ptrs, lens, s, query=True)
    assert st == pkg.OK, pkg.last_error()
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=tensors[0].device)
    st = pkg.call_export(name, constants, ptrs, lens, s,
                         workspace=ws.data_ptr() if need else None,
                         workspace_bytes=need)
    assert st == pkg.OK, pkg.last_error()
    torch.cuda.synchronize()


def fp16_ok(oracle, got, ref, bound=2e-3):
    err = oracle.fp16_parity(got, ref)
    assert err <= bound, err


@pytest.mark.parametrize("causal,head", [(False, 128), (True, 128),
                                         (True, 64)])
def test_attention_layer_region(pkg, oracle, dev, causal, head):
    batch, seq = 4, 512
    print(f"attention region causal={causal} head={head}", flush=True)
    ops = attention_chain(pkg, causal=causal, head=head, batch=batch, seq=seq)
    m = pkg.match_region(ops)
    assert m.taken and m.export == "attention_f16", m.reason
    pv = ops[m.root - 1]  # the truncation's producer: P . V
    b, s_q, d = (extent(pv, m.batch_loop), extent(pv, m.m_loop),
                 extent(pv, m.n_loop))
    s_kv = extent(pv, m.k_loop)
    assert (b, s_q, s_kv, d) == (batch, seq, seq, head)
    g = torch.Generator().manual_seed(head + causal)
    q, k, v = (torch.randn(b, 1, s_q, d, generator=g).half()
               for _ in range(3))
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    o = torch.empty_like(qd)
    # the region's batch dim is the kernel's batch, one head each
    dispatch(pkg, "attention_f16",
             pkg.attention_constants(b, 1, s_q, s_kv, d, m.scale, m.flags),
             [qd, kd, vd, o])
    got = o.cpu().numpy()
    # the region's scale is the product of its two factors, 128^-1/2, which
    # is 1/sqrt(d) only at d = 128
    assert abs(m.scale - 128 ** -0.5) < 1e-7
    ref = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(),
                               scale=m.scale, causal=causal)
    fp16_ok(oracle, got, ref)
    if head != 128:
        default = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(),
                                       causal=causal)
        assert oracle.fp16_parity(got, default) > 1e-2


def test_dequant_matmul_region(pkg, oracle, inputs, dev):
    m_, n_, k_ = 64, 1024, 512
    dq = dequant(pkg)
    mm = named(pkg, pkg.OP_MATMUL, "m n k", ["k"], ["m k", "k n", "m n"],
               ["f16", "f16", "f16"], {"m": m_, "n": n_, "k": k_},
               producers=["arg", 0, ZERO_INIT])
    m = pkg.match_region([dq, mm])
    assert m.taken and m.export == "w8a16_matmul", m.reason
    mm_op = [dq, mm][m.root]
    mm_, nn_, kk_ = (extent(mm_op, m.m_loop), extent(mm_op, m.n_loop),
                     extent(mm_op, m.k_loop))
    x, w, s = inputs.c5_w8a16(mm_, n=nn_, k=kk_)
    xd, wd, sd = x.to(dev), w.to(dev), s.to(dev)
    y = torch.empty(mm_, nn_, dtype=torch.float16, device=dev)
    dispatch(pkg, m.export,
             pkg.matmul_constants(mm_, nn_, kk_, kk_, nn_, nn_, m.flags),
             [xd, wd, sd, y])
    ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    fp16_ok(oracle, y.cpu().numpy(), ref)


@pytest.mark.parametrize("init", ["zero_fill", "argument", "fill_5"])
def test_transposed_b_generic_region(pkg, oracle, dev, init):
    m_, n_, k_ = 192, 256, 96
    ext = {"d0": m_, "d1": n_, "d2": k_}
    maps = ["d0 d2", "d1 d2", "d0 d1"]
    if init == "argument":
        ops = [generic(pkg, "d0 d1 d2", ["d2"], maps, ["f16", "f16", "f32"],
                       MIXED_BODY, ext)]
    else:
        value = 0.0 if init == "zero_fill" else 5.0
        ops = [fill(pkg, "d0 d1", "f32", value),
               generic(pkg, "d0 d1 d2", ["d2"], maps, ["f16", "f16", "f32"],
                       MIXED_BODY, ext, producers=["arg", "arg", 0])]
    m = pkg.match_region(ops)
    assert m.taken and m.export == "matmul_f16", m.reason
    assert m.flags & pkg.B_TRANSPOSED and m.flags & pkg.OUT_F32
    g = torch.Generator().manual_seed(7)
    a = torch.randn(m_, k_, generator=g).half()
    bt = torch.randn(n_, k_, generator=g).half()
    c0 = torch.randn(m_, n_, generator=g)
    c = c0.clone().to(dev)
    if m.init_fill:
        c.fill_(m.init_value)
    dispatch(pkg, m.export,
             pkg.matmul_constants(m_, n_, k_, k_, k_, n_, m.flags),
             [a.to(dev), bt.to(dev), c])
    prod = oracle.matmul_f16(a.numpy(), bt.numpy(), b_transposed=True,
                             out_f32=True)
    want = {"zero_fill": prod, "argument": prod + c0.numpy(),
            "fill_5": prod + np.float32(5.0)}[init]
    assert bool(m.flags & pkg.ACCUMULATE) == (init != "zero_fill")
    fp16_ok(oracle, c.cpu().numpy(), want, bound=1e-5)


def test_quantized_matmul_region(pkg, oracle, dev):
    m_, n_, k_ = 256, 512, 1024
    op = pkg.linalg_op(pkg.OP_QUANTIZED_MATMUL, "m n k",
                       ["m k", "n k", "", "", "m n"],
                       ["i8", "i8", "i32", "i32", "i32"], inputs=4,
                       reductions=["k"], extents={"m": m_, "n": n_, "k": k_},
                       producers=["arg", "arg", ("const", 0), ("const", 0),
                                  ZERO_INIT])
    m = pkg.match_region([op])
    assert m.taken and m.export == "matmul_i8", m.reason
    assert m.flags == pkg.B_TRANSPOSED
    g = torch.Generator().manual_seed(3)
    a = torch.randint(-128, 128, (m_, k_), generator=g).to(torch.int8)
    bt = torch.randint(-128, 128, (n_, k_), generator=g).to(torch.int8)
    c = torch.full((m_, n_), -1, dtype=torch.int32, device=dev)
    dispatch(pkg, m.export,
             pkg.matmul_constants(m_, n_, k_, k_, k_, n_, m.flags),
             [a.to(dev), bt.to(dev), c])
    ref = oracle.matmul_i8(a.numpy(), bt.numpy(), b_transposed=True)
    assert np.array_equal(c.cpu().numpy(), ref)


def mask_strides(op, index, m, sizes):
    """Element strides (batch, head, row, key) of a contiguous mask whose map
    selects some of the match's (batch, head, M, K2) loops; 0 where it
    broadcasts."""
    loops = [op.map[index][r] for r in range(op.map_rank[index])]
    strides, acc = {}, 1
    for l in reversed(loops):
        strides[l] = acc
        acc *= sizes[l]
    return [strides.get(l, 0) for l in (m.batch_loop, m.head_loop, m.m_loop,
                                        m.k_loop)]


@pytest.mark.parametrize("case", ["pipeline_fixture", "mask_rows",
                                  "mask_full_causal"])
def test_attention_op_general_region(pkg, oracle, dev, case):
    print(f"attention op {case}", flush=True)
    if case == "pipeline_fixture":
        op = att_op(pkg, 4, head_v=5, out="f32", batch_dims="b",
                    sizes={"b": 1, "m": 2, "k2": 3}, scale=0.5)
        mshape = None
    elif case == "mask_rows":
        op = att_op(pkg, 96, head_v=64, mask="m k2",
                    sizes={"b": 2, "h": 3, "m": 100, "k2": 150}, scale=0.1)
        mshape = (100, 150)
    else:
        op = att_op(pkg, 40, mask="b h m k2", out="f32",
                    sizes={"b": 1, "h": 2, "m": 64, "k2": 64}, scale=0.2)
        mshape = (1, 2, 64, 64)
    m = pkg.match_region([op])
    assert m.taken and m.export == "attention_f16", m.reason
    sizes = [int(x) for x in op.loop_extent[:op.num_loops]]
    b = sizes[m.batch_loop]
    h = sizes[m.head_loop] if m.head_loop >= 0 else 1
    sq, skv = sizes[m.m_loop], sizes[m.k_loop]
    d, dv = sizes[m.head_dim_loop], sizes[m.n_loop]
    out_f32 = bool(m.flags & pkg.ATTENTION_OUT_F32)
    causal = case == "mask_full_causal"
    flags = m.flags | (pkg.CAUSAL if causal else 0)
    g = torch.Generator().manual_seed(len(case))
    q = torch.randn(b, h, sq, d, generator=g).half()
    k = torch.randn(b, h, skv, d, generator=g).half()
    v = torch.randn(b, h, skv, dv, generator=g).half()
    o = torch.full((b, h, sq, dv), float("nan"),
                   dtype=torch.float32 if out_f32 else torch.float16)
    tensors = [q, k, v, o]
    ms = [0, 0, 0, 0]
    mask = None
    if mshape is not None:
        mask = (2 * torch.randn(*mshape, generator=g)).half()
        mask[torch.rand(*mshape, generator=g) < 0.2] = float("-inf")
        ms = mask_strides(op, 4, m, sizes)
        tensors.append(mask)
    dev_t = [t.to(dev) for t in tensors]
    dispatch(pkg, "attention_f16",
             pkg.attention_constants(b, h, sq, skv, d, m.scale, flags,
                                     head_dim_v=dv, mask_strides=ms),
             dev_t)
    got = dev_t[3].cpu().numpy()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=m.scale,
                           causal=causal, out_f32=out_f32,
                           mask=None if mask is None else mask.numpy())
    fp16_ok(oracle, got, ref, bound=4e-4 if out_f32 else 2e-3)


def test_attention_chain_head96_f32(pkg, oracle, dev):
    # the decomposed chain of attention_layer.mlir at head dim 96, without
    # its final truncation: an f32 result
    batch, seq, head = 2, 200, 96
    ops = attention_chain(pkg, head=head, batch=batch, seq=seq, out="f32")
    m = pkg.match_region(ops)
    assert m.taken and m.flags == pkg.ATTENTION_OUT_F32, m.reason
    pv = ops[m.root]
    d = extent(pv, m.head_dim_loop)
    assert d == extent(pv, m.n_loop) == head
    g = torch.Generator().manual_seed(96)
    q, k, v = (torch.randn(batch, 1, seq, head, generator=g).half()
               for _ in range(3))
    o = torch.empty(batch, 1, seq, head, dtype=torch.float32, device=dev)
    dispatch(pkg, "attention_f16",
             pkg.attention_constants(batch, 1, seq, seq, head, m.scale,
                                     m.flags, head_dim_v=head),
             [q.to(dev), k.to(dev), v.to(dev), o])
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), scale=m.scale,
                           out_f32=True)
    # the MFMA kernel takes head dim 96: f16 probabilities before PV
    fp16_ok(oracle, o.cpu().numpy(), ref, bound=4e-4)
