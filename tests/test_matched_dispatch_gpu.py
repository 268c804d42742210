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
  * linalg.quantized_matmul with zero points 0.
"""
import numpy as np
import pytest
import torch

from test_matcher_cpu import (MIXED_BODY, ZERO_INIT, attention_chain, dequant,
                              fill, generic, named)

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
