"""Row-dot GEMV: skinny matmuls (M <= 4; W8A16 up to 16 in launches of up
to 8 rows) with the weights stored [N, K] (B_TRANSPOSED, a torch Linear's
layout), f16 and W8A16 (csrc/gemv.hip gemv_rowdot_kernel). One wave reduces
a whole row of W, so K is never split.

Bars: f16 and f32 results max|y - y_cpu| / max|y_cpu| <= 2e-3 (the
fp16 parity bound) against the oracle; nothing outside the output view is
written.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

FP16_BOUND = 2e-3


def canary_out(shape, dtype, dev, fill):
    m, n = shape
    buf = torch.full((m + 2, n + 64), fill, dtype=dtype, device=dev)
    return buf, buf[1:m + 1, :n]


def check_canary(buf, m, n, fill):
    host = buf.cpu()
    inner = torch.zeros_like(host, dtype=torch.bool)
    inner[1:m + 1, :n] = True
    assert bool((host[~inner] == fill).all()), "write outside the output view"


SHAPES = [(1, 11008, 4096), (1, 4096, 4096), (1, 4096, 11008),
          (2, 4096, 11008), (3, 11008, 4096), (4, 4096, 4096),
          (1, 1000, 1040), (4, 24, 16), (2, 1, 8192)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("kind", ["f16", "f16f32", "w8a16"])
def test_rowdot_planned(pkg, oracle, dev, kind, m, n, k):
    print(f"rowdot {kind} m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m * 131 + n + 7 * k)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    if kind == "w8a16":
        w = torch.randint(-128, 128, (n, k), generator=g).to(torch.int8)
        sc = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_I8, pkg.ELEM_F16, m, n, k,
                             pkg.B_TRANSPOSED, has_scale=True)
        dt = torch.float16
    else:
        w = (torch.randn(n, k, generator=g) * 0.5).half()
        f32 = kind == "f16f32"
        dt = torch.float32 if f32 else torch.float16
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16,
                             pkg.ELEM_F32 if f32 else pkg.ELEM_F16, m, n, k,
                             pkg.B_TRANSPOSED)
    plan = pkg.plan(desc)
    assert plan.config_name.decode() == f"gemv_rowdot_{kind}_r{m}"
    assert plan.workspace_bytes == 0
    buf, y = canary_out((m, n), dt, dev, 3.0)
    xd, wd = x.to(dev), w.to(dev)
    if kind == "w8a16":
        pkg.quantized_matmul(xd, wd, sc.to(dev), y, w_transposed=True)
        ref = oracle.w8a16(x.numpy(), w.numpy(), sc.numpy(), w_transposed=True)
    else:
        pkg.matmul(xd, wd, y, b_transposed=True, out_dtype=dt)
        ref = oracle.matmul_f16(x.numpy(), w.numpy(), b_transposed=True,
                                out_f32=dt == torch.float32)
    torch.cuda.synchronize()
    check_canary(buf, m, n, 3.0)
    err = oracle.fp16_parity(y.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"


@pytest.mark.parametrize("m,k", [(5, 4096), (8, 4096), (13, 4096),
                                 (16, 4096), (8, 2048), (3, 11008)])
def test_rowdot_w8a16_row_blocks(pkg, oracle, dev, m, k):
    """W8A16 with W [N, K] in launches of up to 8 rows of x and y, as many
    as x's LDS allows (7 at K = 4096, 8 at 2048, 2 at 11008), dealt
    evenly."""
    n = 2048
    print(f"rowdot w8a16 blocks m={m} k={k}", flush=True)
    g = torch.Generator().manual_seed(40 + m)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    w = torch.randint(-128, 128, (n, k), generator=g).to(torch.int8)
    sc = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
    d = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_I8, pkg.ELEM_F16, m, n, k,
                      pkg.B_TRANSPOSED, has_scale=True)
    assert pkg.plan(d).config_name.decode() == f"gemv_rowdot_w8a16_r{m}"
    buf, y = canary_out((m, n), torch.float16, dev, 3.0)
    pkg.quantized_matmul(x.to(dev), w.to(dev), sc.to(dev), y, w_transposed=True)
    ref = oracle.w8a16(x.numpy(), w.numpy(), sc.numpy(), w_transposed=True)
    torch.cuda.synchronize()
    check_canary(buf, m, n, 3.0)
    err = oracle.fp16_parity(y.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"


def test_rowdot_accumulate(pkg, oracle, dev):
    """C += x . W^T: each output is read once by the lane that stores it."""
    m, n, k = 3, 4096, 4096
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    w = (torch.randn(n, k, generator=g) * 0.5).half()
    c0 = torch.randn(m, n, generator=g).half()
    c = c0.to(dev)
    pkg.matmul(x.to(dev), w.to(dev), c, b_transposed=True, accumulate=True)
    ref = oracle.matmul_f16(x.numpy(), w.numpy(), c0.numpy(),
                            b_transposed=True)
    err = oracle.fp16_parity(c.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"


@pytest.mark.parametrize("shared_b", [False, True])
@pytest.mark.parametrize("act", [None, "silu"])
def test_rowdot_batched_epilogue(pkg, oracle, dev, shared_b, act):
    """batch_matmul with B [Z, N, K] (or one shared [N, K]), bias, an
    activation and a gating multiplier: batch z's rows of x, W and y, and
    the multiplier's rows, are offset by their batch strides."""
    z, m, n, k = 3, 2, 1536, 2048
    g = torch.Generator().manual_seed(22 + shared_b)
    a = (torch.randn(z, m, k, generator=g) * 0.5).half()
    b = (torch.randn(n, k, generator=g) if shared_b else
         torch.randn(z, n, k, generator=g)).half()
    bias = torch.randn(n, generator=g).half()
    mul = torch.randn(z, m, n, generator=g).half()
    d = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16, pkg.ELEM_F16, m, n, k,
                      pkg.B_TRANSPOSED, batch=z)
    assert pkg.plan(d).config_name.decode() == "gemv_rowdot_f16_r2"
    y = pkg.batch_matmul(a.to(dev), b.to(dev), b_transposed=True,
                         bias=bias.to(dev), activation=act,
                         multiplier=mul.to(dev))
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), b_transposed=True,
                                  bias=bias.numpy(),
                                  activation=pkg._ACT_NAMES[act],
                                  multiplier=mul.numpy())
    err = oracle.fp16_parity(y.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"
