"""Column splits: a grid of 256x256 tiles that ends in a ragged round runs
as its whole rounds plus one round of half-size tiles, two launches on the
caller's stream (csrc/gemm.hip launch_column_split).

Each case runs at a shape the planner gives a column split and checks:
  - the planner's pick is that split;
  - the output is bit-identical to the head configuration run alone over
    the whole shape (every element is computed by one tile of either grid,
    in the same K order);
  - the output matches the oracle: int8 bit-exact, f16 within the
    fp16 parity bound (max|y - y_cpu| / max|y_cpu| <= 2e-3);
  - nothing outside the output view is written.
The column-indexed operands of the tail launch (B, C, the W8A16 scale, the
epilogue's bias and multiplier) start n_head columns on; the epilogue and
accumulate cases check that offset.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

FP16_BOUND = 2e-3

# 2048 x 9216: a head of 8192 columns (256 tiles of 256x256, one round of
# the 256 CUs) and a tail of 1024 columns (64 tiles of 256x128 or 128x256).
M, N, K = 2048, 9216, 256


def canary_out(shape, dtype, dev, fill):
    m, n = shape
    buf = torch.full((m + 2, n + 64), fill, dtype=dtype, device=dev)
    return buf, buf[1:m + 1, :n]


def check_canary(buf, m, n, fill):
    host = buf.cpu()
    inner = torch.zeros_like(host, dtype=torch.bool)
    inner[1:m + 1, :n] = True
    assert bool((host[~inner] == fill).all()), "write outside the output view"


def cfg_index(pkg, name):
    return next(c.index for c in pkg.mfma_configs() if c.name == name)


CASES = [
    ("f16_nn", "f16_nn_256x256x64_w2x4_s2_m16", "f16_nn_256x128x64_w2x4_s2_m16"),
    ("f16_tn", "f16_tn_256x256x64_w2x4_s2_m16", "f16_tn_256x128x64_w2x4_s2_m16"),
    ("f16_at", "f16at_nn_256x256x64_w2x4_s2_m16", "f16at_nn_256x128x64_w2x4_s2"),
    ("f16_at_tn", "f16at_tn_256x256x64_w2x4_s2_m16", "f16at_tn_256x128x64_w2x4_s2"),
    ("i8_tn", "i8_tn_256x256x128_w2x4_s2_m16", "i8_tn_256x128x128_w2x4_s2_m16"),
    ("i8_nn", "i8_nn_256x256x128_w2x4_s2_m16", "i8_nn_128x256x128_w2x4_s2"),
    ("w8a16", "w8a16_nn_256x256x64_w2x4_s3", "w8a16_nn_128x256x64_w2x4_s4"),
    ("f16f32_nn", "f16f32_nn_256x256x64_w2x4_s2_m16",
     "f16f32_nn_256x128x64_w2x4_s2_m16"),
    ("f16f32_tn", "f16f32_tn_256x256x64_w2x4_s2_m16",
     "f16f32_tn_256x128x64_w2x4_s2_m16"),
    ("f16f32_at", "f16f32at_nn_256x256x64_w2x4_s2_m16",
     "f16f32at_nn_256x128x64_w2x4_s2"),
    ("f16f32_at_tn", "f16f32at_tn_256x256x64_w2x4_s2_m16",
     "f16f32at_tn_256x128x64_w2x4_s2"),
]


@pytest.mark.parametrize("kind,head,tail", CASES)
def test_column_split_planned(pkg, oracle, dev, kind, head, tail):
    print(f"column split {kind} {M}x{N}x{K}", flush=True)
    g = torch.Generator().manual_seed(sum(map(ord, kind)))
    if kind.startswith("i8"):
        bt = kind == "i8_tn"
        a = torch.randint(-128, 128, (M, K), generator=g).to(torch.int8)
        b = torch.randint(-128, 128, (N, K) if bt else (K, N),
                          generator=g).to(torch.int8)
        desc = pkg.make_desc(pkg.ELEM_I8, pkg.ELEM_I8, pkg.ELEM_I32, M, N, K,
                             pkg.B_TRANSPOSED if bt else 0)
        fill, dt = -7, torch.int32
    elif kind == "w8a16":
        a = (torch.randn(M, K, generator=g) * 0.5).half()
        b = torch.randint(-128, 128, (K, N), generator=g).to(torch.int8)
        sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_I8, pkg.ELEM_F16, M, N, K,
                             0, has_scale=True)
        fill, dt = 3.0, torch.float16
    else:
        bt, at = kind.endswith("_tn"), "_at" in kind
        f32 = kind.startswith("f16f32")
        a = (torch.randn(*((K, M) if at else (M, K)), generator=g) * 0.5).half()
        b = (torch.randn(*((N, K) if bt else (K, N)), generator=g) * 0.5).half()
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16,
                             pkg.ELEM_F32 if f32 else pkg.ELEM_F16, M, N, K,
                             (pkg.B_TRANSPOSED if bt else 0) |
                             (pkg.A_TRANSPOSED if at else 0))
        fill, dt = 3.0, torch.float32 if f32 else torch.float16
    plan = pkg.plan(desc)
    # "<head>+<tail without the head's type and B form prefix>"
    pre = head[:head.index("_", head.index("_") + 1) + 1]
    assert plan.config_name.decode() == f"{head}+{tail[len(pre):]}"
    assert plan.workspace_bytes == 0
    ad, bd = a.to(dev), b.to(dev)
    buf, c = canary_out((M, N), dt, dev, fill)
    solo = torch.empty(M, N, dtype=dt, device=dev)
    if kind == "w8a16":
        scd = sc.to(dev)
        pkg.quantized_matmul(ad, bd, scd, c)
        pkg.matmul_mfma_config(cfg_index(pkg, head), ad, bd, solo, scale=scd)
        ref = oracle.w8a16(a.numpy(), b.numpy(), sc.numpy())
    elif kind.startswith("i8"):
        pkg.matmul(ad, bd, c, b_transposed=bt)
        pkg.matmul_mfma_config(cfg_index(pkg, head), ad, bd, solo)
        ref = oracle.matmul_i8(a.numpy(), b.numpy(), b_transposed=bt)
    else:
        pkg.matmul(ad, bd, c, b_transposed=bt, a_transposed=at,
                   out_dtype=dt)
        pkg.matmul_mfma_config(cfg_index(pkg, head), ad, bd, solo)
        ref = oracle.matmul_f16(a.numpy(), b.numpy(), b_transposed=bt,
                                a_transposed=at, out_f32=f32)
    torch.cuda.synchronize()
    check_canary(buf, M, N, fill)
    assert torch.equal(c, solo), "column split differs from its head alone"
    got = c.cpu().numpy()
    if kind.startswith("i8"):
        assert (got == ref).all()
    else:
        err = oracle.fp16_parity(got, ref)
        assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"


@pytest.mark.parametrize("act", [None, "gelu_tanh"])
def test_column_split_epilogue(pkg, oracle, dev, act):
    """One-matrix batch_matmul with bias, activation and multiplier: the
    tail grid reads bias and multiplier columns from n_head on."""
    print(f"column split epilogue act={act}", flush=True)
    g = torch.Generator().manual_seed(11)
    a = (torch.randn(1, M, K, generator=g) * 0.5).half()
    b = (torch.randn(K, N, generator=g) * 0.5).half()
    bias = torch.randn(N, generator=g).half()
    mul = torch.randn(1, M, N, generator=g).half()
    d = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16, pkg.ELEM_F16, M, N, K, 0)
    assert b"+" in pkg.plan(d).config_name
    y = pkg.batch_matmul(a.to(dev), b.to(dev), bias=bias.to(dev),
                         activation=act, multiplier=mul.to(dev))
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), bias=bias.numpy(),
                                  activation=pkg._ACT_NAMES[act],
                                  multiplier=mul.numpy())
    err = oracle.fp16_parity(y.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"


def test_column_split_accumulate(pkg, oracle, dev):
    """C += A.B through both grids (the tail reads C from n_head on)."""
    print("column split accumulate", flush=True)
    g = torch.Generator().manual_seed(12)
    a = (torch.randn(M, K, generator=g) * 0.5).half()
    b = (torch.randn(K, N, generator=g) * 0.5).half()
    c0 = torch.randn(M, N, generator=g).half()
    d = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16, pkg.ELEM_F16, M, N, K,
                      pkg.ACCUMULATE)
    assert b"+" in pkg.plan(d).config_name
    c = c0.to(dev)
    pkg.matmul(a.to(dev), b.to(dev), c, accumulate=True)
    ref = oracle.matmul_f16(a.numpy(), b.numpy(), c0.numpy())
    err = oracle.fp16_parity(c.cpu().numpy(), ref)
    assert err <= FP16_BOUND, f"fp16 parity {err:.3e}"
