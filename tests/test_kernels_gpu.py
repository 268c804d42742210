"""Parity of the gfx950 kernels with the CPU oracle, through the C-ABI.

Bars: int8 -> i32 bit-exact; f16 max|y - y_cpu| / max|y_cpu| <= 2e-3 (the
BASELINE fp16 rule), plus the reference's allclose + relative-L2 recipe with
each micro model's tolerances (IT/stages/checking.py:46-132).
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

FP16_BOUND = 2e-3


def fp16_ok(oracle, got, ref, bound=FP16_BOUND):
    err = oracle.fp16_parity(got, ref)
    assert err <= bound, f"fp16 parity {err:.3e} > {bound}"
    return err


def canary_out(shape, dtype, dev, fill):
    """Output view inside a larger buffer whose margins hold `fill`."""
    m, n = shape
    pad = 64
    buf = torch.full((m + 2, n + pad), fill, dtype=dtype, device=dev)
    return buf, buf[1:m + 1, :n]


def check_canary(buf, m, n, fill):
    host = buf.cpu()
    inner = torch.zeros_like(host, dtype=torch.bool)
    inner[1:m + 1, :n] = True
    assert bool((host[~inner] == fill).all()), "write outside the output view"


# ------------------------------------------------------------ f16 matmul ----

def test_c1_matmul_f16(pkg, oracle, inputs, dev):
    a, b = inputs.c1_matmul_f16()
    c = pkg.matmul(a.to(dev), b.to(dev))
    ref = oracle.matmul_f16(a.numpy(), b.numpy())
    fp16_ok(oracle, c.cpu().numpy(), ref)
    rel, _, close = oracle.compare_arrays(ref, c.cpu().numpy(), 5e-2, 5e-3)
    assert close and rel < 0.05


@pytest.mark.parametrize("name", ["small_prime_17x19x23", "ragged_m_65x64x64",
                                  "ragged_n_64x65x64", "ragged_k_64x64x65",
                                  "square_32x32x32"])
@pytest.mark.parametrize("transposed", [False, True])
def test_matmul_f16_micro_models(pkg, oracle, dev, name, transposed):
    d = np.load(os.path.join(GOLDEN, f"matmul_{name}.npz"))
    atol, rtol, rel_l2 = d["tol"]
    a = torch.from_numpy(d["a"]).to(dev)
    b = torch.from_numpy(d["b"])
    if transposed:
        b = b.t().contiguous()
    m, n = d["expected"].shape
    buf, c = canary_out((m, n), torch.float32, dev, -7.0)
    pkg.matmul(a, b.to(dev), c, b_transposed=transposed,
               out_dtype=torch.float32)
    got = c.cpu().numpy()
    check_canary(buf, m, n, -7.0)
    rel, _, close = oracle.compare_arrays(d["expected"], got, atol, rtol)
    assert close and rel <= rel_l2
    fp16_ok(oracle, got, d["expected"], 1e-5)


@pytest.mark.parametrize("shape", [(256, 256, 64), (512, 512, 256),
                                   (512, 256, 1024), (256, 768, 512)])
def test_matmul_f16_tn_configs(pkg, oracle, dev, shape):
    m, n, k = shape
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn(m, k, generator=g).half()
    bt = torch.randn(n, k, generator=g).half()
    ref16 = oracle.matmul_f16(a.numpy(), bt.numpy(), b_transposed=True)
    ref32 = oracle.matmul_f16(a.numpy(), bt.numpy(), b_transposed=True,
                              out_f32=True)
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if (cfg.a_elem != pkg.ELEM_F16 or cfg.b_form != pkg.B_FORM_TN
                or cfg.a_transposed):
            continue
        if m % cfg.tile_m or n % cfg.tile_n or k % cfg.tile_k:
            continue
        out32 = cfg.c_elem == pkg.ELEM_F32
        c = torch.empty(m, n, dtype=torch.float32 if out32 else torch.float16,
                        device=dev)
        pkg.matmul_mfma_config(cfg.index, a.to(dev), bt.to(dev), c)
        fp16_ok(oracle, c.cpu().numpy(), ref32 if out32 else ref16)
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("shape", [(256, 256, 64), (512, 512, 256),
                                   (256, 768, 192)])
def test_matmul_f16_nn_configs(pkg, oracle, dev, shape):
    m, n, k = shape
    g = torch.Generator().manual_seed(7 * m + n + k)
    a = torch.randn(m, k, generator=g).half()
    b = torch.randn(k, n, generator=g).half()
    ref16 = oracle.matmul_f16(a.numpy(), b.numpy())
    ref32 = oracle.matmul_f16(a.numpy(), b.numpy(), out_f32=True)
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if cfg.b_form != pkg.B_FORM_NN or cfg.a_transposed:
            continue
        if m % cfg.tile_m or n % cfg.tile_n or k % cfg.tile_k:
            continue
        out32 = cfg.c_elem == pkg.ELEM_F32
        c = torch.empty(m, n, dtype=torch.float32 if out32 else torch.float16,
                        device=dev)
        pkg.matmul_mfma_config(cfg.index, a.to(dev), b.to(dev), c)
        fp16_ok(oracle, c.cpu().numpy(), ref32 if out32 else ref16)
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("shape", [(128, 256, 64), (256, 512, 256),
                                   (128, 768, 384)])
def test_w8a16_mfma_configs(pkg, oracle, dev, shape):
    m, n, k = shape
    g = torch.Generator().manual_seed(5 * m + n + k)
    x = torch.randn(m, k, generator=g).half()
    w = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
    s = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
    ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if cfg.b_form != pkg.B_FORM_W8A16:
            continue
        if m % cfg.tile_m or n % cfg.tile_n or k % cfg.tile_k:
            continue
        y = torch.empty(m, n, dtype=torch.float16, device=dev)
        pkg.matmul_mfma_config(cfg.index, x.to(dev), w.to(dev), y,
                               scale=s.to(dev))
        fp16_ok(oracle, y.cpu().numpy(), ref)
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("m,n,k,form", [
    (16, 4096, 4096, "nn"), (5, 512, 1024, "nn"), (100, 512, 768, "nn"),
    (128, 4096, 4096, "nn"), (37, 1024, 1024, "tn"), (64, 4096, 4096, "tn"),
    (16, 11008, 4096, "w8"), (37, 1024, 2048, "w8")])
def test_split_k_skinny(pkg, oracle, dev, m, n, k, form):
    """Split-K MFMA plans (ragged M, partials reduced in-kernel by the last
    workgroup of each tile); two calls in a row re-use the re-armed
    counters of the library workspace."""
    g = torch.Generator().manual_seed(m * 31 + n + k)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    if form == "w8":
        w = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
        s = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
        p = pkg.plan(pkg.make_desc(0, 1, 0, m, n, k, 0, has_scale=True))
        ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    else:
        w = (torch.randn(n, k, generator=g) if form == "tn" else
             torch.randn(k, n, generator=g)).half()
        flags = pkg.B_TRANSPOSED if form == "tn" else 0
        p = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, flags))
        ref = oracle.matmul_f16(x.numpy(), w.numpy(), b_transposed=form == "tn")
    assert p.family == pkg.FAMILY_MFMA and p.splits > 1, p.config_name
    for _ in range(2):
        buf, y = canary_out((m, n), torch.float16, dev, 5.0)
        if form == "w8":
            pkg.quantized_matmul(x.to(dev), w.to(dev), s.to(dev), y)
        else:
            pkg.matmul(x.to(dev), w.to(dev), y, b_transposed=form == "tn")
        fp16_ok(oracle, y.cpu().numpy(), ref)
        check_canary(buf, m, n, 5.0)


@pytest.mark.parametrize("cfg_name,m,n,k,form", [
    # C5 W8A16 M=512: 172 tiles of 64 K stages in runs of 43 (3 layers)
    ("w8a16_nn_128x256x64_w2x4_s4_sk", 512, 11008, 4096, "w8"),
    ("w8a16_nn_32x256x64_w1x4_s4_sk", 37, 2048, 2048, "w8"),  # ragged M
    ("f16_nn_64x128x64_w2x2_s4_sk", 200, 384, 1088, "nn"),    # 17 stages
    ("f16_nn_128x128x64_w2x2_s4_sk", 256, 4096, 4096, "nn"),
    ("f16_tn_128x128x64_w2x2_s4_sk", 128, 1024, 8192, "tn"),  # 32 runs a tile
    ("f16f32_nn_32x128x64_w1x4_s4_sk", 64, 1024, 1024, "f32"),
    ("f16_nn_64x128x64_w2x2_s4_sk", 1024, 2048, 4096, "nn"),  # one run a tile
])
def test_stream_k(pkg, oracle, dev, cfg_name, m, n, k, form):
    """Stream-K (each workgroup an equal run of the (tile, K stage) pairs;
    a tile spanning several runs is summed in K order by the last to
    arrive) against the oracle, two calls in a row (re-armed counters),
    with nothing written outside the output view."""
    cfg = next(c for c in pkg.mfma_configs() if c.name == cfg_name)
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    scale = None
    if form == "w8":
        w = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
        scale = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
        ref = oracle.w8a16(x.numpy(), w.numpy(), scale.numpy())
        scale = scale.to(dev)
    else:
        w = (torch.randn(n, k, generator=g) if form == "tn" else
             torch.randn(k, n, generator=g)).half()
        ref = oracle.matmul_f16(x.numpy(), w.numpy(), b_transposed=form == "tn",
                                out_f32=form == "f32")
    out_dtype = torch.float32 if form == "f32" else torch.float16
    xd, wd = x.to(dev), w.to(dev)
    for _ in range(2):
        buf, y = canary_out((m, n), out_dtype, dev, 5.0)
        pkg.matmul_mfma_config(cfg.index, xd, wd, y, scale=scale,
                               splits=pkg.SPLITS_STREAM_K)
        fp16_ok(oracle, y.cpu().numpy(), ref)
        check_canary(buf, m, n, 5.0)


def test_workspace_shared_across_kernels(pkg, oracle, dev):
    """GEMV and split-K GEMM calls of different shapes, interleaved on the
    library's one workspace: no call's partials may land on another call's
    arrival counters (regression: a GEMV's partials once overwrote the
    counters of split-K tiles past the 64th)."""
    g = torch.Generator().manual_seed(11)
    cases = [(1, 11008, 2048), (64, 8448, 2048), (3, 4096, 1024),
             (96, 8448, 2048), (1, 4096, 1024), (64, 11008, 2048),
             (2, 11008, 2048), (64, 8448, 2048)]
    for m, n, k in cases:
        p = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0))
        assert p.splits > 1 and (p.family == pkg.FAMILY_GEMV or
                                 p.workgroups // p.splits > 64), (m, n, k)
        x = (torch.randn(m, k, generator=g) * 0.5).half()
        w = torch.randn(k, n, generator=g).half()
        y = pkg.matmul(x.to(dev), w.to(dev))
        ref = oracle.matmul_f16(x.numpy(), w.numpy())
        fp16_ok(oracle, y.cpu().numpy(), ref)


def test_split_k_accumulate_f32(pkg, oracle, dev):
    g = torch.Generator().manual_seed(77)
    m, n, k = 24, 2048, 4096
    x = torch.randn(m, k, generator=g).half()
    w = torch.randn(k, n, generator=g).half()
    init = torch.randn(m, n, generator=g)
    p = pkg.plan(pkg.make_desc(0, 0, 3, m, n, k, pkg.ACCUMULATE | pkg.OUT_F32))
    assert p.splits > 1
    y = init.to(dev).clone()
    pkg.matmul(x.to(dev), w.to(dev), y, accumulate=True, out_dtype=torch.float32)
    ref = oracle.matmul_f16(x.numpy(), w.numpy(), init.numpy(), out_f32=True)
    fp16_ok(oracle, y.cpu().numpy(), ref)


def test_matmul_f16_accumulate(pkg, oracle, dev):
    g = torch.Generator().manual_seed(3)
    for m, n, k, bt in ((512, 512, 256, True), (100, 70, 90, False)):
        a = torch.randn(m, k, generator=g).half()
        b = torch.randn(n, k, generator=g).half() if bt else torch.randn(
            k, n, generator=g).half()
        init = torch.randn(m, n, generator=g)
        c = init.to(dev).clone()
        pkg.matmul(a.to(dev), b.to(dev), c, b_transposed=bt, accumulate=True,
                   out_dtype=torch.float32)
        ref = oracle.matmul_f16(a.numpy(), b.numpy(), init.numpy(),
                                b_transposed=bt, out_f32=True)
        fp16_ok(oracle, c.cpu().numpy(), ref)
        c16 = init.half().to(dev)
        pkg.matmul(a.to(dev), b.to(dev), c16, b_transposed=bt, accumulate=True)
        ref16 = oracle.matmul_f16(a.numpy(), b.numpy(), init.half().numpy(),
                                  b_transposed=bt)
        fp16_ok(oracle, c16.cpu().numpy(), ref16)


# The shapes of the reference's micro/hmx models (IT/models/micro/hmx/*):
# ragged-large, skinny, tall, wide, deep-K and the rhs-transposed square.
@pytest.mark.parametrize("m,n,k,bt", [(1537, 1539, 257, False),
                                      (1, 1024, 1024, False),
                                      (4096, 32, 256, False),
                                      (32, 4096, 256, False),
                                      (32, 32, 4096, False),
                                      (1024, 1024, 1024, True)])
def test_matmul_f16_reference_micro_shapes(pkg, oracle, dev, m, n, k, bt):
    g = torch.Generator().manual_seed(m * 7 + n * 3 + k)
    a = (torch.rand(m, k, generator=g) * 2 - 1).half()
    b = (torch.rand(*((n, k) if bt else (k, n)), generator=g) * 2 - 1).half()
    buf, c = canary_out((m, n), torch.float16, dev, 3.0)
    pkg.matmul(a.to(dev), b.to(dev), c, b_transposed=bt)
    check_canary(buf, m, n, 3.0)
    ref = oracle.matmul_f16(a.numpy(), b.numpy(), b_transposed=bt)
    fp16_ok(oracle, c.cpu().numpy(), ref)


# Every BASELINE C3 point: M in {1, 16, 128, 2048} x (N, K) in
# {(4096, 4096), (11008, 4096), (4096, 11008)}, each on the kernel the planner
# picks for it, compared over the whole output.
C3_POINTS = [(m, n, k) for m in (1, 16, 128, 2048)
             for n, k in ((4096, 4096), (11008, 4096), (4096, 11008))]


@pytest.mark.parametrize("m,n,k", C3_POINTS)
def test_c3_linear_sweep(pkg, oracle, inputs, dev, m, n, k):
    x, w = inputs.c3_linear_f16(m, n, k)
    print(f"c3 sweep m={m} n={n} k={k} plan="
          f"{pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).config_name.decode()}",
          flush=True)
    y = pkg.matmul(x.to(dev), w.to(dev))
    ref = oracle.matmul_f16(x.numpy(), w.numpy(),
                            threads=oracle.default_threads())
    fp16_ok(oracle, y.cpu().numpy(), ref)


def test_c3_linear_transposed_weights_full(pkg, oracle, inputs, dev):
    x, w = inputs.c3_linear_f16(2048, 4096, 4096)
    wt = w.t().contiguous()
    y = pkg.matmul(x.to(dev), wt.to(dev), b_transposed=True)
    ref = oracle.matmul_f16(x.numpy(), wt.numpy(), b_transposed=True)
    fp16_ok(oracle, y.cpu().numpy(), ref)


# ------------------------------------------------------------------ GEMV ----

@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 11008, 4096),
                                   (1, 4096, 11008), (2, 520, 1000),
                                   (4, 4096, 4096), (3, 8, 7), (1, 1024, 1024),
                                   (1, 2048, 4096), (3, 2048, 1000),
                                   (2, 11008, 4100), (4, 4096, 11008)])
def test_gemv_f16(pkg, oracle, dev, m, n, k):
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = (torch.randn(m, k, generator=g) * 0.02).half()
    w = (torch.randn(k, n, generator=g) * 0.02).half()
    assert pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).family == pkg.FAMILY_GEMV
    buf, y = canary_out((m, n), torch.float16, dev, 3.0)
    pkg.matmul(x.to(dev), w.to(dev), y)
    ref = oracle.matmul_f16(x.numpy(), w.numpy())
    check_canary(buf, m, n, 3.0)
    fp16_ok(oracle, y.cpu().numpy(), ref)
    # f32 output and accumulate through the same kernel
    init = torch.randn(m, n, generator=g)
    y32 = init.to(dev).clone()
    pkg.matmul(x.to(dev), w.to(dev), y32, accumulate=True,
               out_dtype=torch.float32)
    ref32 = oracle.matmul_f16(x.numpy(), w.numpy(), init.numpy(), out_f32=True)
    fp16_ok(oracle, y32.cpu().numpy(), ref32)


@pytest.mark.parametrize("m,n,k,w8,form", [
    (1, 4096, 4096, False, "_h2"),     # 16 column blocks x 16 splits
    (1, 11008, 4096, False, ""),       # the full-wave form keeps 242 groups
    (2, 1000, 3004, False, "_h2"),     # last split: a wave of 12 rows (8 + 4)
    (2, 1000, 3000, False, "_h2"),     # last split: a wave of 8 rows (8 + 0)
    (3, 1024, 3004, True, "_h2"),
    (1, 11008, 4096, True, "_h2"),
    (1, 4096, 100, False, "_h2"),      # one split: no partials at all
])
def test_gemv_lane_group_forms(pkg, oracle, dev, m, n, k, w8, form):
    """Both GEMV forms (a wave streams one row, or its two 32-lane halves
    stream runs of their own), including the last split's ragged runs, where
    the second half has fewer rows than the first or none."""
    g = torch.Generator().manual_seed(m * 13 + n + k)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    p = pkg.plan(pkg.make_desc(0, 1 if w8 else 0, 0, m, n, k, 0,
                               has_scale=w8))
    assert p.family == pkg.FAMILY_GEMV
    assert p.config_name.decode().endswith(f"_r{m}{form}"), p.config_name
    buf, y = canary_out((m, n), torch.float16, dev, 3.0)
    if w8:
        w = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
        s = (torch.rand(n, generator=g) * 0.01 + 0.001).half()
        pkg.quantized_matmul(x.to(dev), w.to(dev), s.to(dev), y)
        ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    else:
        w = (torch.randn(k, n, generator=g) * 0.05).half()
        pkg.matmul(x.to(dev), w.to(dev), y)
        ref = oracle.matmul_f16(x.numpy(), w.numpy())
    check_canary(buf, m, n, 3.0)
    fp16_ok(oracle, y.cpu().numpy(), ref)


def test_gemv_repeated_calls_rearm_counters(pkg, oracle, dev):
    g = torch.Generator().manual_seed(11)
    for n, k in ((4096, 4096), (2048, 8192), (4096, 4096), (512, 300)):
        x = torch.randn(1, k, generator=g).half()
        w = (torch.randn(k, n, generator=g) * 0.05).half()
        y = pkg.matmul(x.to(dev), w.to(dev))
        fp16_ok(oracle, y.cpu().numpy(), oracle.matmul_f16(x.numpy(), w.numpy()))


def test_gemv_caller_workspace(pkg, oracle, dev):
    lib = pkg.library()
    m, n, k = 1, 4096, 4096
    need = lib.iree_mi355x_matmul_workspace_bytes(m, n, k, 0)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(m, k, generator=g).half().to(dev)
    w = (torch.randn(k, n, generator=g) * 0.02).half().to(dev)
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    st = lib.iree_mi355x_matmul_f16(x.data_ptr(), w.data_ptr(), y.data_ptr(),
                                    m, n, k, k, n, n, 0, ws.data_ptr(), 16, s)
    assert st == pkg.WORKSPACE_TOO_SMALL
    for _ in range(2):
        st = lib.iree_mi355x_matmul_f16(x.data_ptr(), w.data_ptr(),
                                        y.data_ptr(), m, n, k, k, n, n, 0,
                                        ws.data_ptr(), need, s)
        assert st == pkg.OK
        ref = oracle.matmul_f16(x.cpu().numpy(), w.cpu().numpy())
        fp16_ok(oracle, y.cpu().numpy(), ref)


# ------------------------------------------------------------- int8 matmul --

def test_matmul_i8_golden(pkg, dev):
    d = np.load(os.path.join(GOLDEN, "matmul_i8.npz"))
    c = pkg.matmul(torch.from_numpy(d["a"]).to(dev),
                   torch.from_numpy(d["bt"]).to(dev), b_transposed=True)
    assert np.array_equal(c.cpu().numpy(), d["expected"])


@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 512, 512),
                                   (256, 1024, 384), (37, 768, 1024)])
@pytest.mark.parametrize("form", ["tn", "nn"])
def test_matmul_i8_configs(pkg, oracle, dev, shape, form):
    """Every int8 configuration of the B form (macro-tiles where the shape
    tiles, split-K tiles also at a ragged M), bit-exact, twice in a row
    (the split-K counters re-armed)."""
    m, n, k = shape
    tn = form == "tn"
    g = torch.Generator().manual_seed(m + 2 * n + k + tn)
    a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8)
    b = torch.randint(-128, 128, (n, k) if tn else (k, n),
                      generator=g).to(torch.int8)
    ref = oracle.matmul_i8(a.numpy(), b.numpy(), b_transposed=tn)
    want_form = pkg.B_FORM_TN if tn else pkg.B_FORM_NN8
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if cfg.a_elem != pkg.ELEM_I8 or cfg.b_form != want_form:
            continue
        split = "_sk" in cfg.name
        if (not split and m % cfg.tile_m) or n % cfg.tile_n or k % cfg.tile_k:
            continue
        for _ in range(2):
            buf, c = canary_out((m, n), torch.int32, dev, 12345)
            pkg.matmul_mfma_config(cfg.index, a.to(dev), b.to(dev), c)
            assert np.array_equal(c.cpu().numpy(), ref), cfg.name
            check_canary(buf, m, n, 12345)
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("m,n,k,bt", [(17, 19, 23, False), (65, 64, 64, True),
                                      (100, 130, 257, False), (1, 4096, 4096, False),
                                      (33, 70, 129, True)])
def test_matmul_i8_general(pkg, oracle, dev, m, n, k, bt):
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8)
    b = torch.randint(-128, 128, (n, k) if bt else (k, n), generator=g).to(torch.int8)
    init = torch.randint(-10 ** 6, 10 ** 6, (m, n), generator=g, dtype=torch.int32)
    buf, c = canary_out((m, n), torch.int32, dev, 12345)
    c.copy_(init.to(dev))
    pkg.matmul(a.to(dev), b.to(dev), c, b_transposed=bt, accumulate=True)
    ref = oracle.matmul_i8(a.numpy(), b.numpy(), init.numpy(), b_transposed=bt)
    assert np.array_equal(c.cpu().numpy(), ref)
    check_canary(buf, m, n, 12345)


def test_fast_tiles_accumulate_and_odd_pitch(pkg, oracle, dev):
    """Every unsplit int8 / f16 macro-tile (not W8A16) through its two
    per-element epilogue paths: C += A.B into a contiguous C, and a plain
    store into a C view whose row pitch is not a multiple of 16 bytes.
    The 16x16 tiles store transposed fragments; this covers their
    non-vector paths, which the 4096^3 and sweep shapes do not reach."""
    m, n, k = 256, 256, 128
    g = torch.Generator().manual_seed(77)
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if "_sk" in cfg.name or cfg.b_form == pkg.B_FORM_W8A16:
            continue
        if m % cfg.tile_m or n % cfg.tile_n or k % cfg.tile_k:
            continue
        i8 = cfg.a_elem == pkg.ELEM_I8
        tn = cfg.b_form == pkg.B_FORM_TN
        if i8:
            a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8)
            b = torch.randint(-128, 128, (n, k) if tn else (k, n),
                              generator=g).to(torch.int8)
            cdt = torch.int32
            init = torch.randint(-10 ** 6, 10 ** 6, (m, n), generator=g,
                                 dtype=torch.int32)
            ref_acc = oracle.matmul_i8(a.numpy(), b.numpy(), init.numpy(),
                                       b_transposed=tn)
            ref = oracle.matmul_i8(a.numpy(), b.numpy(), b_transposed=tn)
        else:
            a = torch.randn(*((k, m) if cfg.a_transposed else (m, k)),
                            generator=g).half()
            b = torch.randn(*((n, k) if tn else (k, n)), generator=g).half()
            f32 = cfg.c_elem == pkg.ELEM_F32
            cdt = torch.float32 if f32 else torch.float16
            init = torch.randn(m, n, generator=g).to(cdt)
            kw = dict(b_transposed=tn, a_transposed=bool(cfg.a_transposed),
                      out_f32=f32)
            ref_acc = oracle.matmul_f16(a.numpy(), b.numpy(), init.numpy(), **kw)
            ref = oracle.matmul_f16(a.numpy(), b.numpy(), **kw)
        ad, bd = a.to(dev), b.to(dev)
        c = init.to(dev).clone()
        pkg.matmul_mfma_config(cfg.index, ad, bd, c, accumulate=True)
        # odd pitch: one element past n, inside a canary-filled buffer
        fill = 12345 if i8 else 3.0
        buf = torch.full((m, n + 1), fill, dtype=cdt, device=dev)
        cv = buf[:, :n]
        pkg.matmul_mfma_config(cfg.index, ad, bd, cv)
        got_acc, got = c.cpu().numpy(), cv.cpu().numpy()
        if i8:
            assert np.array_equal(got_acc, ref_acc), cfg.name
            assert np.array_equal(got, ref), cfg.name
        else:
            fp16_ok(oracle, got_acc, ref_acc)
            fp16_ok(oracle, got, ref)
        assert bool((buf[:, n].cpu() == fill).all()), cfg.name
        ran += 1
    assert ran >= 8


def test_matmul_i8_nn_4096_bit_exact(pkg, oracle, inputs, dev):
    """C2's operands with B row-major ([K, N], linalg.matmul's default map):
    a row-major int8 macro-tile, bit-exact."""
    a, bt = inputs.c2_matmul_i8()
    b = bt.t().contiguous()
    p = pkg.plan(pkg.make_desc(pkg.ELEM_I8, pkg.ELEM_I8, pkg.ELEM_I32, 4096,
                               4096, 4096, 0))
    assert p.config_name.startswith(b"i8_nn_"), p.config_name
    c = pkg.matmul(a.to(dev), b.to(dev))
    got = c.cpu().numpy()
    row_sums = a.numpy().astype(np.int64) @ b.numpy().astype(np.int64).sum(1)
    assert np.array_equal(got.astype(np.int64).sum(1), row_sums)
    ref = oracle.matmul_i8(a.numpy(), bt.numpy(), b_transposed=True)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("m", [1, 16, 128])
@pytest.mark.parametrize("bt", [False, True])
def test_matmul_i8_skinny(pkg, oracle, dev, m, bt):
    """Skinny int8 at N = K = 4096 through the planner: a split-K MFMA tile
    (never the general kernel), bit-exact, with the C-ABI's workspace from
    the wrapper; twice, so the re-armed counters are reused."""
    n = k = 4096
    p = pkg.plan(pkg.make_desc(pkg.ELEM_I8, pkg.ELEM_I8, pkg.ELEM_I32, m, n,
                               k, pkg.B_TRANSPOSED if bt else 0))
    assert p.family == pkg.FAMILY_MFMA, p.config_name
    g = torch.Generator().manual_seed(m + bt)
    a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8)
    b = torch.randint(-128, 128, (n, k) if bt else (k, n),
                      generator=g).to(torch.int8)
    ref = oracle.matmul_i8(a.numpy(), b.numpy(), b_transposed=bt)
    ad, bd = a.to(dev), b.to(dev)
    for _ in range(2):
        buf, c = canary_out((m, n), torch.int32, dev, -5)
        pkg.matmul(ad, bd, c, b_transposed=bt)
        assert np.array_equal(c.cpu().numpy(), ref)
        check_canary(buf, m, n, -5)


def test_c2_matmul_i8_4096_bit_exact(pkg, oracle, inputs, dev):
    a, bt = inputs.c2_matmul_i8()
    c = pkg.matmul(a.to(dev), bt.to(dev), b_transposed=True)
    got = c.cpu().numpy()
    # size-independent check first: row sums = A . (sum of B rows), in int64
    row_sums = a.numpy().astype(np.int64) @ bt.numpy().astype(np.int64).sum(0)
    assert np.array_equal(got.astype(np.int64).sum(1), row_sums)
    ref = oracle.matmul_i8(a.numpy(), bt.numpy(), b_transposed=True)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ W8A16 ---

@pytest.mark.parametrize("m", [1, 4])
def test_c5_w8a16_gemv(pkg, oracle, inputs, dev, m):
    x, w, s = inputs.c5_w8a16(m)
    y = pkg.quantized_matmul(x.to(dev), w.to(dev), s.to(dev))
    ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    fp16_ok(oracle, y.cpu().numpy(), ref)


@pytest.mark.parametrize("m,transposed", [(512, False), (37, True), (5, False)])
def test_w8a16_general(pkg, oracle, inputs, dev, m, transposed):
    x, w, s = inputs.c5_w8a16(m, n=1100 if m != 512 else 11008, k=4096)
    if transposed:
        w = w.t().contiguous()
    y = pkg.quantized_matmul(x.to(dev), w.to(dev), s.to(dev),
                             w_transposed=transposed)
    ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy(),
                       w_transposed=transposed, threads=oracle.default_threads())
    fp16_ok(oracle, y.cpu().numpy(), ref)


# -------------------------------------------------------------- attention ---

@pytest.mark.parametrize("name", ["b1h2s128d64_causal", "b1h2s128d64",
                                  "b1h1s160d128_causal"])
def test_attention_golden(pkg, oracle, dev, name):
    d = np.load(os.path.join(GOLDEN, f"attention_{name}.npz"))
    q, k, v = (torch.from_numpy(d[x]).to(dev) for x in ("q", "k", "v"))
    o = pkg.attention(q, k, v, causal=bool(d["causal"]))
    got = o.cpu().numpy()
    atol, rtol, rel_l2 = d["tol"]
    rel, _, close = oracle.compare_arrays(d["expected"], got, atol, rtol)
    assert close and rel <= rel_l2
    fp16_ok(oracle, got, d["expected"])


@pytest.mark.parametrize("shape,causal", [((1, 4, 512, 128), True),
                                          ((2, 3, 200, 64), False),
                                          ((1, 2, 333, 128), True),
                                          ((4, 1, 1024, 128), False)])
def test_attention_vs_oracle(pkg, oracle, dev, shape, causal):
    g = torch.Generator().manual_seed(sum(shape))
    q, k, v = (torch.randn(shape, generator=g).half() for _ in range(3))
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=causal)
    ref = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), causal=causal)
    fp16_ok(oracle, o.cpu().numpy(), ref)


def test_c4_attention_full(pkg, oracle, inputs, dev):
    q, k, v = inputs.c4_attention_f16()
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=True)
    got = o.cpu().numpy()
    # query 0 attends only key 0
    assert np.array_equal(got[:, :, 0], v.numpy()[:, :, 0])
    ref = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), causal=True)
    fp16_ok(oracle, got, ref)


# Sequence lengths that differ (seq_q against seq_kv, both ways, a single
# query row) and scales other than 1/sqrt(d): the product of
# attention_layer.mlir's two 128^-1/4 factors at d = 64, 0.5, 0.297.
@pytest.mark.parametrize("sq,skv,d,causal,scale", [
    (128, 2048, 128, True, 0.297), (128, 2048, 128, False, 0.5),
    (1, 2048, 128, True, 0.297), (1, 2048, 64, False, 0.5),
    (2048, 128, 128, True, 0.5), (300, 1000, 64, True,
                                  0.29730177875068026 ** 2),
    (1000, 300, 64, False, 0.297), (64, 64, 128, True, 0.5),
    # scale <= 0 takes the kernel's masked-scaling softmax on every block
    (200, 300, 64, False, -0.3), (100, 100, 128, True, 0.0)])
def test_attention_lengths_and_scales(pkg, oracle, dev, sq, skv, d, causal,
                                      scale):
    print(f"attention sq={sq} skv={skv} d={d} causal={causal} "
          f"scale={scale}", flush=True)
    g = torch.Generator().manual_seed(sq + 7 * skv + d)
    q = torch.randn(1, 4, sq, d, generator=g).half()
    k = torch.randn(1, 4, skv, d, generator=g).half()
    v = torch.randn(1, 4, skv, d, generator=g).half()
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                      scale=scale)
    got = o.cpu().numpy()
    ref = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), scale=scale,
                               causal=causal)
    fp16_ok(oracle, got, ref)
    if causal:
        # query 0 sees key 0 only, whatever the scale
        assert np.array_equal(got[:, :, 0], v.numpy()[:, :, 0])
    elif abs(scale - d ** -0.5) > 1e-2:
        # the scale reached the kernel: the default one gives another answer
        other = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(),
                                     causal=causal)
        assert oracle.fp16_parity(got, other) > 1e-2


def test_attention_cache_slice_model(pkg, oracle, dev):
    # integration_tests/models/micro/attention-cache-slice-f16: 9 query heads
    # over 3 KV heads, the first 64 of 128 cache rows, output [B, S, H, D],
    # against its golden under its model.yaml tolerances
    d = np.load(os.path.join(GOLDEN, "attention_cache_slice.npz"))
    ctx = int(d["context"])
    q = torch.from_numpy(d["q"]).to(dev)
    kc = torch.from_numpy(d["k_cache"]).to(dev)
    vc = torch.from_numpy(d["v_cache"]).to(dev)
    b, hq, sq, dim = q.shape
    out = torch.full((b, sq, hq, dim), float("nan"), dtype=torch.float16,
                     device=dev)
    pkg.attention(q, kc[:, :, :ctx], vc[:, :, :ctx], out.permute(0, 2, 1, 3),
                  causal=False)
    got = out.cpu().numpy()
    atol, rtol, rel_l2 = d["tol"]
    for key in ("expected", "expected_f32"):
        rel, _, close = oracle.compare_arrays(d[key], got, atol, rtol)
        assert close and rel <= rel_l2, (key, rel)
    fp16_ok(oracle, got, d["expected_f32"])


@pytest.mark.parametrize("hq,hkv,s,dim,causal", [(16, 4, 1024, 128, True),
                                                 (8, 1, 700, 64, False),
                                                 (6, 3, 1, 128, True)])
def test_attention_grouped_strided(pkg, oracle, dev, hq, hkv, s, dim, causal):
    # K / V: the first s rows of a cache twice as long; Q read from and O
    # written to [B, S, H, D] buffers
    print(f"gqa hq={hq} hkv={hkv} s={s} d={dim} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(hq * 100 + hkv + s)
    q_bshd = torch.randn(2, s, hq, dim, generator=g).half()
    kc = torch.randn(2, hkv, 2 * s, dim, generator=g).half()
    vc = torch.randn(2, hkv, 2 * s, dim, generator=g).half()
    q_d, kc_d, vc_d = q_bshd.to(dev), kc.to(dev), vc.to(dev)
    out = torch.full((2, s, hq, dim), float("nan"), dtype=torch.float16,
                     device=dev)
    pkg.attention(q_d.permute(0, 2, 1, 3), kc_d[:, :, :s], vc_d[:, :, :s],
                  out.permute(0, 2, 1, 3), causal=causal)
    got = out.permute(0, 2, 1, 3).cpu().numpy()
    ref = oracle.attention_f16(q_bshd.numpy().transpose(0, 2, 1, 3),
                               kc.numpy()[:, :, :s], vc.numpy()[:, :, :s],
                               causal=causal)
    fp16_ok(oracle, got, ref)


def test_attention_strided_argument_checks(pkg, dev):
    q = torch.zeros(1, 4, 64, 64, dtype=torch.float16, device=dev)
    k = torch.zeros(1, 3, 64, 64, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="dividing"):
        pkg.attention(q, k, k)  # 4 query heads over 3 KV heads
    st = pkg.AttentionStrides()
    for f, t in (("q", q), ("k", k), ("v", k), ("o", q)):
        getattr(st, f)[:] = list(t.stride()[:3])
    assert pkg.library().iree_mi355x_attention_f16_strided(
        q.data_ptr(), k.data_ptr(), k.data_ptr(), q.data_ptr(), 1, 4, 3, 64,
        64, 64, 0.125, 0, ctypes.byref(st), None) == pkg.INVALID_ARGUMENT
    kc = torch.zeros(1, 2, 64, 68, dtype=torch.float16, device=dev)
    with pytest.raises(pkg.MI355XError) as e:
        pkg.attention(q, kc[..., :64], kc[..., :64])  # row pitch 68
    assert e.value.status == pkg.MISALIGNED


# ------------------------------------------------------ executable library --

def test_dispatch_through_export_table(pkg, oracle, dev):
    g = torch.Generator().manual_seed(21)
    m, n, k = 256, 512, 128
    a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8).to(dev)
    bt = torch.randint(-128, 128, (n, k), generator=g).to(torch.int8).to(dev)
    c = torch.zeros(m, n, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    st = pkg.call_export(
        "matmul_i8", pkg.matmul_constants(m, n, k, k, k, n, pkg.B_TRANSPOSED),
        [a.data_ptr(), bt.data_ptr(), c.data_ptr()],
        [a.numel(), bt.numel(), c.numel() * 4], s)
    assert st == pkg.OK, pkg.last_error()
    ref = oracle.matmul_i8(a.cpu().numpy(), bt.cpu().numpy(), b_transposed=True)
    assert np.array_equal(c.cpu().numpy(), ref)
    q, kk, v = (torch.randn(1, 2, 128, 64, generator=g).half().to(dev)
                for _ in range(3))
    o = torch.empty_like(q)
    nbytes = q.numel() * 2
    st = pkg.call_export("attention_f16",
                         pkg.attention_constants(1, 2, 128, 128, 64, 0.125, 1),
                         [q.data_ptr(), kk.data_ptr(), v.data_ptr(), o.data_ptr()],
                         [nbytes] * 4, s)
    assert st == pkg.OK, pkg.last_error()
    ref = oracle.attention_f16(q.cpu().numpy(), kk.cpu().numpy(),
                               v.cpu().numpy(), scale=0.125, causal=True)
    fp16_ok(oracle, o.cpu().numpy(), ref)
    # the strided, grouped form: 4 query heads over 2 KV heads, K / V the
    # first 96 rows of 160-row caches, O written [B, S, H, D]
    q4 = torch.randn(1, 4, 128, 64, generator=g).half().to(dev)
    kc, vc = (torch.randn(1, 2, 160, 64, generator=g).half().to(dev)
              for _ in range(2))
    o4 = torch.zeros(1, 128, 4, 64, dtype=torch.float16, device=dev)
    o4v = o4.permute(0, 2, 1, 3)
    strides = (list(q4.stride()[:3]) + list(kc.stride()[:3]) +
               list(vc.stride()[:3]) + list(o4v.stride()[:3]))
    consts = pkg.attention_constants(1, 4, 128, 96, 64, 0.5, 0, kv_heads=2,
                                     strides=strides)
    assert len(consts) == 32
    ptrs = [q4.data_ptr(), kc.data_ptr(), vc.data_ptr(), o4.data_ptr()]
    lens = [q4.numel() * 2, kc.numel() * 2, vc.numel() * 2, o4.numel() * 2]
    # K is read up to the end of row 95 of KV head 1: a binding of that many
    # bytes is enough, two bytes fewer is refused before launch
    k_reach = ((2 - 1) * kc.stride(1) + 95 * kc.stride(2) + 64) * 2
    assert k_reach == 32768 < lens[1]
    st = pkg.call_export("attention_f16", consts, ptrs,
                         [lens[0], k_reach - 2] + lens[2:], s)
    assert st == pkg.INVALID_ARGUMENT
    lens[1] = k_reach
    st = pkg.call_export("attention_f16", consts, ptrs, lens, s)
    assert st == pkg.OK, pkg.last_error()
    ref = oracle.attention_f16(q4.cpu().numpy(), kc.cpu().numpy()[:, :, :96],
                               vc.cpu().numpy()[:, :, :96], scale=0.5,
                               causal=False)
    fp16_ok(oracle, o4v.cpu().numpy(), ref)
    # batched matmul with a SiLU-gated epilogue through the export table
    z, m, n, k = 3, 64, 256, 128
    a = (torch.randn(z, m, k, generator=g) * 0.5).half()
    b = torch.randn(z, k, n, generator=g).half()
    bias = torch.randn(n, generator=g).half()
    mul = torch.randn(z, m, n, generator=g).half()
    a_d, b_d, bias_d, mul_d = (t.to(dev) for t in (a, b, bias, mul))
    y = torch.empty(z, m, n, dtype=torch.float16, device=dev)
    st = pkg.call_export(
        "batch_matmul_f16",
        pkg.batch_matmul_constants(m, n, k, k, n, n, 0, z, m * k, k * n, m * n,
                                   pkg.ACT_SILU, True, True, n, m * n),
        [a_d.data_ptr(), b_d.data_ptr(), y.data_ptr(), bias_d.data_ptr(),
         mul_d.data_ptr()],
        [a.numel() * 2, b.numel() * 2, y.numel() * 2, n * 2, mul.numel() * 2], s)
    assert st == pkg.OK, pkg.last_error()
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), bias=bias.numpy(),
                                  activation=3, multiplier=mul.numpy())
    fp16_ok(oracle, y.cpu().numpy(), ref)
    # a multiplier binding one byte short is rejected before launch
    st = pkg.call_export(
        "batch_matmul_f16",
        pkg.batch_matmul_constants(m, n, k, k, n, n, 0, z, m * k, k * n, m * n,
                                   pkg.ACT_SILU, True, True, n, m * n),
        [a_d.data_ptr(), b_d.data_ptr(), y.data_ptr(), bias_d.data_ptr(),
         mul_d.data_ptr()],
        [a.numel() * 2, b.numel() * 2, y.numel() * 2, n * 2, mul.numel() * 2 - 1], s)
    assert st == pkg.INVALID_ARGUMENT


# --------------------------------------------- batch matmul + epilogue ----

def test_batch_matmul_reference_micro_model(pkg, oracle, dev):
    """IT/models/micro/hmx/batch-matmul-4x1024x1024x128-f16: a [4,1024,128],
    b [4,128,1024] normal seeds 0/1, f32 result, the model's tolerances."""
    a = torch.randn(4, 1024, 128, generator=torch.Generator().manual_seed(0)).half()
    b = torch.randn(4, 128, 1024, generator=torch.Generator().manual_seed(1)).half()
    c = pkg.batch_matmul(a.to(dev), b.to(dev), out_dtype=torch.float32)
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), out_f32=True)
    got = c.cpu().numpy()
    rel, _, close = oracle.compare_arrays(ref, got, 1.5e-1, 5.0e-3)
    assert close and rel <= 0.05
    fp16_ok(oracle, got, ref)


@pytest.mark.parametrize("z,m,n,k,bt,shared_b", [
    (3, 1, 4096, 1024, False, True),     # GEMV, shared weights
    (2, 4, 2048, 512, False, False),     # GEMV, 4 rows
    (4, 16, 2048, 1024, False, True),    # split-K skinny
    (2, 100, 512, 768, False, False),    # split-K ragged M
    (2, 256, 512, 256, True, False),     # macro-tile TN
    (3, 256, 256, 512, False, True),     # macro-tile NN, shared B
    (2, 17, 19, 23, True, False),        # general kernel
    (16, 16, 2048, 512, False, True),    # ragged M, one split per tile
])
@pytest.mark.parametrize("act", [None, "relu", "gelu_tanh", "silu"])
def test_batch_matmul_epilogue_paths(pkg, oracle, dev, z, m, n, k, bt, shared_b, act):
    g = torch.Generator().manual_seed(z * 1000 + m * 7 + n + k)
    a = (torch.randn(z, m, k, generator=g) * 0.5).half()
    bshape = (n, k) if bt else (k, n)
    b = (torch.randn(*bshape, generator=g) if shared_b else
         torch.randn(z, *bshape, generator=g)).half()
    bias = torch.randn(n, generator=g).half()
    mul = torch.randn(z, m, n, generator=g).half()
    y = pkg.batch_matmul(a.to(dev), b.to(dev), b_transposed=bt, bias=bias.to(dev),
                         activation=act, multiplier=mul.to(dev))
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), b_transposed=bt,
                                  bias=bias.numpy(),
                                  activation=pkg._ACT_NAMES[act],
                                  multiplier=mul.numpy())
    fp16_ok(oracle, y.cpu().numpy(), ref)


@pytest.mark.parametrize("m,n,k", [(192, 11008, 11008), (128, 11008, 4096)])
def test_stream_k_planned(pkg, oracle, dev, m, n, k):
    """Shapes the planner runs in stream-K (measured entries; the second is
    BASELINE's C5 W8A16 M=128), through the quantized_matmul entry point,
    whole outputs, twice in a row (re-armed counters)."""
    assert pkg.plan(pkg.make_desc(0, 1, 0, m, n, k, 0,
                                  has_scale=True)).stream_k_steps > 0
    g = torch.Generator().manual_seed(m)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    w = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
    s = (torch.rand(n, generator=g) * 0.019 + 0.001).half()
    ref = oracle.w8a16(x.numpy(), w.numpy(), s.numpy())
    xd, wd, sd = x.to(dev), w.to(dev), s.to(dev)
    for _ in range(2):
        buf, y = canary_out((m, n), torch.float16, dev, 5.0)
        pkg.quantized_matmul(xd, wd, sd, y)
        fp16_ok(oracle, y.cpu().numpy(), ref)
        check_canary(buf, m, n, 5.0)


def test_batch_matmul_accumulate_f32_and_strided_batches(pkg, oracle, dev):
    """Accumulate into an f32 init, with A and C views whose batch stride is
    larger than a matrix (every batch still separate)."""
    g = torch.Generator().manual_seed(41)
    z, m, n, k = 3, 64, 256, 128
    abig = (torch.randn(z, m + 8, k, generator=g) * 0.5).half()
    a = abig[:, :m, :]
    b = torch.randn(z, k, n, generator=g).half()
    init = torch.randn(z, m, n, generator=g)
    cbig = torch.zeros(z, m + 4, n)
    cbig[:, :m, :] = init
    c_d = cbig.to(dev)
    pkg.batch_matmul(abig.to(dev)[:, :m, :], b.to(dev),
                     c_d[:, :m, :], accumulate=True, out_dtype=torch.float32,
                     bias=torch.ones(n, dtype=torch.float16, device=dev),
                     activation="relu")
    ref = oracle.batch_matmul_f16(a.contiguous().numpy(), b.numpy(),
                                  init.numpy(), out_f32=True,
                                  bias=np.ones(n, np.float16), activation=1)
    fp16_ok(oracle, c_d[:, :m, :].cpu().numpy(), ref)
    assert bool((c_d[:, m:, :] == 0).all().item()), "write outside the batches"


def test_geglu_epilogue_reference_shape(pkg, oracle, dev):
    """The reference's fused-epilogue test dispatch
    (hexagon_hmx_epilogue_keeps_config.mlir): x [1,256] . W^T, W [2048,256],
    tanh-GELU, gated by up [1,2048]. Checked against the f32 oracle and the
    reference IR's f16-per-op form."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1, 256, generator=g)).half()
    w = (torch.randn(2048, 256, generator=g) * 0.1).half()
    up = torch.randn(1, 2048, generator=g).half()
    y = pkg.linear(x.to(dev), w.to(dev), activation="gelu_tanh",
                   multiplier=up.to(dev), w_transposed=True)
    got = y.cpu().numpy()
    ref32 = oracle.batch_matmul_f16(x.numpy()[None], w.numpy(), b_transposed=True,
                                    activation=2, multiplier=up.numpy())[0]
    fp16_ok(oracle, got, ref32)
    acc = oracle.matmul_f16(x.numpy(), w.numpy(), b_transposed=True, out_f32=True)
    ref16 = oracle.geglu_f16_ops(acc, up.numpy()).reshape(1, 2048)
    fp16_ok(oracle, got, ref16.astype(np.float32))


def test_batch_matmul_argument_errors(pkg, dev):
    a = torch.zeros(2, 8, 8, dtype=torch.float16, device=dev)
    b = torch.zeros(2, 8, 8, dtype=torch.float16, device=dev)
    lib = pkg.library()
    c = torch.zeros(2, 8, 8, dtype=torch.float16, device=dev)
    # stride_c 0 with two batches would write both into one matrix
    st = lib.iree_mi355x_batch_matmul_f16(a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                          2, 8, 8, 8, 8, 8, 8, 64, 64, 0, 0,
                                          None, None, 0, None)
    assert st == 1
    e = pkg.Epilogue()
    e.activation = 9
    st = lib.iree_mi355x_batch_matmul_f16(a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                          2, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0,
                                          ctypes.byref(e), None, 0, None)
    assert st == 1


# ------------------------------------------------------------ transposed A --

@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 512, 256),
                                   (256, 768, 192)])
def test_transposed_a_configs(pkg, oracle, dev, shape):
    """Every transposed-A macro-tile (A stored [K, M]) with both B forms."""
    m, n, k = shape
    g = torch.Generator().manual_seed(3 * m + n + k)
    a = torch.randn(m, k, generator=g).half()
    b = torch.randn(k, n, generator=g).half()
    at, bt = a.t().contiguous(), b.t().contiguous()
    ref16 = oracle.matmul_f16(a.numpy(), b.numpy())
    ref32 = oracle.matmul_f16(a.numpy(), b.numpy(), out_f32=True)
    ran = 0
    for cfg in pkg.mfma_configs():
        if "+" in cfg.name:  # a column split: its own tests
            continue
        if not cfg.a_transposed:
            continue
        if m % cfg.tile_m or n % cfg.tile_n or k % cfg.tile_k:
            continue
        out32 = cfg.c_elem == pkg.ELEM_F32
        c = torch.empty(m, n, dtype=torch.float32 if out32 else torch.float16,
                        device=dev)
        bb = bt if cfg.b_form == pkg.B_FORM_TN else b
        pkg.matmul_mfma_config(cfg.index, at.to(dev), bb.to(dev), c)
        fp16_ok(oracle, c.cpu().numpy(), ref32 if out32 else ref16)
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("m,n,k,bt", [
    (64, 128, 96, True),      # convert_matmul_to_hmx.mlir:87-115 (both transposed)
    (512, 1024, 256, False),  # transposed-A macro-tile, B [K, N]
    (1024, 512, 384, True),   # transposed-A macro-tile, B [N, K]
    (100, 200, 300, False),   # ragged: general kernel
    (3, 512, 256, False),     # skinny: general kernel
    (1, 4096, 4096, False),   # one row of unit pitch: streamed as a GEMV
])
@pytest.mark.parametrize("out32", [False, True])
def test_matmul_transposed_a(pkg, oracle, dev, m, n, k, bt, out32):
    g = torch.Generator().manual_seed(m + 3 * n + 7 * k + out32)
    a = (torch.randn(m, k, generator=g) * 0.5).half()
    b = torch.randn(n, k, generator=g).half() if bt else torch.randn(
        k, n, generator=g).half()
    at = a.t().contiguous()
    ref = oracle.matmul_f16(at.numpy(), b.numpy(), a_transposed=True,
                            b_transposed=bt, out_f32=out32)
    dt = torch.float32 if out32 else torch.float16
    buf, c = canary_out((m, n), dt, dev, -7.0)
    pkg.matmul(at.to(dev), b.to(dev), c, a_transposed=True, b_transposed=bt,
               out_dtype=dt)
    fp16_ok(oracle, c.cpu().numpy(), ref)
    check_canary(buf, m, n, -7.0)


def test_large_outputs_written_through_on_every_store_path(pkg, oracle, dev):
    """Unsplit tiles with an output of at least 8 MiB store it written
    through past the L2. The paths that store element by element (a row
    pitch not a multiple of 16 bytes, a fused epilogue) must treat that
    mode as a plain store: over a canary-filled buffer, the result equals
    the product, not the product added to the canary."""
    g = torch.Generator().manual_seed(23)
    m = n = 2048  # 8 MiB of f16: the smallest output written through
    k = 256
    a = (torch.randn(m, k, generator=g) * 0.5).half()
    b = (torch.randn(k, n, generator=g) * 0.5).half()
    ref = oracle.matmul_f16(a.numpy(), b.numpy())
    ad, bd = a.to(dev), b.to(dev)
    p = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0))
    assert p.family == pkg.FAMILY_MFMA and p.splits == 1
    for pitch in (n, n + 4):  # staged 16-byte rows; odd pitch: per element
        buf = torch.full((m, pitch), 3.0, dtype=torch.float16, device=dev)
        y = buf[:, :n]
        pkg.matmul(ad, bd, y)
        fp16_ok(oracle, y.cpu().numpy(), ref)
        if pitch > n:
            assert bool((buf[:, n:] == 3.0).all())
    # fused epilogue (bias): per-element stores of the epilogue path
    bias = (torch.randn(n, generator=g) * 0.5).half()
    y = torch.full((m, n), 3.0, dtype=torch.float16, device=dev)
    pkg.batch_matmul(ad, bd, y, bias=bias.to(dev))
    ref_b = oracle.batch_matmul_f16(a.numpy()[None], b.numpy()[None],
                                    bias=bias.numpy())[0]
    fp16_ok(oracle, y.cpu().numpy(), ref_b)


def test_matmul_transposed_a_accumulate_and_pitch(pkg, oracle, dev):
    """Accumulate into the init, with A [K, M] a view of a wider buffer
    (lda > M) on the fast path."""
    g = torch.Generator().manual_seed(77)
    m, n, k = 256, 512, 192
    abig = (torch.randn(k, m + 64, generator=g) * 0.5).half()
    at = abig[:, :m]
    b = torch.randn(k, n, generator=g).half()
    init = torch.randn(m, n, generator=g).half()
    c = init.to(dev)
    pkg.matmul(abig.to(dev)[:, :m], b.to(dev), c, a_transposed=True,
               accumulate=True)
    ref = oracle.matmul_f16(at.contiguous().numpy(), b.numpy(), init.numpy(),
                            a_transposed=True)
    fp16_ok(oracle, c.cpu().numpy(), ref)


def test_batch_matmul_transposed_a_epilogue(pkg, oracle, dev):
    """Batch of A [Z, K, M] with a shared B, bias and GELU in the store."""
    g = torch.Generator().manual_seed(78)
    z, m, n, k = 3, 256, 512, 128
    a = (torch.randn(z, m, k, generator=g) * 0.5).half()
    b = torch.randn(k, n, generator=g).half()
    bias = torch.randn(n, generator=g).half()
    y = pkg.batch_matmul(a.transpose(1, 2).contiguous().to(dev), b.to(dev),
                         a_transposed=True, bias=bias.to(dev),
                         activation="gelu_tanh")
    ref = oracle.batch_matmul_f16(a.numpy(), b.numpy(), bias=bias.numpy(),
                                  activation=pkg.ACT_GELU_TANH)
    fp16_ok(oracle, y.cpu().numpy(), ref)


# ------------------------------------------------------ kernel resources ----

def test_export_attributes_cover_their_kernels(pkg):
    """The executable library's static per-export attributes (largest LDS
    and workgroup of any kernel the export may launch) equal what the loaded
    kernels report; every kernel fits the CU's LDS and is resident at its
    launch size; the configuration table's LDS formula matches the compiler."""
    ks = pkg.kernel_resources()
    lib = pkg.executable_library()
    names = pkg.export_names()
    for i, export in enumerate(names):
        mine = [k for k in ks if export in k["exports"]]
        attrs = lib.exports.attrs[i]
        assert attrs.lds_bytes == max(k["lds_bytes"] for k in mine), export
        assert attrs.threads == max(k["threads"] for k in mine), export
    cfg_lds = {c.name: c.lds_bytes for c in pkg.mfma_configs()}
    for k in ks:
        assert k["lds_bytes"] <= 160 * 1024, k
        assert k["workgroups_per_cu"] >= 1, k
        assert k["max_threads"] >= k["threads"], k
        if k["name"] in cfg_lds:
            assert k["lds_bytes"] == cfg_lds[k["name"]], k


# ----------------------------------------------- workspace, streams --------

def test_c_abi_refuses_a_missing_workspace(pkg, oracle, dev):
    """The C-ABI allocates nothing: a split-K or GEMV plan without a
    workspace is refused before launch (the output is untouched); with one
    sized by the query it runs."""
    lib = pkg.library()
    g = torch.Generator().manual_seed(23)
    s = torch.cuda.current_stream().cuda_stream
    for m, n, k in [(16, 4096, 4096), (1, 4096, 4096)]:
        x = (torch.randn(m, k, generator=g) * 0.5).half()
        w = (torch.randn(k, n, generator=g) * 0.02).half()
        xd, wd = x.to(dev), w.to(dev)
        y = torch.full((m, n), 3.0, dtype=torch.float16, device=dev)
        args = (xd.data_ptr(), wd.data_ptr(), y.data_ptr(), m, n, k, k, n, n,
                0)
        assert lib.iree_mi355x_matmul_f16(*args, None, 0, s) == \
            pkg.WORKSPACE_TOO_SMALL
        torch.cuda.synchronize()
        assert bool((y == 3.0).all())
        need = lib.iree_mi355x_matmul_workspace_bytes(m, n, k, 0)
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        assert lib.iree_mi355x_matmul_f16(*args, ws.data_ptr(), need, s) == \
            pkg.OK, pkg.last_error()
        ref = oracle.matmul_f16(x.numpy(), w.numpy())
        fp16_ok(oracle, y.cpu().numpy(), ref)


def test_split_k_on_two_streams_library_workspace(pkg, oracle, dev):
    """Calls without a workspace on two streams at once: the wrapper gives
    each stream its own workspace, so the two split-K reductions (and two
    GEMVs) cannot share arrival counters or partials."""
    g = torch.Generator().manual_seed(21)
    cases = [(16, 4096, 4096), (1, 4096, 4096)]
    for m, n, k in cases:
        assert pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).workspace_bytes > 0
        xs = [(torch.randn(m, k, generator=g) * 0.5).half() for _ in range(2)]
        ws = [(torch.randn(k, n, generator=g) * 0.02).half() for _ in range(2)]
        xd = [x.to(dev) for x in xs]
        wd = [w.to(dev) for w in ws]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        torch.cuda.synchronize()
        outs = [[], []]
        for rep in range(8):  # interleaved on both streams
            for i, s in enumerate(streams):
                with torch.cuda.stream(s):
                    outs[i].append(pkg.matmul(xd[i], wd[i]))
        torch.cuda.synchronize()
        for i in range(2):
            ref = oracle.matmul_f16(xs[i].numpy(), ws[i].numpy())
            for y in outs[i]:
                fp16_ok(oracle, y.cpu().numpy(), ref)


def test_library_workspace_under_capture(pkg, oracle, dev):
    """A capturing stream never allocates: with no workspace for it yet the
    wrapper refuses the call (WORKSPACE_TOO_SMALL, nothing captured); after
    one eager call on that stream the workspace exists and the captured
    split-K matmul replays correctly, with eager work between replays."""
    m, n, k = 16, 4096, 4096
    g = torch.Generator().manual_seed(22)
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    w = (torch.randn(k, n, generator=g) * 0.02).half()
    xd, wd = x.to(dev), w.to(dev)
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    ref = oracle.matmul_f16(x.numpy(), w.numpy())
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(pkg.MI355XError) as err:
        with torch.cuda.graph(graph, stream=s):
            y.zero_()  # the graph is not empty when the matmul is refused
            pkg.matmul(xd, wd, y)
    assert err.value.status == pkg.WORKSPACE_TOO_SMALL
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        pkg.matmul(xd, wd, y)  # sizes this stream's workspace
    torch.cuda.synchronize()
    fp16_ok(oracle, y.cpu().numpy(), ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        pkg.matmul(xd, wd, y)
    x2 = (torch.randn(m, k, generator=g) * 0.5).half()
    ref2 = oracle.matmul_f16(x2.numpy(), w.numpy())
    x2d = x2.to(dev)
    for rep in range(4):
        y.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        fp16_ok(oracle, y.cpu().numpy(), ref)
        with torch.cuda.stream(s):  # eager split-K on the same workspace
            y2 = pkg.matmul(x2d, wd)
        torch.cuda.synchronize()
        fp16_ok(oracle, y2.cpu().numpy(), ref2)
