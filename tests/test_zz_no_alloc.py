"""The allocation-free entry point against the existing one, through the
C-ABI: iree_mi355x_matmul_f16_no_alloc keeps its split-K partials and arrival
counters in the library's static device scratch, so its results must equal
iree_mi355x_matmul_f16's (same plan, same kernels, the same fixed reduction
order) bit for bit, and meet the fp16 bar against the oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FP16_BOUND = 2e-3


def _call(pkg, fn, x, w, y, stream):
    lib = pkg.library()
    m, k = x.shape
    n = w.shape[1]
    args = (x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, x.stride(0),
            w.stride(0), y.stride(0), 0)
    if fn == "no_alloc":
        return lib.iree_mi355x_matmul_f16_no_alloc(*args, stream)
    # the existing entry point takes its scratch from a caller workspace
    ws, wsb = pkg.stream_workspace(
        lib.iree_mi355x_matmul_workspace_bytes(m, n, k, 0), x.device, stream)
    return lib.iree_mi355x_matmul_f16(*args, ws, wsb, stream)


def test_no_alloc_matches_matmul_f16(pkg, oracle, dev):
    lib = pkg.library()
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(31)
    # A split-K MFMA shape, then a smaller GEMV shape: both use the scratch,
    # the second right after the first on the same stream.
    shapes = [(64, 11008, 4096), (1, 4096, 4096)]
    for m, n, k in shapes:
        p = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0))
        assert 0 < p.workspace_bytes <= 32 << 20, (m, n, k)
    host, dev_in, outs = [], [], []
    for m, n, k in shapes:
        x = (torch.randn(m, k, generator=g) * 0.5).half()
        w = (torch.randn(k, n, generator=g) * 0.02).half()
        host.append((x, w))
        dev_in.append((x.to(dev), w.to(dev)))
    torch.cuda.synchronize()
    for (x, w) in dev_in:
        y = torch.full((x.shape[0], w.shape[1]), 3.0, dtype=torch.float16,
                       device=dev)
        print(f"no_alloc m={x.shape[0]} n={w.shape[1]} k={x.shape[1]}",
              flush=True)
        assert _call(pkg, "no_alloc", x, w, y, s) == pkg.OK, pkg.last_error()
        outs.append(y)
    torch.cuda.synchronize()
    for (x, w), (xh, wh), y in zip(dev_in, host, outs):
        y_ref = torch.empty_like(y)
        assert _call(pkg, "workspace", x, w, y_ref, s) == pkg.OK
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint16),
                              y_ref.cpu().numpy().view(np.uint16))
        err = oracle.fp16_parity(got, oracle.matmul_f16(xh.numpy(), wh.numpy()))
        assert err <= FP16_BOUND, err


def test_no_alloc_repeated_and_rejects_oversized_plans(pkg, oracle, dev):
    lib = pkg.library()
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(32)
    # repeated calls leave the counters armed for the next one
    m, n, k = 16, 4096, 4096
    x = (torch.randn(m, k, generator=g) * 0.5).half()
    w = (torch.randn(k, n, generator=g) * 0.02).half()
    xd, wd = x.to(dev), w.to(dev)
    ref = oracle.matmul_f16(x.numpy(), w.numpy())
    ys = [torch.empty(m, n, dtype=torch.float16, device=dev) for _ in range(4)]
    for y in ys:
        assert _call(pkg, "no_alloc", xd, wd, y, s) == pkg.OK
    torch.cuda.synchronize()
    for y in ys:
        assert oracle.fp16_parity(y.cpu().numpy(), ref) <= FP16_BOUND
    # a plan needing more than the 32 MiB scratch is refused, nothing written
    m, n, k = 256, 11008, 11008
    assert pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).workspace_bytes > 32 << 20
    x = torch.zeros(m, k, dtype=torch.float16, device=dev)
    w = torch.zeros(k, n, dtype=torch.float16, device=dev)
    y = torch.full((m, n), 5.0, dtype=torch.float16, device=dev)
    assert _call(pkg, "no_alloc", x, w, y, s) == pkg.WORKSPACE_TOO_SMALL
    assert "workspace" in pkg.last_error()
    torch.cuda.synchronize()
    assert bool((y == 5.0).all())
