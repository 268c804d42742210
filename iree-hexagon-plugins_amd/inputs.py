"""Seeded synthetic inputs for the benchmark configurations.

Mirrors the reference harness's generators (IT/stages/importing.py:218-262):
one torch.Generator per input seeded with that input's seed, ``normal`` =
torch.randn in f32 then cast, integer ``uniform`` = torch.randint(low, high).
Two generators the reference lacks are added for the BASELINE configs:
float ``uniform`` over [low, high) and a scaled normal (std != 1).
Tensors are produced on the host; callers move them to the device.
"""
from __future__ import annotations

import torch


def generate(shape, dtype, generator: str, seed: int, *, low=None, high=None,
             std: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    integral = dtype in (torch.int8, torch.int32, torch.int64, torch.bool)
    if generator == "normal":
        if integral:
            raise ValueError("normal generator needs a float dtype")
        t = torch.randn(shape, generator=g, dtype=torch.float32)
        if std != 1.0:
            t = t * std
        return t.to(dtype)
    if generator == "uniform":
        if integral:
            return torch.randint(low, high, shape, generator=g).to(dtype)
        t = torch.rand(shape, generator=g, dtype=torch.float32)
        return (t * (high - low) + low).to(dtype)
    if generator == "zeros":
        return torch.zeros(shape, dtype=dtype)
    if generator == "ones":
        return torch.ones(shape, dtype=dtype)
    raise ValueError(f"unknown generator {generator!r}")


# BASELINE.json configs, inputs in argument order with seeds 0, 1, 2.
def c1_matmul_f16():
    a = generate((128, 256), torch.float16, "uniform", 0, low=-1.0, high=1.0)
    b = generate((256, 512), torch.float16, "uniform", 1, low=-1.0, high=1.0)
    return a, b


def c2_matmul_i8(m=4096, n=4096, k=4096):
    a = generate((m, k), torch.int8, "uniform", 0, low=-128, high=128)
    # column-major B == B^T stored row-major [N, K]
    bt = generate((n, k), torch.int8, "uniform", 1, low=-128, high=128)
    return a, bt


def c3_linear_f16(m, n, k):
    x = generate((m, k), torch.float16, "normal", 0, std=0.02)
    w = generate((k, n), torch.float16, "normal", 1, std=0.02)
    return x, w


def c4_attention_f16(batch=1, heads=32, seq=2048, head_dim=128):
    shape = (batch, heads, seq, head_dim)
    return tuple(generate(shape, torch.float16, "normal", s) for s in range(3))


def c5_w8a16(m, n=11008, k=4096):
    x = generate((m, k), torch.float16, "normal", 0)
    w = generate((k, n), torch.int8, "uniform", 1, low=-128, high=128)
    s = generate((n,), torch.float16, "uniform", 2, low=0.001, high=0.02)
    return x, w, s
