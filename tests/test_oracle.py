"""The CPU oracle pinned against golden vectors, closed forms and independent
implementations (no GPU). A check here must fail for a plausible mistake in
the oracle: a dropped term, a wrong sign or index, a transposed operand."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN


# ------------------------------------------------------------------ f16 ----

def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    got = oracle.f16_to_f32(h)
    want = h.astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 100,
        rng.standard_normal(100000).astype(np.float32) * 1e-5,   # subnormals
        (np.arange(65536, dtype=np.uint32).astype(np.uint16)
         .view(np.float16).astype(np.float32)),                 # exact halves
        # ties: midpoints between adjacent halves round to even
        ((np.arange(1, 30000, dtype=np.uint32).astype(np.uint16).view(np.float16)
          .astype(np.float64) + np.arange(2, 30001, dtype=np.uint32)
          .astype(np.uint16).view(np.float16).astype(np.float64)) / 2)
        .astype(np.float32),
        np.array([65504, 65519.9, 65520, 1e9, -1e9, np.inf, -np.inf, 0.0, -0.0,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], np.float32),
    ])
    got = oracle.f32_to_f16(x)
    want = x.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


# -------------------------------------------------------------- matmul i8 --

@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (17, 19, 23), (64, 65, 63),
                                   (5, 300, 257)])
@pytest.mark.parametrize("bt", [False, True])
def test_matmul_i8_vs_int64(oracle, m, n, k, bt):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k) if bt else (k, n), dtype=np.int8)
    want = a.astype(np.int64) @ (b.T if bt else b).astype(np.int64)
    got = oracle.matmul_i8(a, b, b_transposed=bt)
    assert np.array_equal(got, want.astype(np.int32))
    init = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
    got = oracle.matmul_i8(a, b, init, b_transposed=bt)
    assert np.array_equal(got, (want + init).astype(np.int32))


def test_matmul_i8_extreme_values_no_overflow(oracle):
    # |sum| <= 4096 * 128 * 128 = 2^26 < 2^31: the worst case is exact.
    k = 4096
    a = np.full((2, k), -128, np.int8)
    b = np.full((k, 3), -128, np.int8)
    assert (oracle.matmul_i8(a, b) == 128 * 128 * k).all()
    b[:, 1] = 127
    assert (oracle.matmul_i8(a, b)[:, 1] == -128 * 127 * k).all()


def test_matmul_i8_golden(oracle):
    d = np.load(os.path.join(GOLDEN, "matmul_i8.npz"))
    got = oracle.matmul_i8(d["a"], d["bt"], b_transposed=True)
    assert np.array_equal(got, d["expected"])


# ------------------------------------------------------------- matmul f16 --

@pytest.mark.parametrize("name", ["small_prime_17x19x23", "ragged_m_65x64x64",
                                  "ragged_n_64x65x64", "ragged_k_64x64x65",
                                  "square_32x32x32"])
def test_matmul_f16_golden_micro_models(oracle, name):
    d = np.load(os.path.join(GOLDEN, f"matmul_{name}.npz"))
    atol, rtol, rel_l2 = d["tol"]
    got = oracle.matmul_f16(d["a"], d["b"], out_f32=True)
    rel, _, close = oracle.compare_arrays(d["expected"], got, atol, rtol)
    assert close and rel <= rel_l2
    # f32 accumulation of exact f16 products: far inside the model tolerance
    assert oracle.fp16_parity(got, d["expected"]) < 1e-5


def test_matmul_f16_exact_small_integers(oracle):
    # products and partial sums are small integers: exact in f32, order-free
    rng = np.random.default_rng(1)
    a = rng.integers(-3, 4, (33, 70)).astype(np.float16)
    b = rng.integers(-3, 4, (70, 45)).astype(np.float16)
    want = a.astype(np.int64) @ b.astype(np.int64)
    got = oracle.matmul_f16(a, b, out_f32=True)
    assert np.array_equal(got, want.astype(np.float32))
    got_t = oracle.matmul_f16(a, np.ascontiguousarray(b.T), b_transposed=True,
                              out_f32=True)
    assert np.array_equal(got_t, want.astype(np.float32))
    got16 = oracle.matmul_f16(a, b)
    assert np.array_equal(got16, want.astype(np.float16))


def test_matmul_f16_identity_and_accumulate(oracle):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((40, 24)).astype(np.float16)
    eye = np.eye(24, dtype=np.float16)
    assert np.array_equal(oracle.matmul_f16(a, eye), a)
    init = rng.standard_normal((40, 24)).astype(np.float32)
    got = oracle.matmul_f16(a, eye, init, out_f32=True)
    assert np.array_equal(got, init + a.astype(np.float32))


def test_matmul_f16_rounds_once_rne(oracle):
    # 1 + 2^-11 is a tie between 1 and 1+2^-10 in f16: RNE gives 1.0
    a = np.array([[1.0, 2.0 ** -11]], np.float16)
    b = np.array([[1.0], [1.0]], np.float16)
    assert oracle.matmul_f16(a, b)[0, 0] == np.float16(1.0)
    a = np.array([[1.0 + 2.0 ** -10, 2.0 ** -11]], np.float16)
    assert oracle.matmul_f16(a, b)[0, 0] == np.float16(1.0 + 2.0 ** -9)


def test_matmul_f16_sensitive_to_transpose(oracle):
    # a transposed-operand bug cannot pass the comparisons above
    rng = np.random.default_rng(3)
    a = rng.standard_normal((16, 16)).astype(np.float16)
    b = rng.standard_normal((16, 16)).astype(np.float16)
    good = oracle.matmul_f16(a, b, out_f32=True)
    wrong = oracle.matmul_f16(a, b, b_transposed=True, out_f32=True)
    assert oracle.fp16_parity(wrong, good) > 0.1


def test_matmul_f16_a_transposed_exact(oracle):
    """A stored [K, M] (LIT/codegen/transforms/convert_matmul_to_hmx.mlir:
    87-115, the both-transposed case at its 64x128x96 shape and ragged
    ones): small-integer operands make every sum exact, so the result must
    equal the int64 product of the logical A and B bit for bit."""
    rng = np.random.default_rng(4)
    for m, n, k in [(64, 128, 96), (33, 45, 70), (1, 8, 5), (7, 1, 13)]:
        a = rng.integers(-3, 4, (m, k)).astype(np.float16)
        b = rng.integers(-3, 4, (k, n)).astype(np.float16)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        at = np.ascontiguousarray(a.T)
        bt = np.ascontiguousarray(b.T)
        got = oracle.matmul_f16(at, b, a_transposed=True, out_f32=True)
        assert got.shape == (m, n) and np.array_equal(got, want)
        got = oracle.matmul_f16(at, bt, a_transposed=True, b_transposed=True,
                                out_f32=True)
        assert np.array_equal(got, want)


def test_matmul_f16_a_transposed_random_and_sensitive(oracle):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((48, 80)).astype(np.float16)
    b = rng.standard_normal((80, 32)).astype(np.float16)
    ref = oracle.matmul_f16(a, b, out_f32=True)
    got = oracle.matmul_f16(np.ascontiguousarray(a.T), b, a_transposed=True,
                            out_f32=True)
    assert np.array_equal(got, ref)          # same sums in the same k order
    sq = rng.standard_normal((40, 40)).astype(np.float16)
    wrong = oracle.matmul_f16(sq, b[:40], a_transposed=True, out_f32=True)
    good = oracle.matmul_f16(sq, b[:40], out_f32=True)
    assert oracle.fp16_parity(wrong, good) > 0.1


# ------------------------------------------------------------------ w8a16 --

def test_w8a16_exact_power_of_two_scales(oracle):
    rng = np.random.default_rng(4)
    x = rng.integers(-4, 5, (3, 64)).astype(np.float16)
    w = rng.integers(-128, 128, (64, 48), dtype=np.int8)
    s = (2.0 ** -rng.integers(3, 8, 48)).astype(np.float16)
    want = (x.astype(np.int64) @ w.astype(np.int64)) * s.astype(np.float64)
    got = oracle.w8a16(x, w, s)
    assert np.array_equal(got, want.astype(np.float16))
    got_t = oracle.w8a16(x, np.ascontiguousarray(w.T), s, w_transposed=True)
    assert np.array_equal(got_t, got)


def test_w8a16_matches_per_element_dequant(oracle, inputs):
    x, w, s = (t.numpy() for t in inputs.c5_w8a16(4, n=512, k=1024))
    got = oracle.w8a16(x, w, s)
    deq = (w.astype(np.float64) * s.astype(np.float64)).astype(np.float16)
    want = x.astype(np.float64) @ deq.astype(np.float64)
    assert oracle.fp16_parity(got, want) < 2e-3


# -------------------------------------------------------------- attention --

@pytest.mark.parametrize("name", ["b1h2s128d64_causal", "b1h2s128d64",
                                  "b1h1s160d128_causal"])
def test_attention_golden_sdpa(oracle, name):
    d = np.load(os.path.join(GOLDEN, f"attention_{name}.npz"))
    got = oracle.attention_f16(d["q"], d["k"], d["v"], causal=bool(d["causal"]))
    atol, rtol, rel_l2 = d["tol"]
    rel, _, close = oracle.compare_arrays(d["expected"], got, atol, rtol)
    assert close and rel <= rel_l2
    assert oracle.fp16_parity(got, d["expected"]) < 1e-3


def test_attention_causal_invariants(oracle):
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((1, 2, 50, 64)).astype(np.float16)
               for _ in range(3))
    o = oracle.attention_f16(q, k, v, causal=True)
    # query 0 sees only key 0: output is V[0] exactly
    assert np.array_equal(o[:, :, 0], v[:, :, 0])
    # q = 0: uniform weights, row i is the mean of V[0..i]
    o0 = oracle.attention_f16(np.zeros_like(q), k, v, causal=True)
    csum = np.cumsum(v.astype(np.float64), axis=2)
    mean = csum / np.arange(1, 51)[None, None, :, None]
    assert np.abs(o0.astype(np.float64) - mean).max() < 2e-3
    # future keys/values do not change earlier rows
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 30:] = 7
    v2[:, :, 30:] = -7
    o2 = oracle.attention_f16(q, k2, v2, causal=True)
    assert np.array_equal(o2[:, :, :30], o[:, :, :30])


def test_attention_vs_torch_sdpa_nonsquare(oracle):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 3, 40, 64, generator=g).half()
    k = torch.randn(1, 3, 72, 64, generator=g).half()
    v = torch.randn(1, 3, 72, 64, generator=g).half()
    want = F.scaled_dot_product_attention(q.float(), k.float(), v.float())
    got = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), causal=False)
    assert oracle.fp16_parity(got, want.numpy()) < 1e-3


# The scales a matched region hands over besides 1/sqrt(d): the product of
# attention_layer.mlir's two 128^-1/4 factors with d = 64 (0.297...^2 is not
# 1/8), an explicit 0.5, and a scale so small the softmax is nearly uniform.
def sdpa_f64(q, k, v, scale, causal):
    """softmax(q k^T scale + top-left causal mask) v in float64 numpy, for
    scales torch's sdpa cannot take (its math path multiplies q and k by
    sqrt(scale) each, so a negative scale gives nan)."""
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64),
                  k.astype(np.float64)) * scale
    if causal:
        sq, skv = s.shape[-2:]
        s = np.where(np.arange(skv)[None, :] > np.arange(sq)[:, None],
                     -np.inf, s)
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    return np.einsum("bhqk,bhkd->bhqd", s / s.sum(axis=-1, keepdims=True),
                     v.astype(np.float64))


@pytest.mark.parametrize("scale", [0.29730177875068026 ** 2, 0.5, 0.297,
                                   1e-3, -0.3])
@pytest.mark.parametrize("sq,skv,causal", [(40, 72, False), (40, 72, True),
                                           (72, 40, True), (1, 96, False),
                                           (1, 96, True), (33, 33, True)])
def test_attention_scale_and_lengths_vs_sdpa(oracle, scale, sq, skv, causal):
    # F.sdpa(scale=, is_causal=) is the pin: its causal mask is top-left
    # aligned (key j hidden from query i when j > i) for any Sq, Skv.
    g = torch.Generator().manual_seed(sq * 1000 + skv)
    q = torch.randn(1, 2, sq, 64, generator=g).half()
    k = torch.randn(1, 2, skv, 64, generator=g).half()
    v = torch.randn(1, 2, skv, 64, generator=g).half()
    if scale > 0:
        want = F.scaled_dot_product_attention(
            q.float(), k.float(), v.float(), is_causal=causal,
            scale=scale).numpy()
    else:
        want = sdpa_f64(q.numpy(), k.numpy(), v.numpy(), scale, causal)
    got = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), scale=scale,
                               causal=causal)
    assert oracle.fp16_parity(got, want) < 1e-3
    # a wrong scale is caught: the oracle at 1/sqrt(d) differs here
    if abs(scale - 0.125) > 1e-2:
        other = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(),
                                     causal=causal)
        if not (causal and sq == 1):  # one visible key: scale-independent
            assert oracle.fp16_parity(other, want) > 1e-2


@pytest.mark.parametrize("sq,skv,causal", [(40, 72, True), (72, 40, False)])
def test_attention_zero_scale_is_the_mean(oracle, sq, skv, causal):
    # scale 0: every visible key weighs the same, row i is the mean of the
    # V rows it sees (torch's sdpa returns nan here under a causal mask)
    rng = np.random.default_rng(sq + skv)
    q = rng.standard_normal((1, 2, sq, 64)).astype(np.float16)
    k, v = (rng.standard_normal((1, 2, skv, 64)).astype(np.float16)
            for _ in range(2))
    o = oracle.attention_f16(q, k, v, scale=0.0, causal=causal)
    vf = v.astype(np.float64)
    for i in range(sq):
        last = min(i, skv - 1) if causal else skv - 1
        want = vf[:, :, :last + 1].mean(axis=2)
        assert np.abs(o[:, :, i].astype(np.float64) - want).max() < 2e-3


def test_attention_single_query_row_causal(oracle):
    # seq_q = 1 under a top-left causal mask sees key 0 only: O = V[0]
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 1, 128)).astype(np.float16)
    k, v = (rng.standard_normal((1, 2, 300, 128)).astype(np.float16)
            for _ in range(2))
    o = oracle.attention_f16(q, k, v, causal=True, scale=0.7)
    assert np.array_equal(o[:, :, 0], v[:, :, 0])


@pytest.mark.parametrize("hq,hkv,causal", [(8, 2, False), (6, 3, True),
                                           (4, 1, True)])
def test_attention_grouped_heads_vs_sdpa(oracle, hq, hkv, causal):
    g = torch.Generator().manual_seed(hq * 10 + hkv)
    q = torch.randn(2, hq, 70, 64, generator=g).half()
    k = torch.randn(2, hkv, 90, 64, generator=g).half()
    v = torch.randn(2, hkv, 90, 64, generator=g).half()
    want = F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                          is_causal=causal, enable_gqa=True)
    got = oracle.attention_f16(q.numpy(), k.numpy(), v.numpy(), causal=causal)
    assert oracle.fp16_parity(got, want.numpy()) < 1e-3
    # the same as repeating each KV head over its query heads
    rep = hq // hkv
    got2 = oracle.attention_f16(q.numpy(), np.repeat(k.numpy(), rep, axis=1),
                                np.repeat(v.numpy(), rep, axis=1),
                                causal=causal)
    assert np.array_equal(got, got2)
    # and not the same as interleaving them (head h reading KV head h % hkv)
    if hkv > 1:
        got3 = oracle.attention_f16(q.numpy(), np.tile(k.numpy(), (1, rep, 1, 1)),
                                    np.tile(v.numpy(), (1, rep, 1, 1)),
                                    causal=causal)
        assert not np.array_equal(got, got3)


def test_attention_strided_views(oracle):
    # K, V a slice of a longer cache, Q a head-major view of a [B, S, H, D]
    # buffer, O written into a [B, S, H, D] buffer: the same values as the
    # contiguous call
    rng = np.random.default_rng(11)
    q_bshd = rng.standard_normal((2, 50, 4, 64)).astype(np.float16)
    kc, vc = (rng.standard_normal((2, 2, 130, 64)).astype(np.float16)
              for _ in range(2))
    q = q_bshd.transpose(0, 2, 1, 3)
    k, v = kc[:, :, :77], vc[:, :, :77]
    o_bshd = np.full((2, 50, 4, 64), np.nan, np.float16)
    oracle.attention_f16(q, k, v, causal=True, out=o_bshd.transpose(0, 2, 1, 3))
    want = oracle.attention_f16(np.ascontiguousarray(q), np.ascontiguousarray(k),
                                np.ascontiguousarray(v), causal=True)
    assert np.array_equal(o_bshd.transpose(0, 2, 1, 3), want)


def test_attention_cache_slice_golden(oracle):
    # the reference's grouped-query KV-cache micro model, its tolerances
    d = np.load(os.path.join(GOLDEN, "attention_cache_slice.npz"))
    ctx = int(d["context"])
    k, v = d["k_cache"][:, :, :ctx], d["v_cache"][:, :, :ctx]
    q = d["q"]
    b, hq, sq, dim = q.shape
    out = np.empty((b, sq, hq, dim), np.float16)
    oracle.attention_f16(q, k, v, causal=False,
                         out=out.transpose(0, 2, 1, 3))
    atol, rtol, rel_l2 = d["tol"]
    for key in ("expected", "expected_f32"):
        rel, _, close = oracle.compare_arrays(d[key], out, atol, rtol)
        assert close and rel <= rel_l2, (key, rel)
    assert oracle.fp16_parity(out, d["expected_f32"]) < 2e-3


# ------------------------------------------------ attention, general form ---

def attention_f64(q, k, v, scale, causal=False, mask=None):
    """softmax(q k^T scale + mask [+ top-left causal]) v in float64 with
    numpy broadcasting of the mask and grouped KV heads; a row with no
    unmasked key is 0."""
    rep = q.shape[1] // k.shape[1]
    k = np.repeat(k.astype(np.float64), rep, axis=1)
    v = np.repeat(v.astype(np.float64), rep, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)
    if causal:
        sq, skv = s.shape[-2:]
        s = np.where(np.arange(skv)[None, :] > np.arange(sq)[:, None],
                     -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    dead = mx == -np.inf
    p = np.where(dead, 0.0, np.exp(s - np.where(dead, 0.0, mx)))
    den = p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p / np.where(den > 0, den, 1.0), v)


def random_mask(rng, shape, dead_frac=0.2):
    """An f16 additive mask: N(0, 2) values with some keys at -inf."""
    m = (2 * rng.standard_normal(shape)).astype(np.float16)
    m[rng.random(shape) < dead_frac] = -np.inf
    return m


@pytest.mark.parametrize("dqk,dv,mask_shape", [
    (24, 40, (2, 1, 37, 53)), (4, 5, (1, 3, 1, 53)), (64, 64, (2, 3, 37, 53)),
    (96, 32, (1, 53))])
def test_attention_general_vs_sdpa_mask(oracle, dqk, dv, mask_shape):
    # torch's SDPA adds attn_mask after the scale, as iree_linalg_ext
    # attention does; a broadcast mask (batch, head or row of 1) reads with
    # stride 0
    rng = np.random.default_rng(dqk * 100 + dv)
    b, h, sq, skv = 2, 3, 37, 53
    q = rng.standard_normal((b, h, sq, dqk)).astype(np.float16)
    k = rng.standard_normal((b, h, skv, dqk)).astype(np.float16)
    v = rng.standard_normal((b, h, skv, dv)).astype(np.float16)
    mask = random_mask(rng, mask_shape, 0.1)
    full = np.broadcast_to(mask, (b, h, sq, skv))
    assert not (full == -np.inf).all(axis=-1).any()
    scale = 0.37
    want = F.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(k).float(),
        torch.from_numpy(v).float(), attn_mask=torch.from_numpy(mask).float(),
        scale=scale).numpy()
    got32 = oracle.attention(q, k, v, scale=scale, mask=mask, out_f32=True)
    assert got32.dtype == np.float32 and got32.shape == (b, h, sq, dv)
    assert oracle.fp16_parity(got32, want) < 1e-5
    got16 = oracle.attention(q, k, v, scale=scale, mask=mask)
    # the f16 output is the f32 one rounded once
    assert np.array_equal(got16, got32.astype(np.float16))
    # the mask added before the scale would be a different function
    wrong = attention_f64(q, k, v, 1.0, mask=mask.astype(np.float64) / scale)
    assert oracle.fp16_parity(got32, wrong * 1.0) > 1e-2 or scale == 1.0


def test_attention_general_reference_fixture_shape(oracle):
    # the shapes of hexagon_lower_executable_target.mlir:195-233: Q 1x2x4,
    # K 1x3x4, V 1x3x5 f16, scale 0.5, f32 result; against the float64
    # closed form (no mask, not causal)
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 1, 2, 4)).astype(np.float16)
    k = rng.standard_normal((1, 1, 3, 4)).astype(np.float16)
    v = rng.standard_normal((1, 1, 3, 5)).astype(np.float16)
    got = oracle.attention(q, k, v, scale=0.5, out_f32=True)
    want = attention_f64(q, k, v, 0.5)
    assert np.abs(got - want).max() < 1e-6
    # brute force of the first row, term by term
    s = [0.5 * sum(float(q[0, 0, 0, d]) * float(k[0, 0, j, d])
                   for d in range(4)) for j in range(3)]
    e = [np.exp(x - max(s)) for x in s]
    row = [sum(e[j] * float(v[0, 0, j, n]) for j in range(3)) / sum(e)
           for n in range(5)]
    assert np.abs(got[0, 0, 0] - row).max() < 1e-6


def test_attention_general_masked_keys_drop_out(oracle):
    # a -inf key weighs exactly 0: the same bits as the call without it
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 9, 16)).astype(np.float16)
    k = rng.standard_normal((1, 2, 30, 16)).astype(np.float16)
    v = rng.standard_normal((1, 2, 30, 24)).astype(np.float16)
    keep = np.ones(30, bool)
    keep[[0, 7, 8, 29]] = False
    mask = np.where(keep, 0.0, -np.inf).astype(np.float16)
    got = oracle.attention(q, k, v, scale=0.25, mask=mask)
    want = oracle.attention(q, np.ascontiguousarray(k[:, :, keep]),
                            np.ascontiguousarray(v[:, :, keep]), scale=0.25)
    assert np.array_equal(got, want)
    # a zero mask is no mask
    zero = np.zeros(30, np.float16)
    assert np.array_equal(oracle.attention(q, k, v, scale=0.25, mask=zero),
                          oracle.attention(q, k, v, scale=0.25))


def test_attention_general_fully_masked_rows_are_zero(oracle):
    # the all-masked guard of attention_layer.mlir:80-102 writes 0 (as the
    # SDPA of this torch does; earlier releases wrote nan)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 1, 6, 8)).astype(np.float16)
    k = rng.standard_normal((1, 1, 10, 8)).astype(np.float16)
    v = rng.standard_normal((1, 1, 10, 8)).astype(np.float16)
    mask = np.zeros((6, 10), np.float16)
    mask[[1, 4]] = -np.inf
    got = oracle.attention(q, k, v, scale=0.5, mask=mask, out_f32=True)
    assert (got[0, 0, [1, 4]] == 0).all()
    want = attention_f64(q, k, v, 0.5, mask=mask)
    assert np.abs(got - want).max() < 1e-6
    sdpa = F.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(k).float(),
        torch.from_numpy(v).float(), attn_mask=torch.from_numpy(mask).float(),
        scale=0.5).numpy()
    assert np.abs(got - sdpa).max() < 1e-5


@pytest.mark.parametrize("hq,hkv", [(6, 2), (4, 4)])
def test_attention_general_causal_mask_gqa(oracle, hq, hkv):
    # causal and a mask together, grouped KV heads, unequal head dims
    rng = np.random.default_rng(hq + hkv)
    q = rng.standard_normal((2, hq, 45, 20)).astype(np.float16)
    k = rng.standard_normal((2, hkv, 60, 20)).astype(np.float16)
    v = rng.standard_normal((2, hkv, 60, 12)).astype(np.float16)
    mask = random_mask(rng, (2, hq, 45, 60), 0.3)
    got = oracle.attention(q, k, v, scale=-0.4, causal=True, mask=mask,
                           out_f32=True)
    want = attention_f64(q, k, v, -0.4, causal=True, mask=mask)
    assert np.abs(got - want).max() < 1e-5
    # the general form without mask is the attention_f16 routine
    if hkv == hq:
        q2 = q[..., :16].copy()
        k2 = k[..., :16].copy()
        v2 = v[..., :12].copy()
        v2 = np.concatenate([v2, v2[..., :4]], axis=-1)
        assert np.array_equal(oracle.attention(q2, k2, v2, causal=True),
                              oracle.attention_f16(q2, k2, v2, causal=True))


# --------------------------------------------------------------- planner ---

def test_select_hmx_tile_sizes_lit_goldens(oracle):
    with open(os.path.join(GOLDEN, "tile_search.json")) as f:
        spec = json.load(f)
    for case in spec["cases"]:
        got = oracle.select_hmx_tile_sizes(
            case["m"], case["n"], case["k"], elem_bytes=case["elem_bytes"],
            b_transposed=case["b_transposed"],
            budget_bytes=spec["budget_flag_bytes"],
            double_buffering=spec["double_buffering"])
        assert got == case["expected"], (case, got)


def test_select_hmx_tile_sizes_budget_matters(oracle):
    # without the halve-then-double budget plumbing, the first golden would
    # pick N=64 (a 4 MiB budget admits it): the plumbing is pinned
    got = oracle.select_hmx_tile_sizes(52, 896, 7680, elem_bytes=(2, 2, 4),
                                       b_transposed=True,
                                       budget_bytes=4 * 1024 * 1024)
    assert got == [52, 64, 7680]


def brute_force_tiling_factor(bound, preferred, multiple_of):
    if preferred <= 0:
        return 0
    step = max(1, multiple_of)
    if bound <= 0 or bound % step or preferred < step:
        return min(bound, preferred)
    best = 0
    for d in range(1, bound // step + 1):
        if (bound // step) % d == 0 and d * step <= preferred:
            best = max(best, d * step)
    return best


def test_choose_static_tiling_factor_brute_force(oracle):
    for bound in list(range(-2, 130)) + [4096, 11008, 7680]:
        for preferred in (-1, 0, 1, 3, 8, 13, 32, 64, 200):
            for mult in (0, 1, 2, 8, 32):
                want = brute_force_tiling_factor(bound, preferred, mult)
                got = oracle.choose_static_tiling_factor(bound, preferred, mult)
                assert got == want, (bound, preferred, mult)
    assert oracle.choose_static_tiling_factor(oracle.DYNAMIC, 8, 1) == 8


# ------------------------------------------------ batch matmul / epilogue ----

def test_batch_matmul_equals_per_batch_matmul(oracle):
    g = np.random.default_rng(5)
    a = g.standard_normal((3, 17, 23)).astype(np.float16)
    b = g.standard_normal((3, 23, 19)).astype(np.float16)
    got = oracle.batch_matmul_f16(a, b, out_f32=True)
    for z in range(3):
        ref = oracle.matmul_f16(a[z], b[z], out_f32=True)
        assert np.array_equal(got[z], ref)
    # a 2-D B is shared by every batch; transposed B gives the same sums
    bt = np.ascontiguousarray(b[0].T)
    shared = oracle.batch_matmul_f16(a, bt, b_transposed=True, out_f32=True)
    for z in range(3):
        assert np.array_equal(shared[z], oracle.matmul_f16(a[z], b[0], out_f32=True))


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_batch_matmul_epilogue_closed_forms(oracle, act):
    """out = mul * act(acc + bias) against numpy closed forms (f64)."""
    g = np.random.default_rng(6 + act)
    a = g.standard_normal((2, 9, 16)).astype(np.float16)
    b = g.standard_normal((2, 16, 12)).astype(np.float16)
    bias = g.standard_normal(12).astype(np.float16)
    mul = g.standard_normal((2, 9, 12)).astype(np.float16)
    got = oracle.batch_matmul_f16(a, b, out_f32=True, bias=bias, activation=act,
                                  multiplier=mul)
    x = np.einsum("zmk,zkn->zmn", a.astype(np.float64), b.astype(np.float64))
    x = x + bias.astype(np.float64)
    if act == 1:
        x = np.maximum(x, 0.0)
    elif act == 2:
        x = 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
    elif act == 3:
        x = x / (1.0 + np.exp(-x))
    x = x * mul.astype(np.float64)
    assert np.abs(got - x).max() <= 1e-4 * max(1.0, np.abs(x).max())
    # order matters: the bias is added before the activation
    if act == 1:
        wrong = np.maximum(x / mul.astype(np.float64) - bias.astype(np.float64),
                           0.0) + bias.astype(np.float64)
        assert np.abs(got - wrong * mul.astype(np.float64)).max() > 1e-2


def test_activation_points(oracle):
    assert oracle.activation(3.5, 1) == 3.5 and oracle.activation(-3.5, 1) == 0.0
    assert oracle.activation(0.0, 2) == 0.0 and oracle.activation(0.0, 3) == 0.0
    # GELU(x) - GELU(-x) = x (odd part), limits, the value at 1
    for x in (0.3, 1.7, 4.0):
        assert abs(oracle.activation(x, 2) - oracle.activation(-x, 2) - x) < 1e-6
    assert abs(oracle.activation(10.0, 2) - 10.0) < 1e-6
    assert abs(oracle.activation(-10.0, 2)) < 1e-6
    assert abs(oracle.activation(1.0, 2) - 0.8411919906) < 1e-6
    # SiLU(x) = x sigmoid(x); SiLU(x) - SiLU(-x) = x
    assert abs(oracle.activation(2.0, 3) - 2.0 / (1.0 + np.exp(-2.0))) < 1e-6
    assert abs(oracle.activation(1.3, 3) - oracle.activation(-1.3, 3) - 1.3) < 1e-6


def test_geglu_f16_ops_reference_form(oracle):
    """The reference IR's GeGLU epilogue (every op in f16) at hand-computed
    points, and its distance from the f32 epilogue the kernels compute."""
    got = oracle.geglu_f16_ops([1.0, -2.0, 0.0, 8.0, -8.0], [1.0, 1.0, 1.0, 2.0, 1.0])
    assert abs(float(got[0]) - 0.8412) < 2e-3
    assert abs(float(got[1]) + 0.0455) < 2e-4
    assert float(got[2]) == 0.0
    assert float(got[3]) == 16.0
    assert abs(float(got[4])) < 1e-6
    g = np.random.default_rng(7)
    acc = (g.standard_normal(4096) * 2.0).astype(np.float32)
    up = g.standard_normal(4096).astype(np.float16)
    f16_ops = oracle.geglu_f16_ops(acc, up).astype(np.float32)
    f32 = np.array([oracle.activation(float(v), 2) for v in acc], np.float32)
    f32 = f32 * up.astype(np.float32)
    assert np.abs(f16_ops - f32).max() / np.abs(f32).max() <= 2e-3
