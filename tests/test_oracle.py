"""Pins the CPU oracle (oracle/oracle.c) before the HIP engine's results are compared against it.

Each check is chosen so that a plausible restatement mistake fails it: closed forms, float64
brute force, invariants, and an independent implementation (transformers' Qwen3, built from a
local config) through the committed fixtures in tests/golden/.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle


def bf16_rne(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f64(w):
    return (np.asarray(w, np.uint32) << 16).view(np.float32).astype(np.float64)


def test_bf16_to_f32_exhaustive():
    # cpu_inference.rs:182-183: f32::from_bits(u16 << 16), for all 65536 patterns
    L = oracle.lib()
    pats = np.arange(65536, dtype=np.uint32)
    want = (pats << 16).view(np.float32)
    got = np.array([L.or_bf16_to_f32(int(p)) for p in pats], dtype=np.float32)
    # the float return passes through a Python float (double), which quiets signaling NaNs, so
    # NaN patterns are compared as NaN; every other pattern must match bit for bit
    nan = np.isnan(want)
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    assert np.all(np.isnan(got[nan])) and nan.sum() == 2 * 127


@pytest.mark.parametrize("n", [1, 7, 8, 9, 64, 1024, 1027, 3072])
def test_dot_bf16_against_float64(n):
    rng = np.random.default_rng(n)
    w = bf16_rne(rng.normal(0, 0.02, n))
    x = rng.standard_normal(n).astype(np.float32)
    got = oracle.lib().or_dot_bf16(oracle.u16p(w), oracle.f32p(x), n)
    ref = float(bf16_to_f64(w) @ x.astype(np.float64))
    mag = float(np.abs(bf16_to_f64(w)) @ np.abs(x.astype(np.float64)))
    assert abs(got - ref) <= n * 2 ** -24 * mag + 1e-30


def test_dot_bf16_fold_order():
    # the 8-accumulator fold (cpu_inference.rs:243-257) is observable: put a large value in
    # lane 0 and small ones after it; a sequential sum would absorb the small terms
    n = 16
    w = bf16_rne(np.ones(n))
    x = np.zeros(n, np.float32)
    x[0] = 2.0 ** 24
    x[1:8] = 1.0        # accumulators 1..7 hold 1.0 each after chunk 0
    x[8] = 1.0          # accumulator 0: 2^24 + 1 -> 2^24 (round to even)
    got = oracle.lib().or_dot_bf16(oracle.u16p(w), oracle.f32p(x), n)
    # acc = [2^24, 1, 1, 1, 1, 1, 1, 1] summed in order from -0.0: 2^24 + 1 -> 2^24 each time
    assert got == 2.0 ** 24
    # a sequential left-to-right dot would give the same here, so also check a case where the
    # remainder is added after the fold: n = 9 with x[8] landing in the remainder
    w9 = bf16_rne(np.ones(9))
    x9 = np.array([2.0 ** 24, 0, 0, 0, 0, 0, 0, 0, 1.0], np.float32)
    assert oracle.lib().or_dot_bf16(oracle.u16p(w9), oracle.f32p(x9), 9) == 2.0 ** 24


def test_matvec_exact_small_integers_and_row_split():
    rng = np.random.default_rng(0)
    rows, cols = 37, 24
    wi = rng.integers(-3, 4, size=(rows, cols)).astype(np.float32)
    x = rng.integers(-4, 5, size=cols).astype(np.float32)
    w = bf16_rne(wi)
    for threads in (1, 3, 8, 64):
        oracle.set_threads(threads)
        np.testing.assert_array_equal(oracle.matvec(w, x), (wi @ x).astype(np.float32))
    oracle.set_threads(0)


def test_rmsnorm_closed_form():
    # constant vector c with unit gains: out = c / sqrt(c^2 + eps)
    # (c = 0.5 and 3: c^2 and the running sum of squares are exact in f32, so the only
    # roundings left are the mean, +eps, sqrt, divide and the two products)
    L = oracle.lib()
    n, c, eps = 1024, 0.5, 1e-6
    for c in (0.5, 3.0):
        x = np.full(n, c, np.float32)
        w = bf16_rne(np.ones(n))
        out = np.empty(n, np.float32)
        L.or_rmsnorm(oracle.f32p(out), oracle.f32p(x), oracle.u16p(w), n, eps)
        assert np.allclose(out, c / math.sqrt(c * c + eps), rtol=4e-7)
    c = 0.5
    x = np.full(n, c, np.float32)
    w = bf16_rne(np.ones(n))
    out = np.empty(n, np.float32)
    L.or_rmsnorm(oracle.f32p(out), oracle.f32p(x), oracle.u16p(w), n, eps)
    assert np.allclose(out, c / math.sqrt(c * c + eps), rtol=2e-7)
    # gains multiply after normalization: (x*s)*w
    w2 = bf16_rne(np.full(n, 2.0))
    L.or_rmsnorm(oracle.f32p(out), oracle.f32p(x), oracle.u16p(w2), n, eps)
    assert np.allclose(out, 2 * c / math.sqrt(c * c + eps), rtol=2e-7)


def test_rope_identity_and_rotation():
    L = oracle.lib()
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128).astype(np.float32)
    y = x.copy()
    L.or_rope(oracle.f32p(y), 128, 0, 1e6)
    np.testing.assert_array_equal(x, y)  # position 0 is the identity
    for pos in (1, 5, 257, 4095):
        y = x.copy()
        L.or_rope(oracle.f32p(y), 128, pos, 1e6)
        # rotate-half pairs (i, i+64) keep their norm and rotate by pos * theta^(-2i/128)
        for i in (0, 1, 17, 63):
            a, b = float(x[i]), float(x[i + 64])
            ang = pos * 1e6 ** (-2.0 * i / 128)
            ea = a * math.cos(ang) - b * math.sin(ang)
            eb = b * math.cos(ang) + a * math.sin(ang)
            tol = 1e-5 * (1 + pos * 1e6 ** (-2.0 * i / 128))
            assert abs(y[i] - ea) < tol and abs(y[i + 64] - eb) < tol
        np.testing.assert_allclose(np.hypot(y[:64], y[64:]), np.hypot(x[:64], x[64:]), rtol=1e-5)


def test_rope_table_matches_rope():
    # metal_inference.rs:140-154 tabulates the same expressions rope() evaluates
    L = oracle.lib()
    tab = np.empty((300, 64, 2), np.float32)
    L.or_rope_table(oracle.f32p(tab), 300, 128, 1e6)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(128).astype(np.float32)
    for pos in (0, 1, 130, 299):
        y = x.copy()
        L.or_rope(oracle.f32p(y), 128, pos, 1e6)
        c, s = tab[pos, :, 0], tab[pos, :, 1]
        z0 = x[:64] * c - x[64:] * s
        z1 = x[64:] * c + x[:64] * s
        np.testing.assert_array_equal(y, np.concatenate([z0, z1]))


def test_softmax_and_silu():
    L = oracle.lib()
    x = np.full(10, 3.5, np.float32)
    L.or_softmax(oracle.f32p(x), 10)
    np.testing.assert_allclose(x, 0.1, rtol=1e-7)
    for v in (-20.0, -1.0, 0.0, 0.5, 7.0):
        assert abs(L.or_silu(v) - v / (1 + math.exp(-v))) <= 1e-6 * max(1, abs(v))


def _attention_f64(q, k, v, H, Hkv, D):
    n = k.shape[0]
    G = H // Hkv
    out = np.zeros(H * D)
    for h in range(H):
        g = h // G
        s = k[:, g * D:(g + 1) * D].astype(np.float64) @ q[h * D:(h + 1) * D] / math.sqrt(D)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * D:(h + 1) * D] = p @ v[:, g * D:(g + 1) * D]
    return out


@pytest.mark.parametrize("n_pos,H,Hkv", [(1, 4, 2), (3, 16, 8), (50, 16, 8), (33, 8, 1), (20, 4, 4)])
def test_attention_against_float64(n_pos, H, Hkv):
    rng = np.random.default_rng(n_pos + H)
    D = 128
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((n_pos, Hkv * D)).astype(np.float32)
    v = rng.standard_normal((n_pos, Hkv * D)).astype(np.float32)
    got = oracle.attention(q, k, v, H, Hkv, D)
    np.testing.assert_allclose(got, _attention_f64(q, k, v, H, Hkv, D), atol=1e-5, rtol=1e-5)
    if n_pos == 1:  # softmax over one position: output is that position's v (GQA head h -> h // G)
        G = H // Hkv
        for h in range(H):
            np.testing.assert_array_equal(got[h * D:(h + 1) * D], v[0, (h // G) * D:(h // G + 1) * D])


def test_argmax_tie_and_nan_rules():
    # main.rs:37-42: best starts at 0 and moves only on strictly greater
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([5, 5, 5], np.float32)) == 0
    assert oracle.argmax(np.array([np.nan, 9, 10], np.float32)) == 0
    assert oracle.argmax(np.array([1, np.nan, 0.5, 7, np.nan], np.float32)) == 3
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0


def test_kv_bytes_formula():
    # bench.rs:118-119: 2 * L * (pos+1) * Hkv * D * 4
    L = oracle.lib()
    c = oracle._Cfg(1024, 3072, 28, 16, 8, 128, 151936, 1e-6, 1e6, 0)
    assert L.or_kv_bytes_at(ctypes.byref(c), 0) == 229376
    assert L.or_kv_bytes_at(ctypes.byref(c), 257) == 229376 * 258


def _bf16_round_f64(u32: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 from the definition: the two bf16 neighbours of x (its upper
    16 bits truncated, and the next value away from zero), the closer one in float64, the one with
    an even last bit on a tie."""
    x = u32.view(np.float32).astype(np.float64)
    lo_bits = (u32 & 0xFFFF0000).astype(np.uint32)
    hi_bits = (lo_bits.astype(np.uint64) + 0x10000).astype(np.uint32)
    lo = lo_bits.view(np.float32).astype(np.float64)
    hi = hi_bits.view(np.float32).astype(np.float64)  # callers pass values below the overflow boundary
    dlo, dhi = np.abs(x - lo), np.abs(hi - x)
    even_lo = ((lo_bits >> 16) & 1) == 0
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ~even_lo)
    return np.where(pick_hi, hi_bits, lo_bits).astype(np.uint32)


def test_round_bf16_definition_and_torch():
    """or_round_bf16 (the oracle's bf16 KV cache rounding): nearest bf16, ties to even, against
    the float64 definition and against torch's float32 -> bfloat16 conversion, on every bf16
    value with the low halves that decide rounding (0, just below / at / just above the tie,
    all ones), plus random patterns; NaN stays NaN"""
    torch = pytest.importorskip("torch")
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    u = (hi[:, None] | lows[None, :]).ravel()
    u = np.concatenate([u, np.random.default_rng(3).integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)])
    got = np.array([oracle.lib().or_round_bf16(float(v)) for v in u.view(np.float32)], np.float32).view(np.uint32)
    ref_t = torch.from_numpy(u.view(np.float32).copy()).to(torch.bfloat16).to(torch.float32).numpy().view(np.uint32)
    nan = np.isnan(u.view(np.float32))
    assert np.all(np.isnan(got.view(np.float32)[nan]))
    np.testing.assert_array_equal(got[~nan], ref_t[~nan])
    finite = np.isfinite(u.view(np.float32)) & (np.abs(u.view(np.float32)) < 3.3e38)
    np.testing.assert_array_equal(got[finite], _bf16_round_f64(u[finite]))
    # ties go to the even neighbour in both directions
    assert oracle.lib().or_round_bf16(1.0 + 2.0 ** -8) == 1.0
    assert oracle.lib().or_round_bf16(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6
