"""Pins of the oracle's number codecs and generators against the reference's known answers.

Reference tests restated: inference-abi/src/qwen3_moe.rs:738-778 (e4m3 and bf16),
qwen3_moe_omega.rs:1654-1662 (prand, pinned through the KV digests in test_oracle_kv.py).
"""
import math
import struct

import numpy as np
import pytest


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def test_e4m3_decodes_known_values(oracle):
    # qwen3_moe.rs:738-746
    L = oracle.lib()
    assert L.oref_e4m3_to_f32(0x38) == 1.0
    assert L.oref_e4m3_to_f32(0x30) == 0.5
    assert L.oref_e4m3_to_f32(0xC0) == -2.0
    assert L.oref_e4m3_to_f32(0x7E) == 448.0
    assert L.oref_e4m3_to_f32(0x01) == 2.0 ** -9
    assert math.isnan(L.oref_e4m3_to_f32(0x7F))
    assert math.isnan(L.oref_e4m3_to_f32(0xFF))


def test_e4m3_table_matches_the_ocp_definition(oracle):
    # Independent restatement from the OCP e4m3fn definition (sign, 4-bit exponent bias 7,
    # 3-bit mantissa, subnormals at exponent 0, S.1111.111 NaN).
    t = oracle.e4m3_table()
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            assert math.isnan(t[b])
            continue
        want = s * (m / 8.0) * 2.0 ** -6 if e == 0 else s * (1 + m / 8.0) * 2.0 ** (e - 7)
        assert t[b] == np.float32(want), hex(b)


def test_e4m3_encode_rounds_to_nearest_even_and_saturates(oracle):
    # qwen3_moe.rs:748-767
    L = oracle.lib()
    for bits in range(0, 0x7F):
        for code in (bits, bits | 0x80):
            assert L.oref_f32_to_e4m3(L.oref_e4m3_to_f32(code)) == code, hex(code)
    assert L.oref_f32_to_e4m3(1.0625) == 0x38
    assert L.oref_f32_to_e4m3(1.1875) == 0x3A
    assert L.oref_f32_to_e4m3(1.07) == 0x39
    assert L.oref_f32_to_e4m3(1000.0) == 0x7E
    assert L.oref_f32_to_e4m3(-1000.0) == 0xFE
    assert L.oref_f32_to_e4m3(-0.0) == 0x80
    assert L.oref_f32_to_e4m3(float("nan")) == 0x7F


def test_fast_encoder_equals_the_binary_search(oracle):
    L = oracle.lib()
    t = oracle.e4m3_table()
    vals = []
    # every code, both midpoints, and one ulp either side of each midpoint
    finite = sorted(set(float(v) for v in t if np.isfinite(v) and v >= 0))
    for a, b in zip(finite, finite[1:]):
        mid = np.float32((a + b) / 2)
        for v in (a, b, mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))):
            vals += [float(v), -float(v)]
    rng = np.random.default_rng(7)
    vals += list(rng.standard_normal(20000).astype(np.float32) * 50)
    vals += list((rng.standard_normal(5000) * 2.0 ** -8).astype(np.float32))
    vals += [447.9, 448.0, 464.0, 1e30, -1e30, 2.0 ** -10, 2.0 ** -9 * 0.5, 1e-40]
    for v in vals:
        assert L.oref_f32_to_e4m3_fast(v) == L.oref_f32_to_e4m3(v), v


def test_bf16_rounds_to_nearest_even(oracle):
    # qwen3_moe.rs:770-778
    L = oracle.lib()
    assert L.oref_f32_to_bf16(1.0) == 0x3F80
    assert L.oref_bf16_to_f32(L.oref_f32_to_bf16(1.0 + 1.0 / 256.0)) == 1.0
    assert L.oref_bf16_to_f32(L.oref_f32_to_bf16(1.0 + 3.0 / 256.0)) == 1.0 + 4.0 / 256.0
    assert math.isnan(L.oref_bf16_to_f32(L.oref_f32_to_bf16(float("nan"))))
    # kv-cache variant (aien-kv-cache/src/lib.rs:116-121) agrees on finite values
    rng = np.random.default_rng(1)
    for v in rng.standard_normal(2000).astype(np.float32):
        assert L.oref_kv_f32_to_bf16(float(v)) == L.oref_f32_to_bf16(float(v))


def test_numpy_bf16_helper_equals_the_oracle(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(3000) * 10).astype(np.float32)
    got = oracle.f32_to_bf16(x)
    want = np.array([L.oref_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_prand_is_the_reference_formula(oracle):
    # qwen3_moe_omega.rs:1654-1662, restated here in Python integer arithmetic
    L = oracle.lib()
    M = (1 << 64) - 1
    for seed, idx in [(0, 0), (1, 5), (1234567, 999), (2**63, 17)]:
        x = (seed * 0x9E3779B97F4A7C15 + idx + 1) & M
        x ^= x >> 29
        x = (x * 0xBF58476D1CE4E5B9) & M
        x ^= x >> 32
        want = np.float32(np.float32(x & 0xFFFF) / np.float32(32768.0)) - np.float32(1.0)
        assert L.oref_prand(seed, idx) == want


def test_synthetic_normal_has_the_asked_moments_and_is_deterministic(oracle):
    z = oracle.synth_f32(42, 9, 200_000, 1.0)
    assert abs(float(z.mean())) < 0.01
    assert abs(float(z.std()) - 1.0) < 0.01
    # Irwin-Hall(12) has kurtosis 3 - 1.2/12 = 2.9: close to normal
    k = float(((z - z.mean()) ** 4).mean() / z.var() ** 2)
    assert 2.8 < k < 3.0
    np.testing.assert_array_equal(z, oracle.synth_f32(42, 9, 200_000, 1.0))
    assert not np.array_equal(z, oracle.synth_f32(43, 9, 200_000, 1.0))
    # values are exact multiples of sigma * 2^-16
    np.testing.assert_array_equal(z * 65536, np.round(z * 65536))


def test_synthetic_fp8_tensor_rule(oracle):
    # s = bf16(absmax / 448) per 128x128 block and q = e4m3(W / s): the block max lands on 448
    w, s = oracle.synth_fp8(5, 77, 2, 256, 384, 0.02)
    t = oracle.e4m3_table()
    deq = t[w].reshape(2, 2, 128, 3, 128) * oracle.bf16_to_f32(s)[:, :, None, :, None]
    ref = oracle.synth_f32(5, 77, 2 * 256 * 384, 0.02).reshape(2, 2, 128, 3, 128)
    amax = np.abs(ref).max(axis=(2, 4))
    np.testing.assert_array_equal(s, oracle.f32_to_bf16((amax / np.float32(448)).astype(np.float32)))
    # quantisation error is within half an e4m3 step (relative 2^-4) of each value, times s
    err = np.abs(deq - ref)
    bound = np.maximum(np.abs(ref) * 2.0 ** -4, 2.0 ** -10 * oracle.bf16_to_f32(s)[:, :, None, :, None])
    assert (err <= bound * 1.0001).all()
    assert not ((w & 0x7F) == 0x7F).any(), "no NaN code"
