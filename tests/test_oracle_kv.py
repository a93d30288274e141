"""Pins of the KV page layout (aien-kv-cache) and of prand through the reference's own digests.

Known answers: qwen3_moe_omega.rs:5881-5911 (`exported_kv_bytes_match_the_digests_recorded_on_main`):
positions 0..37 of every layer filled with prand rows, the HostPagedPoolV1 export hashed with
FNV-1a 64: tiny geometry 49,152 B -> 0xbbf5a8d45a909242, 30B geometry 4,718,592 B ->
0x60da5a45da835b1a.
"""
import ctypes as C

import numpy as np
import pytest


def rows(oracle, seed, n):
    L = oracle.lib()
    return np.array([L.oref_prand(seed, i) for i in range(n)], dtype=np.float32)


def rows_fast(seed, n):
    M = (1 << 64) - 1
    idx = np.arange(n, dtype=np.uint64)
    x = (np.uint64((seed * 0x9E3779B97F4A7C15) & M) + idx + np.uint64(1))
    x ^= x >> np.uint64(29)
    x = x * np.uint64(0xBF58476D1CE4E5B9)
    x ^= x >> np.uint64(32)
    return ((x & np.uint64(0xFFFF)).astype(np.float32) / np.float32(32768.0)) - np.float32(1.0)


@pytest.mark.parametrize("layers,kv_heads,want", [
    (2, 1, (49_152, 0xBBF5A8D45A909242)),
    (48, 4, (4_718_592, 0x60DA5A45DA835B1A)),
])
def test_exported_kv_bytes_match_the_reference_digests(oracle, layers, kv_heads, want):
    L = oracle.lib()
    hd, bs = 128, 16
    kvd = kv_heads * hd
    lay = oracle.kv_layout(4, bs, layers, kv_heads, hd)   # HostPoolKv::new(&g, 64): 4 blocks
    pool = np.zeros(lay.pool_bytes, dtype=np.uint8)
    assert rows_fast(5, 16).tolist() == rows(oracle, 5, 16).tolist()
    for pos in range(37):
        for l in range(layers):
            s = pos * 100 + l
            k = rows_fast(s, kvd)
            v = rows_fast(s + 7, kvd)
            L.oref_kv_write_token(oracle.ptr(pool), C.byref(lay), pos // bs, l, pos % bs, kvd,
                                  oracle.ptr(k), oracle.ptr(v))
    n = ((37 + bs - 1) // bs) * lay.block_stride_bytes
    payload = pool[:n]
    assert (payload.size, oracle.fnv1a64(payload)) == want


def test_layout_strides_match_an_independent_offset_formula(oracle):
    # tests/paged_attention_parity.rs:15-160 restates the offset independently; so does this:
    # offset = block*BS + layer*LS + isV*PS + token*TS + head*HS + dim*2 with HS = hd*2,
    # TS = kvh*HS, PS = bs*TS, LS = 2*PS, BS = layers*LS.
    import ctypes as C
    L = oracle.lib()
    for (nb, bs, layers, kvh, hd) in [(3, 16, 48, 4, 128), (5, 8, 2, 1, 64), (2, 16, 28, 4, 128)]:
        lay = oracle.kv_layout(nb, bs, layers, kvh, hd)
        HS = hd * 2
        TS = kvh * HS
        PS = bs * TS
        LS = 2 * PS
        BS = layers * LS
        assert (lay.head_stride_bytes, lay.token_stride_bytes, lay.kv_plane_stride_bytes,
                lay.layer_stride_bytes, lay.block_stride_bytes, lay.pool_bytes) == \
            (HS, TS, PS, LS, BS, nb * BS)
        rng = np.random.default_rng(nb)
        for _ in range(50):
            b, l, v, t, h, d = (int(rng.integers(nb)), int(rng.integers(layers)),
                                int(rng.integers(2)), int(rng.integers(bs)), int(rng.integers(kvh)),
                                int(rng.integers(hd)))
            assert L.oref_kv_element_offset(C.byref(lay), b, l, v, t, h, d) == \
                b * BS + l * LS + v * PS + t * TS + h * HS + d * 2
    # the 30B page: HS 256, TS 1 KiB, PS 16 KiB, LS 32 KiB, BS 1.5 MiB
    lay = oracle.kv_layout(1, 16, 48, 4, 128)
    assert (lay.token_stride_bytes, lay.kv_plane_stride_bytes, lay.layer_stride_bytes,
            lay.block_stride_bytes) == (1024, 16384, 32768, 1572864)


def test_write_then_read_round_trips_through_bf16(oracle):
    import ctypes as C
    L = oracle.lib()
    lay = oracle.kv_layout(2, 16, 3, 4, 128)
    pool = np.zeros(lay.pool_bytes, dtype=np.uint8)
    rng = np.random.default_rng(0)
    k = rng.standard_normal(512).astype(np.float32)
    v = rng.standard_normal(512).astype(np.float32)
    L.oref_kv_write_token(oracle.ptr(pool), C.byref(lay), 1, 2, 7, 512, oracle.ptr(k), oracle.ptr(v))
    k2 = np.zeros(512, np.float32)
    v2 = np.zeros(512, np.float32)
    L.oref_kv_read_token(oracle.ptr(pool), C.byref(lay), 1, 2, 7, 512, oracle.ptr(k2), oracle.ptr(v2))
    np.testing.assert_array_equal(k2, oracle.bf16_to_f32(oracle.f32_to_bf16(k)))
    np.testing.assert_array_equal(v2, oracle.bf16_to_f32(oracle.f32_to_bf16(v)))
    assert int((pool != 0).sum()) > 0
    off = L.oref_kv_element_offset(C.byref(lay), 1, 2, 1, 7, 0, 0)
    np.testing.assert_array_equal(pool[off:off + 1024].view(np.uint16), oracle.f32_to_bf16(v))
