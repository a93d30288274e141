"""The HostPagedPoolV1 payload restatement (oracle/pyoracle.py, qwen3_moe_omega_kvio.rs) on the
CPU: the reference's own module tests (round trip, damaged payloads, the pool-layout identity)
restated, plus known offsets worked out by hand and the stride identity with the kv-cache layout
oracle (pinned by the reference's FNV digests)."""
import numpy as np
import pytest


def row_word(layer, head, pos, value, i):
    # the reference test's fake fused cache (qwen3_moe_omega_kvio.rs:215-218)
    return (((layer * 7 + head * 3 + pos * 11 + int(value) * 5 + i) % 65521) | 1) & 0xFFFF


def reader(g):
    def read_row(layer, head, pos):
        k = np.array([row_word(layer, head, pos, False, i) for i in range(g.head_dim)], np.uint16)
        v = np.array([row_word(layer, head, pos, True, i) for i in range(g.head_dim)], np.uint16)
        return k, v
    return read_row


@pytest.fixture
def g(oracle):
    return oracle.PoolBlockGeometry(3, 2, 4, 16)


@pytest.mark.parametrize("geom", [(3, 2, 4, 16), (48, 4, 128, 16)])
def test_geometry_is_the_kv_cache_pool_layout(oracle, geom):
    layers, heads, dim, bs = geom
    pg = oracle.PoolBlockGeometry(layers, heads, dim, bs)
    lay = oracle.kv_layout(4, bs, layers, heads, dim)
    assert (pg.block_stride, pg.layer_stride, pg.kv_plane_stride, pg.token_stride, pg.head_stride) == (
        lay.block_stride_bytes, lay.layer_stride_bytes, lay.kv_plane_stride_bytes, lay.token_stride_bytes,
        lay.head_stride_bytes)


def test_known_offsets(g):
    # block stride 3 layers x 2 planes x 16 tokens x 2 heads x 4 dims x 2 B = 1536; layer 512;
    # plane 256; token 16; head 8: position 17 -> block 1, token 1
    assert g.row_offset(17, 2, True, 1) == 1536 + 2 * 512 + 256 + 16 + 8
    assert g.row_offset(0, 0, False, 0) == 0
    assert g.row_offset(15, 0, True, 1) == 256 + 15 * 16 + 8
    assert g.payload_len(37) == 3 * 1536 and g.payload_len(16) == 1536


@pytest.mark.parametrize("start,length", [(0, 1), (0, 16), (0, 37), (32, 5), (48, 48)])
def test_rows_round_trip_through_the_payload(oracle, g, start, length):
    payload = oracle.kv_rows_to_blocks(g, start, length, reader(g))
    assert payload.size == g.payload_len(length)
    oracle.kv_check_payload(g, length, payload)
    # the first K row little-endian at offset 0, the first V row at the plane stride
    assert int(payload[0]) | int(payload[1]) << 8 == row_word(0, 0, start, False, 0)
    v0 = g.kv_plane_stride
    assert int(payload[v0]) | int(payload[v0 + 1]) << 8 == row_word(0, 0, start, True, 0)
    seen = []

    def write_rows(layer, head, k, v):
        for rel in range(length):
            for i in range(g.head_dim):
                assert k[rel, i] == row_word(layer, head, start + rel, False, i)
                assert v[rel, i] == row_word(layer, head, start + rel, True, i)
        seen.append((layer, head))

    oracle.kv_blocks_to_rows(g, start, length, payload, write_rows)
    assert len(seen) == g.layers * g.kv_heads

    def from_payload(layer, head, pos):
        rel = pos - start
        at_k, at_v = g.row_offset(rel, layer, False, head), g.row_offset(rel, layer, True, head)
        return payload[at_k:at_k + 2 * g.head_dim].view("<u2"), payload[at_v:at_v + 2 * g.head_dim].view("<u2")

    np.testing.assert_array_equal(oracle.kv_rows_to_blocks(g, start, length, from_payload), payload)


def test_damaged_payloads_are_refused_before_any_write(oracle, g):
    payload = oracle.kv_rows_to_blocks(g, 0, 20, lambda l, h, p: (np.full(4, 0x3F80, np.uint16),
                                                                  np.full(4, 0x4000, np.uint16)))
    writes = []
    with pytest.raises(ValueError):
        oracle.kv_blocks_to_rows(g, 0, 20, payload[:-1], lambda *a: writes.append(1))
    bad = payload.copy()
    bad[g.row_offset(20, 1, True, 1) + 3] = 9
    with pytest.raises(ValueError, match="padding"):
        oracle.kv_blocks_to_rows(g, 0, 20, bad, lambda *a: writes.append(1))
    assert not writes
    oracle.kv_zero_padding(g, 20, bad)
    oracle.kv_check_payload(g, 20, bad)
    np.testing.assert_array_equal(bad, payload)
    with pytest.raises(ValueError):
        oracle.kv_rows_to_blocks(g, 3, 4, reader(g))
    with pytest.raises(ValueError):
        oracle.kv_rows_to_blocks(g, 0, 0, reader(g))


def test_a_swapped_plane_is_caught(oracle, g):
    # a planted mistake (K and V planes exchanged while writing) changes the payload's bytes
    good = oracle.kv_rows_to_blocks(g, 0, 5, reader(g))
    swapped = oracle.kv_rows_to_blocks(g, 0, 5, lambda l, h, p: reader(g)(l, h, p)[::-1])
    assert not np.array_equal(good, swapped)
