"""GPU parity of the fused cache's KV park / restore (the HostPagedPoolV1 payload of
qwen3_moe_omega_kvio.rs) against the oracle's row-by-row restatement of rows_to_blocks /
blocks_to_rows. Bars: payload bytes identical to the oracle's for the reference test's
(start, len) cases; import writes exactly the payload's rows (neighbours untouched) and a second
export gives the same bytes; damaged payloads and bad ranges refused before any write; the device
forms equal the host forms."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
LAYERS, MAX_POS, HD, KVH = 2, 256, 128, 4
CASES = [(0, 1), (0, 16), (0, 37), (32, 5), (48, 48), (0, 256), (240, 16)]


def rows_of(layer, head, pos, salt):
    """deterministic u16 rows of (layer, head, pos): K and V [count][128]"""
    p = np.atleast_1d(np.asarray(pos, np.int64))[:, None]
    i = np.arange(HD, dtype=np.int64)[None, :]
    base = layer * 7919 + head * 104729 + p * 131 + i * 3 + salt * 977
    return ((base * 2654435761) >> 7 & 0xFFFF).astype(np.uint16), ((base * 40503 + 17) >> 5 & 0xFFFF).astype(np.uint16)


def fill(cache, salt):
    pos = np.arange(MAX_POS)
    for l in range(LAYERS):
        for h in range(KVH):
            k, v = rows_of(l, h, pos, salt)
            cache.write_rows(l, h, 0, k, v)


@pytest.fixture(scope="module")
def caches(omega):
    a, b = omega.DecodeAttnCache(LAYERS, MAX_POS, 1e6), omega.DecodeAttnCache(LAYERS, MAX_POS, 1e6)
    fill(a, 1)
    yield a, b
    a.free()
    b.free()


@pytest.mark.parametrize("start,length", CASES)
def test_export_matches_the_oracle_and_import_round_trips(omega, oracle, caches, start, length):
    a, b = caches
    g = oracle.PoolBlockGeometry(LAYERS, KVH, HD, 16)
    assert a.payload_len(length) == g.payload_len(length)
    payload, _ = a.export_kv(start, length)
    want = oracle.kv_rows_to_blocks(g, start, length, lambda l, h, p: tuple(r[0] for r in rows_of(l, h, p, 1)))
    np.testing.assert_array_equal(payload, want)
    # the rows the reference's own path would read agree with the payload
    for l, h, p in [(0, 0, start), (LAYERS - 1, KVH - 1, start + length - 1)]:
        k, v = a.read_row(l, h, p)
        rel = p - start
        np.testing.assert_array_equal(k, payload[g.row_offset(rel, l, False, h):][:2 * HD].view("<u2"))
        np.testing.assert_array_equal(v, payload[g.row_offset(rel, l, True, h):][:2 * HD].view("<u2"))
    fill(b, 2)
    b.import_kv(start, length, payload)
    end = start + length
    for l in range(LAYERS):
        for h in range(KVH):
            for p in sorted({start, end - 1, start + length // 2}):
                k, v = b.read_row(l, h, p)
                wk, wv = rows_of(l, h, p, 1)
                np.testing.assert_array_equal(k, wk[0])
                np.testing.assert_array_equal(v, wv[0])
            for p in [q for q in (start - 1, end, end + 1, (end + 15) // 16 * 16 - 1) if 0 <= q < MAX_POS and
                      not start <= q < end]:
                k, v = b.read_row(l, h, p)   # outside the payload: the cache's own rows
                wk, wv = rows_of(l, h, p, 2)
                np.testing.assert_array_equal(k, wk[0])
                np.testing.assert_array_equal(v, wv[0])
    again, _ = b.export_kv(start, length)
    np.testing.assert_array_equal(again, payload)


def test_device_forms_equal_the_host_forms(omega, caches):
    a, b = caches
    start, length = 16, 45
    host, _ = a.export_kv(start, length)
    buf = omega.DeviceBuffer(host.nbytes)
    a.export_kv_dev(start, length, buf.ptr, host.nbytes)
    np.testing.assert_array_equal(buf.download(np.uint8, host.nbytes), host)
    fill(b, 3)
    b.import_kv_dev(start, length, buf.ptr, host.nbytes)
    back, _ = b.export_kv(start, length)
    np.testing.assert_array_equal(back, host)
    k, v = b.read_row(0, 0, start + length)   # past the payload: untouched
    np.testing.assert_array_equal(k, rows_of(0, 0, start + length, 3)[0][0])
    buf.free()


def test_damaged_payloads_and_bad_ranges_are_refused(omega, oracle, caches):
    a, b = caches
    g = oracle.PoolBlockGeometry(LAYERS, KVH, HD, 16)
    payload, _ = a.export_kv(0, 20)
    fill(b, 4)
    before, _ = b.export_kv(0, 32)
    with pytest.raises(omega.OmegaGpuError):
        b.import_kv(0, 20, payload[:-1])                 # wrong size
    bad = payload.copy()
    bad[g.row_offset(20, 1, True, 1) + 3] = 9            # a padding byte
    with pytest.raises(omega.OmegaGpuError, match="padding"):
        b.import_kv(0, 20, bad)
    dev = omega.DeviceBuffer(bad.nbytes)
    dev.upload(bad)
    with pytest.raises(omega.OmegaGpuError, match="padding"):
        b.import_kv_dev(0, 20, dev.ptr, bad.nbytes)
    dev.free()
    after, _ = b.export_kv(0, 32)
    np.testing.assert_array_equal(after, before)          # nothing written
    for start, length in [(3, 4), (0, 0), (240, 17), (256, 1)]:
        with pytest.raises(omega.OmegaGpuError):
            a.export_kv(start, length)
