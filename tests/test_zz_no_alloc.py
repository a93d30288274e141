"""The no-allocation paged attention (omega_gpu_paged_attention_batch_dev_noalloc) against the
entry point it varies, omega_gpu_paged_attention_batch_dev, through the C-ABI.

Both run the same kernels with the same split plan; only the partials' address differs (a static
device array instead of the library's growable scratch), so the outputs must be bit-identical.
Two calls in a row, the second on a smaller batch with shorter contexts (the array keeps the
first call's partials, which the second must not read), each also held to the oracle's f64
attention (max abs error over max abs value <= 2e-3, the paged attention's bar). The library's
allocation counters must not move across the no-allocation calls, and a shape whose partials
exceed the array is refused with TOO_LARGE before any device work (all its buffers are still
sized for the call).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3
QH, KVH, HD = 32, 4, 128
TOO_LARGE = -2


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def layout(omega, lay):
    return omega.KvLayout(lay.block_stride_bytes, lay.layer_stride_bytes, lay.kv_plane_stride_bytes,
                          lay.token_stride_bytes, lay.head_stride_bytes, lay.pool_bytes,
                          lay.num_blocks, lay.num_layers, lay.block_size)


def call(omega, fn, pool_dev, L, q, tabs, lens, layer):
    """One call of `fn` on device copies of (q, tabs, lens); returns (rc, out or None)."""
    seqs, maxb = tabs.shape
    bufs = [omega.DeviceBuffer.from_array(x) for x in (q, tabs.astype(np.int32), lens.astype(np.int32))]
    od = omega.DeviceBuffer(q.nbytes)
    try:
        rc = fn(bufs[0].ptr, pool_dev.ptr, C.byref(L), bufs[1].ptr, bufs[2].ptr, maxb, seqs,
                int(lens.max()), layer, QH, KVH, HD, od.ptr)
        out = od.download(np.float32, q.size).reshape(seqs, QH * HD) if rc == 0 else None
    finally:
        for b in bufs + [od]:
            b.free()
    return rc, out


def test_noalloc_matches_the_allocating_entry_on_two_calls(omega, oracle):
    lib = omega.lib()
    rng = np.random.default_rng(77)
    nb, layer = 1024, 1
    lay = oracle.kv_layout(nb, 16, 2, KVH, HD)
    host = oracle.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    L = layout(omega, lay)
    pool = omega.DeviceBuffer.from_array(host)
    # the larger call first, then a smaller batch with shorter contexts
    cases = [np.array([3000, 17, 1, 2048, 777, 16, 1500, 2999], np.int32), np.array([5, 300, 33], np.int32)]
    try:
        for i, lens in enumerate(cases):
            maxb = int((lens.max() + 15) // 16)
            tabs = np.stack([rng.permutation(nb)[:maxb] for _ in lens]).astype(np.int32)
            q = rng.standard_normal((lens.size, QH * HD)).astype(np.float32)
            s0 = omega.alloc_stats()
            rc, got = call(omega, lib.omega_gpu_paged_attention_batch_dev_noalloc, pool, L, q, tabs, lens, layer)
            assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
            s1 = omega.alloc_stats()
            assert s1 == s0, (s0, s1)  # no allocation, no free, no refusal
            rc, want = call(omega, lib.omega_gpu_paged_attention_batch_dev, pool, L, q, tabs, lens, layer)
            assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
            assert np.isfinite(got).all()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}: outputs differ"
            for b in range(lens.size):
                ref = np.zeros(QH * HD, np.float32)
                oracle.lib().oref_paged_attention(oracle.ptr(np.ascontiguousarray(q[b])), oracle.ptr(host),
                                                  C.byref(lay), oracle.ptr(tabs[b]), int(lens[b]), layer, QH, KVH,
                                                  HD, oracle.ptr(ref))
                e = rel_err(got[b], ref)
                assert e <= TOL, (i, b, int(lens[b]), e)
    finally:
        pool.free()


def test_noalloc_refuses_partials_beyond_its_array(omega, oracle):
    # 1024 sequences of 32 tokens: one split each, 1024 x 32 heads x 528 B = 17.3 MB > 16 MiB.
    # Every buffer is sized for the call, so nothing is out of bounds even if it ran.
    lib = omega.lib()
    rng = np.random.default_rng(78)
    nb, seqs, ctx = 64, 1024, 32
    lay = oracle.kv_layout(nb, 16, 1, KVH, HD)
    host = oracle.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    L = layout(omega, lay)
    pool = omega.DeviceBuffer.from_array(host)
    try:
        tabs = rng.integers(0, nb, (seqs, ctx // 16)).astype(np.int32)
        lens = np.full(seqs, ctx, np.int32)
        q = rng.standard_normal((seqs, QH * HD)).astype(np.float32)
        rc, _ = call(omega, lib.omega_gpu_paged_attention_batch_dev_noalloc, pool, L, q, tabs, lens, 0)
        assert rc == TOO_LARGE, rc
        assert "static scratch" in omega._s(lib.omega_gpu_attention_last_error())
        # a smaller batch on the same pool still runs
        rc, got = call(omega, lib.omega_gpu_paged_attention_batch_dev_noalloc, pool, L, q[:4], tabs[:4], lens[:4], 0)
        assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
        rc, want = call(omega, lib.omega_gpu_paged_attention_batch_dev, pool, L, q[:4], tabs[:4], lens[:4], 0)
        assert rc == 0 and np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        pool.free()
