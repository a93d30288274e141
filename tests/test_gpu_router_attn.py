"""GPU parity of the router, the fused decode attention, the paged attention and the bf16
lm_head GEMV against the CPU oracle.

Bars: router ids bit-exact (and equal to the reference's sequential-f32 ranking whenever the
rank-8 / rank-9 margin exceeds 1e-4), weights and x' within 1e-5 relative; attention and GEMV
outputs within 2e-3 relative (max abs error over max abs value); cache rows bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3
E, H = 128, 2048


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def make_router(omega, oracle, layers, seed, experts=E, shared=0):
    rng = np.random.default_rng(seed)
    r = omega.Router(layers, experts, shared)
    gates, norms = [], []
    for l in range(layers):
        g = oracle.f32_to_bf16((rng.standard_normal((experts + shared, H)) * 0.02).astype(np.float32))
        w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        r.set_layer(l, g, w)
        dir_gu = np.arange(2 * (experts + shared), dtype=np.uint64) + 1000 * (l + 1)
        dir_dn = np.arange(2 * (experts + shared), dtype=np.uint64) + 500000 * (l + 1)
        r.set_directory(l, dir_gu, dir_dn)
        gates.append(g)
        norms.append(w)
    return r, gates, norms


def test_router_ids_are_bit_exact_and_outputs_match(omega, oracle):
    r, gates, norms = make_router(omega, oracle, 3, 1)
    rng = np.random.default_rng(2)
    tight = 0
    for t in range(60):
        l = t % 3
        x = (rng.standard_normal(H) * (1 + t % 5)).astype(np.float32)
        ids, w, info = r.route(l, x, 1e-6)
        want_ids, want_w, post, logits = oracle.route(gates[l], norms[l], x, 1e-6, refined=True)
        np.testing.assert_array_equal(ids, want_ids)
        assert np.abs(w - want_w).max() <= 1e-5 * np.abs(want_w).max()
        srt = np.sort(logits)[::-1]
        if srt[7] - srt[8] > 1e-4:
            f32_ids, _, _, _ = oracle.route(gates[l], norms[l], x, 1e-6, refined=False)
            np.testing.assert_array_equal(ids, f32_ids)
        else:
            tight += 1
        xout, tab_gu, tab_dn = r.read_back()
        np.testing.assert_allclose(xout / np.float32(2.0 ** 64), post, rtol=1e-6, atol=0)
        gu = (np.arange(2 * E, dtype=np.uint64) + 1000 * (l + 1)).reshape(E, 2)
        dn = (np.arange(2 * E, dtype=np.uint64) + 500000 * (l + 1)).reshape(E, 2)
        np.testing.assert_array_equal(tab_gu.reshape(8, 2), gu[ids])
        np.testing.assert_array_equal(tab_dn.reshape(8, 2), dn[ids])
        assert info.weight_bytes == 128 * 2048 * 2
    assert tight < 10
    r.free()


def test_router_ties_go_to_the_lower_id(omega, oracle):
    # a gate with duplicated rows makes exactly tied logits
    r = omega.Router(1)
    rng = np.random.default_rng(3)
    g = oracle.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    g[77] = g[5]
    g[100] = g[5]
    g[5] = oracle.f32_to_bf16((oracle.bf16_to_f32(g[5]) * 4).astype(np.float32))
    g[77] = g[5]
    g[100] = g[5]
    w = np.ones(H, np.float32)
    r.set_layer(0, g, w)
    r.set_directory(0, np.zeros(2 * E, np.uint64), np.zeros(2 * E, np.uint64))
    x = oracle.bf16_to_f32(g[5]).astype(np.float32)   # aligned with row 5: its logit is the max
    ids, _, _ = r.route(0, x, 1e-6)
    want, _, _, _ = oracle.route(g, w, x, 1e-6)
    np.testing.assert_array_equal(ids, want)
    assert list(ids[:3]) == [5, 77, 100]
    r.free()


def test_router_shared_slot_and_256_experts(omega, oracle):
    r, gates, norms = make_router(omega, oracle, 1, 4, experts=128, shared=1)
    x = np.random.default_rng(5).standard_normal(H).astype(np.float32)
    ids, w, _ = r.route(0, x, 1e-6)
    post = oracle.rmsnorm(x, norms[0], 1e-6)
    logits = oracle.router_logits(gates[0], post, refined=True)
    p = oracle.moe_plan(logits[:128].copy(), 1, 128, 8)
    np.testing.assert_array_equal(ids[:8], p["topk_experts"])
    assert ids[8] == 128
    assert abs(w[8] - 1 / (1 + np.exp(-np.float64(logits[128])))) < 1e-6
    r.free()
    r, gates, norms = make_router(omega, oracle, 1, 6, experts=256)
    ids, w, _ = r.route(0, x, 1e-6)
    want, want_w, _, _ = oracle.route(gates[0], norms[0], x, 1e-6)
    np.testing.assert_array_equal(ids, want)
    r.free()


@pytest.mark.parametrize("mutant", [1, 2, 3, 4])
def test_router_mutants_are_caught(omega, oracle, mutant):
    # crates/aien-omega-router/src/lib.rs:461-473
    r, gates, norms = make_router(omega, oracle, 1, 7)
    x = np.random.default_rng(8).standard_normal(H).astype(np.float32)
    want_ids, want_w, post, _ = oracle.route(gates[0], norms[0], x, 1e-6)
    omega.lib().omega_gpu_router_test_set_mutant(mutant)
    try:
        ids, w, _ = r.route(0, x, 1e-6)
        xout, tab_gu, _ = r.read_back()
    finally:
        omega.lib().omega_gpu_router_test_set_mutant(0)
    gu = (np.arange(2 * E, dtype=np.uint64) + 1000).reshape(E, 2)
    caught = (not np.array_equal(ids, want_ids) or np.abs(w - want_w).max() > 1e-3
              or np.abs(xout / 2.0 ** 64 - post).max() > 1e-3
              or not np.array_equal(tab_gu.reshape(8, 2), gu[want_ids]))
    assert caught
    r.free()


def _qkv_row(rng):
    return (rng.standard_normal(5120) * 2).astype(np.float32)


def test_decode_attention_sequence_matches_the_oracle(omega, oracle):
    layers, max_pos, theta = 2, 512, 1e6
    c = omega.DecodeAttnCache(layers, max_pos, theta)
    ref = oracle.Dattn(layers, max_pos, theta)
    rng = np.random.default_rng(9)
    for l in range(layers):
        qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        c.set_norms(l, qn, kn)
        ref.set_norms(l, qn, kn)
    worst = 0.0
    for pos in range(300):
        for l in range(layers):
            qkv = _qkv_row(rng)
            out, info = c.attend(l, pos, qkv, 1e-6)
            want = ref.attend(l, pos, qkv, 1e-6)
            worst = max(worst, rel_err(out, want))
            assert info.kv_bytes == 2 * 4 * (pos + 1) * 256
        if pos in (0, 1, 63, 64, 255, 256, 299):
            for l in range(layers):
                for h in range(4):
                    k, v = c.read_row(l, h, pos)
                    wk, wv = ref.read_row(l, h, pos)
                    np.testing.assert_array_equal(k, wk)
                    np.testing.assert_array_equal(v, wv)
    assert worst <= TOL, worst
    c.free()


def test_decode_attention_long_contexts_match_the_oracle(omega, oracle):
    """The fused kernel where each of its 64 splits holds several pages (crates/aien-omega-dattn/
    src/lib.rs:45-48 allows max_pos up to 131072): positions 0..32767 of one layer filled with
    random bf16 K/V rows through cache_write (both caches hold the same rows), then attention at
    the decode benchmark's contexts (517-600), at about 5000 (5 pages per split) and at 32767
    (32 pages per split); the appended K/V rows bit-exact, outputs within 2e-3."""
    max_pos, theta, fill = 33024, 1e6, 32767
    c = omega.DecodeAttnCache(1, max_pos, theta)
    ref = oracle.Dattn(1, max_pos, theta)
    rng = np.random.default_rng(12)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    c.set_norms(0, qn, kn)
    ref.set_norms(0, qn, kn)
    for h in range(4):
        kr = oracle.f32_to_bf16((2 * rng.standard_normal((fill, 128))).astype(np.float32))
        vr = oracle.f32_to_bf16(rng.standard_normal((fill, 128)).astype(np.float32))
        c.write_rows(0, h, 0, kr, vr)
        ref.write_rows(0, h, 0, kr, vr)
        for p in (0, 15, 16, 4097, fill - 1):
            k, v = c.read_row(0, h, p)
            np.testing.assert_array_equal(k, kr[p])
            np.testing.assert_array_equal(v, vr[p])
    worst = {}
    for pos in (517, 520, 531, 544, 559, 600, 4999, 5000, 5003, fill):
        qkv = _qkv_row(rng)
        out, info = c.attend(0, pos, qkv, 1e-6)
        want = ref.attend(0, pos, qkv, 1e-6)
        worst[pos] = rel_err(out, want)
        assert info.kv_bytes == 2 * 4 * (pos + 1) * 256
        for h in range(4):
            k, v = c.read_row(0, h, pos)
            wk, wv = ref.read_row(0, h, pos)
            np.testing.assert_array_equal(k, wk)
            np.testing.assert_array_equal(v, wv)
    print("fused attention rel err by position:", {p: f"{e:.1e}" for p, e in worst.items()})
    assert max(worst.values()) <= TOL, worst
    c.free()


def test_decode_attention_out_scale_and_cache_rows(omega, oracle):
    c = omega.DecodeAttnCache(1, 256, 1e7)
    c.set_norms(0, np.ones(128, np.float32), np.ones(128, np.float32))
    rng = np.random.default_rng(10)
    kr = oracle.f32_to_bf16(rng.standard_normal((40, 128)).astype(np.float32))
    vr = oracle.f32_to_bf16(rng.standard_normal((40, 128)).astype(np.float32))
    c.write_rows(0, 2, 10, kr, vr)
    for i in (0, 17, 39):
        k, v = c.read_row(0, 2, 10 + i)
        np.testing.assert_array_equal(k, kr[i])
        np.testing.assert_array_equal(v, vr[i])
    qkv = _qkv_row(rng)
    a, _ = c.attend(0, 60, qkv, 1e-6, 1.0)
    b, _ = c.attend(0, 60, qkv, 1e-6, 2.0 ** 64)
    np.testing.assert_allclose(b / 2.0 ** 64, a, rtol=1e-6)
    with pytest.raises(omega.OmegaGpuError):
        c.attend(0, 256, qkv, 1e-6)
    c.free()


@pytest.mark.parametrize("mutant", [1, 2, 3, 4])
def test_decode_attention_mutants_are_caught(omega, oracle, mutant):
    # crates/aien-omega-dattn/src/lib.rs:406-417
    c = omega.DecodeAttnCache(1, 1024, 1e6)
    ref = oracle.Dattn(1, 1024, 1e6)
    ones = np.ones(128, np.float32)
    c.set_norms(0, ones, ones)
    ref.set_norms(0, ones, ones)
    rng = np.random.default_rng(11)
    rows = [_qkv_row(rng) for _ in range(700)]
    omega.lib().omega_gpu_decode_attn_test_set_mutant(mutant)
    worst = 0.0
    try:
        for pos, qkv in enumerate(rows):
            out, _ = c.attend(0, pos, qkv, 1e-6)
            worst = max(worst, rel_err(out, ref.attend(0, pos, qkv, 1e-6)))
    finally:
        omega.lib().omega_gpu_decode_attn_test_set_mutant(0)
    assert worst > 0.01
    c.free()


def test_decode_attention_merge_wait_that_runs_out_is_reported(omega, oracle):
    # test mutant 9: every split merge gives up at once (no poll), as when a split never flags;
    # the call reports CHIP_FAIL with its message and the next call at the same position (a new
    # epoch) matches the oracle
    layers, max_pos, theta = 1, 256, 1e6
    c = omega.DecodeAttnCache(layers, max_pos, theta)
    ref = oracle.Dattn(layers, max_pos, theta)
    rng = np.random.default_rng(21)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    c.set_norms(0, qn, kn)
    ref.set_norms(0, qn, kn)
    rows = [_qkv_row(rng) for _ in range(40)]
    for pos in range(39):
        c.attend(0, pos, rows[pos], 1e-6)
        ref.attend(0, pos, rows[pos], 1e-6)
    lib = omega.lib()
    lib.omega_gpu_decode_attn_test_set_mutant(9)
    try:
        with pytest.raises(omega.OmegaGpuError, match="ran out of waits"):
            c.attend(0, 39, rows[39], 1e-6)
    finally:
        lib.omega_gpu_decode_attn_test_set_mutant(0)
    out, _ = c.attend(0, 39, rows[39], 1e-6)
    want = ref.attend(0, 39, rows[39], 1e-6)
    assert rel_err(out, want) <= TOL
    c.free()


def _paged_pool(oracle, rng, nb, layers, kvh=4):
    lay = oracle.kv_layout(nb, 16, layers, kvh, 128)
    pool = oracle.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32))
    return lay, pool.view(np.uint8)


def _omega_layout(omega, lay):
    return omega.KvLayout(lay.block_stride_bytes, lay.layer_stride_bytes, lay.kv_plane_stride_bytes,
                          lay.token_stride_bytes, lay.head_stride_bytes, lay.pool_bytes,
                          lay.num_blocks, lay.num_layers, lay.block_size)


def test_paged_attention_single_and_batch(omega, oracle):
    rng = np.random.default_rng(12)
    layers, nb = 3, 200
    lay, pool = _paged_pool(oracle, rng, nb, layers)
    L = _omega_layout(omega, lay)
    lib = omega.lib()
    # single sequence, permuted pages
    ctx = 517
    blocks = rng.permutation(nb)[: (ctx + 15) // 16].astype(np.uint32)
    q = rng.standard_normal(32 * 128).astype(np.float32)
    out = np.zeros(32 * 128, np.float32)
    info = omega.AttnInfo()
    rc = lib.omega_gpu_paged_attention_bf16(omega.ptr(q), omega.ptr(pool), C.byref(L),
                                            omega.ptr(blocks), blocks.size, ctx, 2, 32, 4, 128,
                                            omega.ptr(out), C.byref(info))
    assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
    want = np.zeros(32 * 128, np.float32)
    oracle.lib().oref_paged_attention(oracle.ptr(q), oracle.ptr(pool), C.byref(lay),
                                      oracle.ptr(blocks.astype(np.int32)), ctx, 2, 32, 4, 128,
                                      oracle.ptr(want))
    assert rel_err(out, want) <= TOL
    assert info.kv_source == 0 and info.kv_blocks_logical == blocks.size
    # ragged batch; the tables share pages (prefix sharing) and pad with -1
    seqs, maxb = 5, 40
    lens = np.array([1, 16, 17, 300, 640], np.int32)
    tabs = np.full((seqs, maxb), -1, np.int32)
    for b in range(seqs):
        nbk = (lens[b] + 15) // 16
        tabs[b, :nbk] = rng.permutation(nb)[:nbk]
    tabs[4, :3] = tabs[3, :3]
    qb = rng.standard_normal(seqs * 32 * 128).astype(np.float32)
    outb = np.zeros_like(qb)
    rc = lib.omega_gpu_paged_attention_batch_bf16(omega.ptr(qb), omega.ptr(pool), C.byref(L),
                                                  omega.ptr(tabs), omega.ptr(lens), maxb, seqs, 1,
                                                  32, 4, 128, omega.ptr(outb), C.byref(info))
    assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
    for b in range(seqs):
        want = np.zeros(32 * 128, np.float32)
        oracle.lib().oref_paged_attention(oracle.ptr(qb[b * 4096:(b + 1) * 4096].copy()),
                                          oracle.ptr(pool), C.byref(lay),
                                          oracle.ptr(tabs[b].copy()), int(lens[b]), 1, 32, 4, 128,
                                          oracle.ptr(want))
        assert rel_err(outb[b * 4096:(b + 1) * 4096], want) <= TOL, b
    assert info.kv_blocks_unique < info.kv_blocks_logical
    # refusals: a table entry outside the pool, a context longer than the table
    bad = tabs.copy()
    bad[0, 0] = nb
    assert lib.omega_gpu_paged_attention_batch_bf16(omega.ptr(qb), omega.ptr(pool), C.byref(L),
                                                    omega.ptr(bad), omega.ptr(lens), maxb, seqs,
                                                    1, 32, 4, 128, omega.ptr(outb),
                                                    C.byref(info)) == -1


def test_paged_attention_over_the_resident_pool(omega, oracle):
    # the pool from omega_gpu_attention_pool_alloc is read in place (no staging)
    rng = np.random.default_rng(13)
    lay, pool_np = _paged_pool(oracle, rng, 64, 2)
    L = _omega_layout(omega, lay)
    lib = omega.lib()
    p = C.c_void_p()
    assert lib.omega_gpu_attention_pool_alloc(lay.pool_bytes, C.byref(p)) == 0
    try:
        C.memmove(p, pool_np.ctypes.data, lay.pool_bytes)
        ctx = 333
        blocks = rng.permutation(64)[: (ctx + 15) // 16].astype(np.uint32)
        q = rng.standard_normal(4096).astype(np.float32)
        out = np.zeros(4096, np.float32)
        info = omega.AttnInfo()
        assert lib.omega_gpu_paged_attention_bf16(omega.ptr(q), p, C.byref(L), omega.ptr(blocks),
                                                  blocks.size, ctx, 1, 32, 4, 128, omega.ptr(out),
                                                  C.byref(info)) == 0
        want = np.zeros(4096, np.float32)
        oracle.lib().oref_paged_attention(oracle.ptr(q), oracle.ptr(pool_np), C.byref(lay),
                                          oracle.ptr(blocks.astype(np.int32)), ctx, 1, 32, 4, 128,
                                          oracle.ptr(want))
        assert rel_err(out, want) <= TOL
        assert info.kv_bytes_staged == 0
    finally:
        lib.omega_gpu_attention_pool_free()


def test_bf16_lm_head_gemv(omega, oracle):
    n, k = 151936, 2048
    w = oracle.synth_bf16(3, 2, (n, k), 0.02)
    t = omega.Bf16Tensor.upload(n, k, w)
    x = np.random.default_rng(14).standard_normal(k).astype(np.float32)
    y, info = t.gemv_f32(x)
    want = oracle.bf16_gemv(w, x, threads=16)
    assert rel_err(y, want) <= TOL
    assert oracle.argmax(y) == oracle.argmax(want)
    td = omega.Bf16Tensor.synth(n, k, 3, 2, 0.02)
    np.testing.assert_array_equal(td.gemv_f32(x)[0], y)       # device generator == host
    xb = oracle.f32_to_bf16(x)
    yb, _ = t.gemv_bf16(xb)
    np.testing.assert_array_equal(yb, t.gemv_f32(oracle.bf16_to_f32(xb))[0])
    assert info.weight_bytes == n * k * 2
    # odd n (padded tile) and the NaN refusal
    t2 = omega.Bf16Tensor.upload(100, 256, w[:100, :256].copy())
    np.testing.assert_allclose(t2.gemv_f32(x[:256].copy())[0],
                               oracle.bf16_gemv(w[:100, :256].copy(), x[:256].copy()), rtol=1e-5,
                               atol=1e-6)
    bad = w[:100, :256].copy()
    bad[3, 4] = 0x7FC0
    with pytest.raises(omega.OmegaGpuError):
        omega.Bf16Tensor.upload(100, 256, bad)
    t.free()
    td.free()
    t2.free()


def test_serving_reservation_bounds_seal_and_counters(omega, oracle):
    # omega_gpu_reserve_serving sizes the host-buffer paged call's buffers for its bounds; calls
    # inside them allocate nothing more, a call past them is refused (TOO_LARGE), the seal refuses
    # any later growth of the library's buffers (a stale refusal), and release lifts both
    rng = np.random.default_rng(31)
    layers, nb = 2, 200
    lay, pool = _paged_pool(oracle, rng, nb, layers)
    L = _omega_layout(omega, lay)
    lib = omega.lib()

    def call(seqs, ctx):
        lens = np.full(seqs, ctx, np.int32)
        maxb = (ctx + 15) // 16
        tabs = np.stack([rng.permutation(nb)[:maxb] for _ in range(seqs)]).astype(np.int32)
        q = rng.standard_normal(seqs * 32 * 128).astype(np.float32)
        out = np.zeros_like(q)
        info = omega.AttnInfo()
        rc = lib.omega_gpu_paged_attention_batch_bf16(omega.ptr(q), omega.ptr(pool), C.byref(L), omega.ptr(tabs),
                                                      omega.ptr(lens), maxb, seqs, 1, 32, 4, 128, omega.ptr(out),
                                                      C.byref(info))
        return rc, omega._s(lib.omega_gpu_attention_last_error())

    with pytest.raises(omega.OmegaGpuError):
        omega.reserve_serving(max_context=640, max_seqs=4, num_q_heads=32, num_kv_heads=4, head_dim=64,
                              kv_block_size=16, max_rows=1, max_k=2048, max_n=2048, max_n_one_row=0, kernel_slots=8)
    try:
        omega.reserve_serving(max_context=640, max_seqs=4, num_q_heads=32, num_kv_heads=4, head_dim=128,
                              kv_block_size=16, max_rows=1, max_k=2048, max_n=2048, max_n_one_row=0, kernel_slots=8)
        s0 = omega.alloc_stats()
        assert call(4, 640)[0] == 0 and call(2, 100)[0] == 0
        assert omega.alloc_stats()["allocs"] == s0["allocs"]     # inside the bounds: nothing allocated
        rc, err = call(5, 64)
        assert rc == -2 and "reservation exceeded" in err          # past max_seqs
        assert call(1, 641 + 15)[0] == -2                          # past max_context
        omega.serving_seal()
        assert call(3, 600)[0] == 0
        # growth of the shared scratch by another family: a prefill attention of 1024 tokens
        # ending at position 131072 sizes its partials for 256 chunks per token (about 4.4 GB),
        # more than any other call here ever holds, so the sealed library must refuse it whatever
        # ran before (and before any of its work reaches the device)
        from omega_amd import prefill as pf
        cache = omega.DecodeAttnCache(2, 131072, 1e6)
        try:
            with pytest.raises(omega.OmegaGpuError, match="reservation exceeded"):
                pf.PrefillAttention(cache).attend(0, 131072 - 1024, 1024, np.zeros((1024, 5120), np.float32),
                                                  1e-6, 1.0)
        finally:
            cache.free()
        assert omega.alloc_stats()["stale_refusals"] == s0["stale_refusals"] + 1
    finally:
        omega.serving_release()
    assert call(5, 64)[0] == 0                                     # released: bounds and seal lifted
