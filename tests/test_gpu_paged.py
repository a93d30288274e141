"""GPU parity of the matrix-core paged decode attention (GQA 32 q / 4 kv heads of 128 over
16-token pages of the aien-kv-cache layout) against the CPU oracle's f64 attention.

Cases: the configuration-3 shapes (batch 1, 8, 32 at contexts up to 32768, page tables drawn
from a free-page pool), ragged contexts that end inside a page whose unwritten slots hold NaN
and infinity, splits longer than 64 pages (the page-table window moves), and the test mutants
(V one position late, the split combine without its maxima) that the parity bar must catch.
Bar: max abs error over max abs value <= 2e-3 (attention_out in fp32 accumulate).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3
QH, KVH, HD = 32, 4, 128


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def _omega_layout(omega, lay):
    return omega.KvLayout(lay.block_stride_bytes, lay.layer_stride_bytes, lay.kv_plane_stride_bytes,
                          lay.token_stride_bytes, lay.head_stride_bytes, lay.pool_bytes,
                          lay.num_blocks, lay.num_layers, lay.block_size)


class Pool:
    """A host pool of N(0,1) bf16 rows and its device copy."""

    def __init__(self, omega, oracle, rng, nb, layers):
        self.lay = oracle.kv_layout(nb, 16, layers, KVH, HD)
        self.host = oracle.f32_to_bf16(
            rng.standard_normal(self.lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
        self.L = _omega_layout(omega, self.lay)
        self.dev = omega.DeviceBuffer.from_array(self.host)

    def poison_tail(self, oracle, table, ctx, layer):
        """NaN / inf bf16 in the slots past `ctx` of the sequence's last page (every head, K and
        V), in the host pool and the device copy."""
        last = int(table[(ctx - 1) // 16])
        lay = self.lay
        for t in range(ctx % 16 or 16, 16):
            for plane in (0, 1):
                off = (last * lay.block_stride_bytes + layer * lay.layer_stride_bytes +
                       plane * lay.kv_plane_stride_bytes + t * lay.token_stride_bytes)
                row = self.host[off:off + KVH * 256].view(np.uint16)
                row[0::2] = 0x7FC0  # NaN
                row[1::2] = 0x7F80  # +inf
        self.dev.upload(self.host)


def run_dev(omega, pool, q, tabs, lens, layer):
    lib = omega.lib()
    seqs, maxb = tabs.shape
    qd = omega.DeviceBuffer.from_array(q)
    td = omega.DeviceBuffer.from_array(tabs.astype(np.int32))
    ld = omega.DeviceBuffer.from_array(lens.astype(np.int32))
    od = omega.DeviceBuffer(q.nbytes)
    rc = lib.omega_gpu_paged_attention_batch_dev(qd.ptr, pool.dev.ptr, C.byref(pool.L), td.ptr,
                                                 ld.ptr, maxb, seqs, int(lens.max()), layer, QH,
                                                 KVH, HD, od.ptr)
    assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
    return od.download(np.float32, q.size)


def oracle_out(oracle, pool, q, table, ctx, layer):
    want = np.zeros(QH * HD, np.float32)
    oracle.lib().oref_paged_attention(oracle.ptr(np.ascontiguousarray(q)), oracle.ptr(pool.host),
                                      C.byref(pool.lay), oracle.ptr(table.astype(np.int32)), int(ctx),
                                      layer, QH, KVH, HD, oracle.ptr(want))
    return want


# all nine configuration-3 points (batch {1, 8, 32} x context {2048, 8192, 32768}); the oracle
# checks every sequence up to 8 x 8192 and three sampled sequences beyond
@pytest.mark.parametrize("seqs,ctx,check", [(1, 2048, None), (1, 8192, None), (1, 32768, None),
                                            (8, 2048, None), (8, 8192, None), (8, 32768, (0, 3, 7)),
                                            (32, 2048, None), (32, 8192, (0, 13, 31)),
                                            (32, 32768, (0, 17, 31))])
def test_config3_shapes(omega, oracle, seqs, ctx, check):
    rng = np.random.default_rng(seqs * 7 + ctx)
    nb = 4096
    pool = Pool(omega, oracle, rng, nb, 2)
    pages = ctx // 16
    # every sequence's table is a random permutation of free pages while the pool lasts, then
    # pages are reused (the kernel never assumes distinct pages)
    tabs = np.stack([rng.permutation(nb)[:pages] if pages <= nb else rng.integers(0, nb, pages)
                     for _ in range(seqs)]).astype(np.int32)
    lens = np.full(seqs, ctx, np.int32)
    q = rng.standard_normal((seqs, QH * HD)).astype(np.float32)
    out = run_dev(omega, pool, q, tabs, lens, 1).reshape(seqs, QH * HD)
    assert np.isfinite(out).all()
    for b in (range(seqs) if check is None else check):
        e = rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], ctx, 1))
        assert e <= TOL, (b, e)


def test_ragged_contexts_ignore_unwritten_slots(omega, oracle):
    rng = np.random.default_rng(31)
    nb = 512
    pool = Pool(omega, oracle, rng, nb, 3)
    lens = np.array([1, 5, 16, 17, 333, 1000, 2047, 4099], np.int32)
    maxb = int((lens.max() + 15) // 16) + 3
    tabs = np.full((lens.size, maxb), -1, np.int32)
    free = rng.permutation(nb)  # disjoint pages: a poisoned tail belongs to its sequence only
    used = 0
    for b, cl in enumerate(lens):
        n_b = (cl + 15) // 16
        tabs[b, :n_b] = free[used:used + n_b]
        used += n_b
    for b, cl in enumerate(lens):
        if cl % 16:
            pool.poison_tail(oracle, tabs[b], int(cl), 2)
    q = rng.standard_normal((lens.size, QH * HD)).astype(np.float32)
    out = run_dev(omega, pool, q, tabs, lens, 2).reshape(lens.size, QH * HD)
    assert np.isfinite(out).all()
    for b, cl in enumerate(lens):
        e = rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], cl, 2))
        assert e <= TOL, (b, int(cl), e)
    # ctx 1: the output of every head is the single V row
    lay = pool.lay
    off = int(tabs[0, 0]) * lay.block_stride_bytes + 2 * lay.layer_stride_bytes + lay.kv_plane_stride_bytes
    v0 = oracle.bf16_to_f32(pool.host[off:off + KVH * 256].view(np.uint16).copy()).reshape(KVH, HD)
    np.testing.assert_allclose(out[0].reshape(QH, HD), np.repeat(v0, QH // KVH, axis=0), rtol=1e-6, atol=1e-6)


def test_splits_longer_than_the_table_window(omega, oracle):
    # 128 (seq, kv head) pairs -> 16 splits; 2560 pages per sequence -> 160 pages per split, so
    # each split crosses two 64-entry windows of its page table
    rng = np.random.default_rng(32)
    nb = 2048
    pool = Pool(omega, oracle, rng, nb, 1)
    seqs, ctx = 32, 40960 - 7
    pages = (ctx + 15) // 16
    tabs = rng.integers(0, nb, (seqs, pages)).astype(np.int32)
    lens = np.full(seqs, ctx, np.int32)
    lens[5] = 16 * 65 + 3
    q = rng.standard_normal((seqs, QH * HD)).astype(np.float32)
    out = run_dev(omega, pool, q, tabs, lens, 0).reshape(seqs, QH * HD)
    for b in (0, 5, 31):
        e = rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], lens[b], 0))
        assert e <= TOL, (b, e)


@pytest.mark.parametrize("mutant", [2, 4])
def test_paged_mutants_are_caught(omega, oracle, mutant):
    rng = np.random.default_rng(33)
    nb = 256
    pool = Pool(omega, oracle, rng, nb, 1)
    lens = np.array([700, 1500], np.int32)
    tabs = np.stack([rng.permutation(nb)[:(1500 + 15) // 16] for _ in range(2)]).astype(np.int32)
    q = (3.0 * rng.standard_normal((2, QH * HD))).astype(np.float32)
    lib = omega.lib()
    lib.omega_gpu_decode_attn_test_set_mutant(mutant)
    try:
        out = run_dev(omega, pool, q, tabs, lens, 0).reshape(2, QH * HD)
    finally:
        lib.omega_gpu_decode_attn_test_set_mutant(0)
    errs = [rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], lens[b], 0)) for b in range(2)]
    assert max(errs) > TOL, errs
    clean = run_dev(omega, pool, q, tabs, lens, 0).reshape(2, QH * HD)
    assert max(rel_err(clean[b], oracle_out(oracle, pool, q[b], tabs[b], lens[b], 0)) for b in range(2)) <= TOL


# ---------------------------------------------------------------- the folded form
# Where a call's split workgroups all fit the device at once (split count a multiple of 16, at
# most 1024 (sequence, split) pairs), the splits are merged in the same launch; the configuration-3
# shapes above run that way. The two forms merge in different orders and agree to f32 rounding.
def run_forms(omega, pool, q, tabs, lens, layer):
    lib = omega.lib()
    try:
        lib.omega_gpu_paged_attention_set_folded(0)
        split = run_dev(omega, pool, q, tabs, lens, layer)
    finally:
        lib.omega_gpu_paged_attention_set_folded(1)
    return run_dev(omega, pool, q, tabs, lens, layer), split


@pytest.mark.parametrize("case", ["1x2048", "1x8192", "ragged8", "32x2048"])
def test_folded_and_split_forms_agree(omega, oracle, case):
    rng = np.random.default_rng(71)
    nb = 1024
    pool = Pool(omega, oracle, rng, nb, 1)
    if case == "ragged8":  # 64 splits planned; a sequence of 1 page keeps one split and merges 32 heads
        lens = np.array([1, 16, 100, 513, 700, 2047, 3000, 4096], np.int32)
    else:
        seqs, ctx = map(int, case.split("x"))
        lens = np.full(seqs, ctx, np.int32)
    maxb = int((lens.max() + 15) // 16)
    tabs = np.stack([rng.permutation(nb)[:maxb] for _ in range(lens.size)]).astype(np.int32)
    q = rng.standard_normal((lens.size, QH * HD)).astype(np.float32)
    folded, split = (o.reshape(lens.size, QH * HD) for o in run_forms(omega, pool, q, tabs, lens, 0))
    assert np.isfinite(folded).all()
    assert rel_err(folded, split) <= 1e-5
    for b in range(lens.size):
        assert rel_err(folded[b], oracle_out(oracle, pool, q[b], tabs[b], lens[b], 0)) <= TOL, b


@pytest.mark.parametrize("mutant", [2, 4])
def test_folded_mutants_are_caught(omega, oracle, mutant):
    # 2 sequences of 2048: 64 splits each, folded
    rng = np.random.default_rng(72)
    nb = 512
    pool = Pool(omega, oracle, rng, nb, 1)
    lens = np.array([2048, 1900], np.int32)
    tabs = np.stack([rng.permutation(nb)[:128] for _ in range(2)]).astype(np.int32)
    q = (3.0 * rng.standard_normal((2, QH * HD))).astype(np.float32)
    lib = omega.lib()
    lib.omega_gpu_decode_attn_test_set_mutant(mutant)
    try:
        out = run_dev(omega, pool, q, tabs, lens, 0).reshape(2, QH * HD)
    finally:
        lib.omega_gpu_decode_attn_test_set_mutant(0)
    errs = [rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], lens[b], 0)) for b in range(2)]
    assert max(errs) > TOL, errs


def test_folded_merge_wait_that_runs_out(omega, oracle):
    # test mutant 9: every in-launch merge gives up at once (no poll). The host-buffer entry
    # reports CHIP_FAIL with its message; the device-pointer entry (it returns before the work
    # ends) writes the merged heads as NaN; the next calls match the oracle.
    rng = np.random.default_rng(73)
    nb = 512
    pool = Pool(omega, oracle, rng, nb, 1)
    lens = np.array([2048], np.int32)
    tabs = rng.permutation(nb)[:128].astype(np.int32).reshape(1, 128)
    q = rng.standard_normal((1, QH * HD)).astype(np.float32)
    lib = omega.lib()
    out = np.zeros(QH * HD, np.float32)
    info = omega.AttnInfo()

    def host_call():
        return lib.omega_gpu_paged_attention_batch_bf16(omega.ptr(q), omega.ptr(pool.host), C.byref(pool.L),
                                                        omega.ptr(tabs), omega.ptr(lens), 128, 1, 0, QH, KVH,
                                                        HD, omega.ptr(out), C.byref(info))

    lib.omega_gpu_decode_attn_test_set_mutant(9)
    try:
        assert host_call() == -4
        assert "ran out of waits" in omega._s(lib.omega_gpu_attention_last_error())
        assert np.isnan(run_dev(omega, pool, q, tabs, lens, 0)).all()
    finally:
        lib.omega_gpu_decode_attn_test_set_mutant(0)
    want = oracle_out(oracle, pool, q[0], tabs[0], 2048, 0)
    assert host_call() == 0
    assert rel_err(out, want) <= TOL
    assert rel_err(run_dev(omega, pool, q, tabs, lens, 0), want) <= TOL


# ---------------------------------------------------------------- the serving step's balanced items
def run_items(omega, pool, q, tabs, lens, layer):
    """omega_gpu_paged_attention_items_dev: sequence b attends over positions 0..lens[b]-1."""
    lib = omega.lib()
    seqs, maxb = tabs.shape
    qd = omega.DeviceBuffer.from_array(q)
    td = omega.DeviceBuffer.from_array(tabs.astype(np.int32))
    od = omega.DeviceBuffer(q.nbytes)
    pos = np.ascontiguousarray(lens - 1, dtype=np.uint32)
    rc = lib.omega_gpu_paged_attention_items_dev(qd.ptr, pool.dev.ptr, C.byref(pool.L), td.ptr, maxb,
                                                 pos.ctypes.data, seqs, layer, od.ptr)
    if rc != 0:
        raise omega.OmegaGpuError(rc, omega._s(lib.omega_gpu_attention_last_error()))
    out = od.download(np.float32, q.size)
    for b in (qd, td, od):
        b.free()
    return out


@pytest.mark.parametrize("case", ["mixed", "one_long", "many_short", "config5_like"])
def test_balanced_items_match_the_oracle(omega, oracle, case):
    # The pages of all sequences are cut into 512 equal runs per kv head: a run may cover several
    # short sequences, a long sequence spans many runs, and a run may start or end inside a page
    # range of any sequence. Contexts ending inside a page have NaN / inf in the unwritten slots.
    rng = np.random.default_rng({"mixed": 41, "one_long": 42, "many_short": 43, "config5_like": 44}[case])
    if case == "mixed":
        lens = np.array([1, 5, 17, 333, 1000, 2047, 4099, 9001, 16000], np.int32)
    elif case == "one_long":
        lens = np.array([32768 - 5], np.int32)
    elif case == "many_short":
        lens = rng.integers(1, 40, 32).astype(np.int32)
    else:
        lens = np.exp(rng.uniform(np.log(1024), np.log(12288), 32)).astype(np.int32)
    pages = (lens + 15) // 16
    nb = max(4096, int(pages.sum()) + 1)
    pool = Pool(omega, oracle, rng, nb, 2)
    maxb = int(pages.max()) + 2
    tabs = np.full((lens.size, maxb), -1, np.int32)
    free = rng.permutation(nb)  # disjoint pages: a poisoned tail belongs to its sequence only
    used = 0
    for b, n_b in enumerate(pages):
        tabs[b, :n_b] = free[used:used + n_b]
        used += n_b
    for b, cl in enumerate(lens):
        if cl % 16:
            pool.poison_tail(oracle, tabs[b], int(cl), 1)
    q = rng.standard_normal((lens.size, QH * HD)).astype(np.float32)
    out = run_items(omega, pool, q, tabs, lens, 1).reshape(lens.size, QH * HD)
    assert np.isfinite(out).all()
    check = range(lens.size) if lens.size <= 9 else (0, 7, 19, 31)
    for b in check:
        e = rel_err(out[b], oracle_out(oracle, pool, q[b], tabs[b], int(lens[b]), 1))
        assert e <= TOL, (case, b, int(lens[b]), e)
    # deterministic: the same call gives the same bits
    np.testing.assert_array_equal(run_items(omega, pool, q, tabs, lens, 1).reshape(lens.size, QH * HD), out)
    pool.dev.free()


def test_balanced_items_refusals(omega, oracle):
    rng = np.random.default_rng(45)
    pool = Pool(omega, oracle, rng, 64, 1)
    q = rng.standard_normal((2, QH * HD)).astype(np.float32)
    tabs = rng.permutation(64)[:8].reshape(2, 4).astype(np.int32)
    with pytest.raises(omega.OmegaGpuError):
        run_items(omega, pool, q, tabs, np.array([65, 3], np.int32), 0)   # position 64 past 4 pages
    with pytest.raises(omega.OmegaGpuError):
        run_items(omega, pool, q, tabs, np.array([3, 3], np.int32), 1)    # layer outside the pool
    q33 = rng.standard_normal((33, QH * HD)).astype(np.float32)
    with pytest.raises(omega.OmegaGpuError):
        run_items(omega, pool, q33, np.zeros((33, 4), np.int32), np.full(33, 3, np.int32), 0)
    out = run_items(omega, pool, q, tabs, np.array([64, 1], np.int32), 0)  # the whole table
    assert np.isfinite(out).all()
    pool.dev.free()


@pytest.mark.parametrize("qh,kvh", [(64, 8), (16, 2), (32, 8)])
def test_other_gqa_geometries(omega, oracle, qh, kvh):
    # GQA group 8 with a kv head count other than four takes the one-head-per-wavefront
    # matrix-core kernel; other groups the VALU kernel
    rng = np.random.default_rng(50 + qh + kvh)
    nb = 256
    lay = oracle.kv_layout(nb, 16, 2, kvh, HD)
    host = oracle.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    L = _omega_layout(omega, lay)
    dev = omega.DeviceBuffer.from_array(host)
    lens = np.array([1, 300, 1777], np.int32)
    maxb = (int(lens.max()) + 15) // 16
    tabs = np.stack([rng.permutation(nb)[:maxb] for _ in lens]).astype(np.int32)
    q = rng.standard_normal((lens.size, qh * HD)).astype(np.float32)
    lib = omega.lib()
    qd, td, ld = (omega.DeviceBuffer.from_array(x) for x in (q, tabs, lens))
    od = omega.DeviceBuffer(q.nbytes)
    rc = lib.omega_gpu_paged_attention_batch_dev(qd.ptr, dev.ptr, C.byref(L), td.ptr, ld.ptr, maxb, lens.size,
                                                 int(lens.max()), 1, qh, kvh, HD, od.ptr)
    assert rc == 0, omega._s(lib.omega_gpu_attention_last_error())
    out = od.download(np.float32, q.size).reshape(lens.size, qh * HD)
    for b, cl in enumerate(lens):
        want = np.zeros(qh * HD, np.float32)
        oracle.lib().oref_paged_attention(oracle.ptr(np.ascontiguousarray(q[b])), oracle.ptr(host), C.byref(lay),
                                          oracle.ptr(tabs[b]), int(cl), 1, qh, kvh, HD, oracle.ptr(want))
        e = rel_err(out[b], want)
        assert e <= TOL, (qh, kvh, b, int(cl), e)
    for x in (qd, td, ld, od, dev):
        x.free()
