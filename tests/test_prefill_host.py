"""Host-side pieces of the whole-prompt prefill boundary (no GPU): the C tile builder against the
host mirror of build_tiles (aien-omega-pf/src/lib.rs:122-160), the C router packer against the
packed layout (lib.rs:460-478), the routing plan of the driver against the oracle's
MoeBatchPlan::from_logits, the host RMSNorm against the oracle's, and the struct layouts."""
import ctypes as C
import os

import numpy as np
import pytest


@pytest.fixture(scope="module")
def pf():
    from omega_amd import prefill

    return prefill


def test_tile_builder_matches_the_host_mirror(pf):
    rng = np.random.default_rng(1)
    for counts in ([5], [64], [65], [0, 0, 3], [130, 0, 1, 64, 200], list(rng.integers(0, 40, 128))):
        e = len(counts)
        w = (np.arange(e, dtype=np.uint64) + 1) * 0x100000
        s = (np.arange(e, dtype=np.uint64) + 1) * 0x1000 + 7
        want = pf.build_tiles(pf.qgemm_bm(), w, s, counts)
        got = pf.tiles_va_c(w, s, counts)
        np.testing.assert_array_equal(got, want)
        assert int(want["cnt"].sum()) == sum(counts)
    # a table that would overflow its room is refused (0 tiles)
    w = np.ones(1, np.uint64)
    tab = np.zeros(2, pf.TILE_DTYPE)
    n = pf.lib().omega_gpu_pf_qgemm_tiles_va(1, w.ctypes.data, w.ctypes.data,
                                             np.array([200], np.uint32).ctypes.data, tab.ctypes.data, 2)
    assert n == 0


def test_router_tile_is_the_reference_engines(pf):
    # the reference's own test of the linked library expects 16 rows per router tile
    # (aien-omega-pf/src/lib.rs:1300); buffers hold whole tiles
    assert pf.router_rows() == 16


def test_router_pack_layout(pf):
    rng = np.random.default_rng(2)
    e, k = 6, 16
    w = rng.standard_normal((e, k)).astype(np.float32)
    wq = pf.pack_router(w)
    assert wq.size == pf.router_packed_len(e, k)
    for g in range(k // 4):
        for ex in range(e):
            np.testing.assert_array_equal(wq[(g * e + ex) * 4:(g * e + ex) * 4 + 4], w[ex, 4 * g:4 * g + 4])
    assert (wq[(k // 4) * e * 4:] == 0).all()


def total_order_topk(lg, k):
    """numpy restatement: stable descending sort of the f32 total-order keys (ties: lower id)"""
    b = lg.view(np.int32).astype(np.int64)
    key = np.where(b < 0, b ^ 0x7FFFFFFF, b)
    return np.argsort(-key, axis=1, kind="stable")[:, :k]


@pytest.mark.parametrize("T,E,K", [(37, 128, 8), (2048, 128, 8), (19, 60, 4), (3, 8, 8)])
def test_routing_plan_matches_the_oracle(pf, oracle, T, E, K):
    rng = np.random.default_rng(3 + T)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[1, 2] = logits[1, E - 1] = logits[1].max() + 1.0   # a tie at the top: lower id first
    logits[2, :] = 0.5                                          # all equal
    logits[0, 3] = -0.0
    logits[0, 4] = 0.0                                          # total order: +0.0 above -0.0
    ids, wts, counts, gtok, a2g = pf.moe_plan(logits.reshape(-1), T, E, K)
    ref = oracle.moe_plan(logits.reshape(-1), T, E, K)
    np.testing.assert_array_equal(ids, total_order_topk(logits, K))
    np.testing.assert_array_equal(ids.reshape(-1), ref["topk_experts"])
    np.testing.assert_array_equal(wts.reshape(-1).view(np.uint32), ref["topk_weights"].view(np.uint32))
    np.testing.assert_array_equal(counts, np.diff(ref["expert_offsets"]))
    np.testing.assert_array_equal(gtok, ref["grouped_token_ids"])
    np.testing.assert_array_equal(a2g, ref["assignment_to_grouped"])
    # the grouping is the stable sort of the assignments by expert
    np.testing.assert_array_equal(np.argsort(np.argsort(ids.reshape(-1), kind="stable"), kind="stable"), a2g)


def test_routing_plan_refusals(pf):
    from omega_amd import OmegaGpuError

    bad = np.zeros((4, 16), np.float32)
    bad[2, 5] = np.nan
    with pytest.raises(OmegaGpuError, match="token 2, expert 5"):
        pf.moe_plan(bad, 4, 16, 4)
    with pytest.raises(OmegaGpuError):
        pf.moe_plan(np.zeros((4, 16), np.float32), 4, 16, 17)   # top_k > experts
    # a long prompt is ranked over several host threads: the first bad logit in row order is named
    bad = np.random.default_rng(5).standard_normal((1500, 128)).astype(np.float32)
    bad[1400, 9] = np.inf
    bad[700, 100] = np.nan
    bad[700, 101] = -np.inf
    with pytest.raises(OmegaGpuError, match="token 700, expert 100"):
        pf.moe_plan(bad, 1500, 128, 8)
    bad[700, 100:102] = 0.0
    with pytest.raises(OmegaGpuError, match="token 1400, expert 9"):
        pf.moe_plan(bad, 1500, 128, 8)
    bad[1400, 9] = 0.0
    ref = pf.moe_plan(bad, 1500, 128, 8)
    for _ in range(3):   # the split over threads does not change the result
        for got, want in zip(pf.moe_plan(bad, 1500, 128, 8), ref):
            np.testing.assert_array_equal(got, want)


@pytest.mark.skipif(not hasattr(os, "fork") or os.path.exists("/dev/kfd"),
                    reason="forks the test process: only where no GPU runtime can be live in it")
def test_routing_plan_in_a_forked_child(pf):
    """The plan's host threads do not follow a fork: a child ranks a long prompt alone, with the
    parent's results."""
    lg = np.random.default_rng(6).standard_normal((1024, 128)).astype(np.float32)
    ref = pf.moe_plan(lg, 1024, 128, 8)  # starts the host threads in this process
    pid = os.fork()
    if pid == 0:
        ok = all(np.array_equal(a, b) for a, b in zip(pf.moe_plan(lg, 1024, 128, 8), ref))
        os._exit(0 if ok else 1)
    _, status = os.waitpid(pid, 0)
    assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0
    for a, b in zip(pf.moe_plan(lg, 1024, 128, 8), ref):  # and the parent's threads still serve
        np.testing.assert_array_equal(a, b)


def test_host_rmsnorm_matches_the_oracle(pf, oracle):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((5, 2048)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    got = pf.rmsnorm_rows(x, w, 1e-6)
    for r in range(5):
        np.testing.assert_array_equal(got[r], oracle.rmsnorm(x[r], w, 1e-6))


def test_struct_layouts(pf):
    assert C.sizeof(pf.OmegaGpuMem) == 40
    assert pf.OmegaGpuMem.va.offset == 24
    assert C.sizeof(pf.PrefillAttnInfo) == 64
    assert pf.PrefillAttnInfo.elapsed_ns.offset == 40
    assert pf.PrefillAttnInfo.kernel_cache_hit.offset == 56
    assert pf.TILE_DTYPE.itemsize == pf.TILE_BYTES
