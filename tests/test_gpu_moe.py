"""GPU parity of the batched MoE block (configuration 2: Qwen3-30B-A3B MoE at token batch 1 and
32) against the CPU oracle: per token the reference route (RMSNorm, f64-refined router logits,
top-8 by total order, renormalised weights) and the engine's FP8 MoE arm (gate|up grouped GEMV,
SwiGLU, down grouped GEMV, slot-order combine).

Bars: expert ids bit-exact, weights within 1e-6 relative, moe_out within 2e-3 relative
(max abs error over max abs value, per token). From 16 tokens on the GEMMs run on the FP8 matrix
cores with the activations split into four e4m3 terms; the one-term mutant (a plain fp8 cast of
the activations) must fail the 2e-3 bar, which shows the bar resolves the split's precision.
Below 16 tokens the projections are grouped GEMVs on the f32 rows, held to 1e-4; one token runs
the decode step's own three launches (router logits, gate|up with the top-8 ranking in its
prologue, down with the slot-order combine), also GEMVs on the f32 rows under the same bar.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3
GEMV_TOL = 1e-4
GEMV_MAX = 16  # token batches below this take the GEMV path
SEED = 20261202
E, H, I = 128, 2048, 768


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


@pytest.fixture(scope="module")
def model(omega, oracle):
    rng = np.random.default_rng(5)
    gu_w, gu_s = oracle.synth_fp8(SEED, 2, E, 2 * I, H)
    dn_w, dn_s = oracle.synth_fp8(SEED, 3, E, H, I)
    gu = omega.Fp8Tensor.synth(E, 2 * I, H, SEED, 2)
    dn = omega.Fp8Tensor.synth(E, H, I, SEED, 3)
    gate = oracle.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    norm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    r = omega.Router(1)
    r.set_layer(0, gate, norm)
    r.set_directory(0, np.zeros(2 * E, np.uint64), np.zeros(2 * E, np.uint64))
    m = dict(gu_w=gu_w, gu_s=gu_s, dn_w=dn_w, dn_s=dn_s, gu=gu, dn=dn, gate=gate, norm=norm, router=r)
    yield m
    r.free()
    gu.free()
    dn.free()


def oracle_block(oracle, m, h, eps=1e-6):
    outs, ids, ws = [], [], []
    for t in range(h.shape[0]):
        i, w, post, _ = oracle.route(m["gate"], m["norm"], h[t], eps, refined=True)
        outs.append(oracle.moe_block(m["gu_w"], m["gu_s"], m["dn_w"], m["dn_s"], i, w, post))
        ids.append(i)
        ws.append(w)
    return np.stack(outs), np.stack(ids), np.stack(ws)


def bf16_rows(oracle, rng, T):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32)))


@pytest.mark.parametrize("T", [1, 3, 4, 5, 15, 16, 17, 32, 64])
def test_moe_block_matches_the_oracle(omega, oracle, model, T):
    h = bf16_rows(oracle, np.random.default_rng(100 + T), T)
    out, ids, w = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    want, want_ids, want_w = oracle_block(oracle, model, h)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_allclose(w, want_w, rtol=1e-6, atol=0)
    errs = [rel_err(out[t], want[t]) for t in range(T)]
    # below 16 tokens the projections are GEMVs on the f32 rows: only the f32 summation order
    # separates them from the oracle
    bar = GEMV_TOL if T < GEMV_MAX else TOL
    print(f"T={T}: worst moe_out rel err {max(errs):.2e} (bar {bar:.0e})")
    assert max(errs) <= bar, (max(errs), int(np.argmax(errs)))
    # deterministic: the same call again gives the same bits
    out2, ids2, _ = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    np.testing.assert_array_equal(out2, out)
    np.testing.assert_array_equal(ids2, ids)


def test_crowded_experts_use_several_row_tiles(omega, oracle, model):
    # 64 near-identical tokens route to the same experts: segments of up to 64 rows (4 MFMA
    # column tiles of 16)
    rng = np.random.default_rng(7)
    base = rng.standard_normal(H).astype(np.float32)
    h = bf16_rows(oracle, rng, 64) * 0.02 + base
    h = oracle.bf16_to_f32(oracle.f32_to_bf16(h.astype(np.float32)))
    out, ids, _ = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    want, want_ids, _ = oracle_block(oracle, model, h)
    np.testing.assert_array_equal(ids, want_ids)
    assert np.bincount(ids.reshape(-1), minlength=E).max() > 48
    assert max(rel_err(out[t], want[t]) for t in range(64)) <= TOL


@pytest.mark.parametrize("T", [1, 32])
def test_device_entry_adds_the_residual(omega, oracle, model, T):
    h = bf16_rows(oracle, np.random.default_rng(9), T)
    out, ids, w = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    lib = omega.lib()
    hd = omega.DeviceBuffer.from_array(h)
    od = omega.DeviceBuffer(h.nbytes)
    idd = omega.DeviceBuffer(T * 8 * 4)
    wd = omega.DeviceBuffer(T * 8 * 4)
    rc = lib.omega_gpu_moe_batch_dev(model["router"].as_raw(), 0, model["gu"].as_raw(),
                                     model["dn"].as_raw(), T, hd.ptr, 1e-6, 1, hd.ptr, idd.ptr,
                                     wd.ptr, od.ptr)
    assert rc == 0
    got = od.download(np.float32, T * H).reshape(T, H)
    np.testing.assert_array_equal(idd.download(np.uint32, T * 8).reshape(T, 8), ids)
    # the same moe rows, then one f32 add of the residual
    np.testing.assert_array_equal(got, (h + out).astype(np.float32))
    # without the residual the device entry writes the moe rows alone
    rc = lib.omega_gpu_moe_batch_dev(model["router"].as_raw(), 0, model["gu"].as_raw(),
                                     model["dn"].as_raw(), T, hd.ptr, 1e-6, 1, None, idd.ptr,
                                     wd.ptr, od.ptr)
    assert rc == 0
    np.testing.assert_array_equal(od.download(np.float32, T * H).reshape(T, H), out)
    np.testing.assert_array_equal(wd.download(np.float32, T * 8).reshape(T, 8), w)


@pytest.mark.parametrize("T,mutant", [(32, 1), (32, 2), (32, 5), (32, 6), (32, 7),
                                       (8, 1), (8, 2), (8, 5), (8, 6), (3, 1), (3, 2)])
def test_moe_mutants_are_caught(omega, oracle, model, T, mutant):
    h = bf16_rows(oracle, np.random.default_rng(11), T)
    want, want_ids, want_w = oracle_block(oracle, model, h)
    lib = omega.lib()
    lib.omega_gpu_moe_test_set_mutant(mutant)
    try:
        out, ids, w = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    finally:
        lib.omega_gpu_moe_test_set_mutant(0)
    caught = (not np.array_equal(ids, want_ids) or
              not np.allclose(w, want_w, rtol=1e-6, atol=0) or
              max(rel_err(out[t], want[t]) for t in range(T)) > TOL)
    assert caught


@pytest.mark.parametrize("T", [8, 32])
def test_a_planner_wait_that_runs_out_is_reported_and_the_next_call_recovers(omega, oracle, model, T):
    # test mutant 9: the grouping planner's bounded wait gives up at once (no poll), as when the
    # rankings never arrive. The f32 entry reports it; the device entry cannot (it returns before
    # the work ends) and adds no expert rows: out = resid. The next calls take fresh epochs.
    h = bf16_rows(oracle, np.random.default_rng(13), T)
    good, good_ids, good_w = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    lib = omega.lib()
    hd = omega.DeviceBuffer.from_array(h)
    od = omega.DeviceBuffer(h.nbytes)
    idd = omega.DeviceBuffer(T * 8 * 4)
    wd = omega.DeviceBuffer(T * 8 * 4)
    lib.omega_gpu_moe_test_set_mutant(9)
    try:
        with pytest.raises(omega.OmegaGpuError, match="timed out"):
            omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
        rc = lib.omega_gpu_moe_batch_dev(model["router"].as_raw(), 0, model["gu"].as_raw(),
                                         model["dn"].as_raw(), T, hd.ptr, 1e-6, 1, hd.ptr, idd.ptr,
                                         wd.ptr, od.ptr)
        assert rc == 0
        np.testing.assert_array_equal(od.download(np.float32, T * H).reshape(T, H), h)
        np.testing.assert_array_equal(idd.download(np.uint32, T * 8).reshape(T, 8), good_ids)
    finally:
        lib.omega_gpu_moe_test_set_mutant(0)
    for _ in range(2):
        out, ids, w = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
        np.testing.assert_array_equal(ids, good_ids)
        np.testing.assert_array_equal(w.view(np.uint32), good_w.view(np.uint32))
        np.testing.assert_array_equal(out.view(np.uint32), good.view(np.uint32))


def test_allocations_are_counted_and_a_sealed_call_builds_no_twin(omega, oracle, model):
    # every allocation the library makes is counted (omega_gpu_session_alloc_stats, "driver
    # allocation counters since the process started", aien-omega-gpu/src/lib.rs:1165-1178); while
    # the serving reservation is sealed, a call that would build a tensor's tiled twin (its first
    # batched use) is refused with TOO_LARGE and counted as a stale refusal; release lifts it
    h = bf16_rows(oracle, np.random.default_rng(17), 32)
    want, want_ids, _ = omega.moe_batch(model["router"], 0, model["gu"], model["dn"], h, 1e-6)
    s0 = omega.alloc_stats()  # the scratch and staging of 32 rows exist now
    gu = omega.Fp8Tensor.synth(E, 2 * I, H, SEED, 2)
    dn = omega.Fp8Tensor.synth(E, H, I, SEED, 3)
    s1 = omega.alloc_stats()
    gu_bytes = E * 2 * I * H + E * (2 * I // 128) * (H // 128) * 4
    dn_bytes = E * H * I + E * (H // 128) * (I // 128) * 4
    assert s1["allocs"] == s0["allocs"] + 4                      # weights and scales of each
    assert s1["alloc_bytes"] == s0["alloc_bytes"] + gu_bytes + dn_bytes
    try:
        omega.serving_seal()
        with pytest.raises(omega.OmegaGpuError, match="reservation exceeded"):
            omega.moe_batch(model["router"], 0, gu, dn, h, 1e-6)
        assert omega.alloc_stats()["stale_refusals"] == s1["stale_refusals"] + 1
        assert omega.alloc_stats()["allocs"] == s1["allocs"]
    finally:
        omega.serving_release()
    out, ids, _ = omega.moe_batch(model["router"], 0, gu, dn, h, 1e-6)  # the same seeded tensors
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))
    s2 = omega.alloc_stats()
    assert s2["allocs"] == s1["allocs"] + 2                      # the two tiled twins
    assert s2["alloc_bytes"] == s1["alloc_bytes"] + E * 2 * I * H + E * H * I
    gu.free()
    dn.free()
    assert omega.alloc_stats()["frees"] == s2["frees"] + 6       # weights, scales and twin of each
