"""GPU parity of the FP8 block-scaled GEMV family against the CPU oracle (HostFp8 order).

Bar: max |y - y_ref| <= 2e-3 * max |y_ref| (f32 accumulation; the observed error is ~1e-6).
Reference: crates/aien-omega-fp8/src/lib.rs (ABI), inference-abi/qwen3_moe_omega.rs:2114-2139
(HostFp8::grouped_f32, the oracle).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def bf16_row(rng, k, oracle):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(k).astype(np.float32)))


def test_native_ocp_e4m3_decode_and_byte_order(omega, oracle):
    # every finite code at every byte position of a 16-byte chunk: W[r][c] = code(r), x one-hot
    n, k = 256, 128
    codes = np.array([r if (r & 0x7F) != 0x7F else 0 for r in range(n)], np.uint8)
    table = oracle.e4m3_table()
    s = np.full((1, n // 128, 1), 0x3F80, np.uint16)     # scale 1.0
    for c in range(16):
        w = np.zeros((1, n, k), np.uint8)
        w[0, :, c] = codes
        t = omega.Fp8Tensor.upload(1, n, k, w, s)
        x = np.zeros(k, np.float32)
        x[c] = 1.0
        y, _ = t.gemv_f32(0, x)
        np.testing.assert_array_equal(y, table[codes])
        t.free()


@pytest.mark.parametrize("experts,n,k", [(1, 5120, 2048), (1, 2048, 4096), (3, 256, 768),
                                         (1, 128, 128), (2, 384, 384), (1, 128, 32768)])
def test_gemv_matches_the_oracle(omega, oracle, experts, n, k):
    w, s = oracle.synth_fp8(11, n * 7 + k, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(n + k)
    for e in range(experts):
        x = bf16_row(rng, k, oracle)
        y, info = t.gemv_f32(e, x)
        ref = oracle.fp8_grouped(w, s, [e], x, threads=8)[0]
        assert rel_err(y, ref) <= TOL, (e, rel_err(y, ref))
        assert info.weight_bytes == n * k and info.sm_architecture == 950
    t.free()


def test_grouped_shared_and_per_group_rows(omega, oracle):
    experts, n, k = 16, 1536, 2048
    w, s = oracle.synth_fp8(12, 5, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(0)
    ids = np.array([3, 15, 0, 3, 7, 9, 1, 12], np.uint32)
    x1 = rng.standard_normal(k).astype(np.float32)
    y1, _ = t.gemv_grouped_f32(ids, x1)
    assert rel_err(y1, oracle.fp8_grouped(w, s, ids, x1, threads=8)) <= TOL
    xg = rng.standard_normal((8, k)).astype(np.float32)
    yg, _ = t.gemv_grouped_f32(ids, xg)
    assert rel_err(yg, oracle.fp8_grouped(w, s, ids, xg, threads=8)) <= TOL
    # 64 groups, the most one launch takes
    ids64 = rng.integers(0, experts, 64).astype(np.uint32)
    y64, info = t.gemv_grouped_f32(ids64, x1)
    assert rel_err(y64, oracle.fp8_grouped(w, s, ids64, x1, threads=8)) <= TOL
    assert info.groups == 64
    t.free()


def test_deterministic_across_calls(omega, oracle):
    w, s = oracle.synth_fp8(13, 1, 1, 5120, 2048)
    t = omega.Fp8Tensor.upload(1, 5120, 2048, w, s)
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    a, _ = t.gemv_f32(0, x)
    for _ in range(3):
        b, _ = t.gemv_f32(0, x)
        np.testing.assert_array_equal(a, b)
    t.free()


def test_device_generator_equals_the_host_generator(omega, oracle):
    # the benchmark's device-side weights are bit-identical to the CPU generator's
    experts, n, k = 2, 768, 2048
    w, s = oracle.synth_fp8(77, 1234, experts, n, k, 0.02)
    th = omega.Fp8Tensor.upload(experts, n, k, w, s)
    td = omega.Fp8Tensor.synth(experts, n, k, 77, 1234, 0.02)
    x = np.random.default_rng(2).standard_normal(k).astype(np.float32)
    for e in range(experts):
        np.testing.assert_array_equal(th.gemv_f32(e, x)[0], td.gemv_f32(e, x)[0])
    th.free()
    td.free()


@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_kernel_mutants_are_caught(omega, oracle, mutant):
    # crates/aien-omega-fp8/src/lib.rs:729-750: each deliberately wrong kernel must fail parity
    experts, n, k = 4, 1536, 2048
    w, s = oracle.synth_fp8(14, 2, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32)
    ids = np.array([1, 2], np.uint32)
    ref = oracle.fp8_grouped(w, s, ids, x, threads=8)
    omega.lib().omega_gpu_fp8_test_set_mutant(mutant)
    try:
        y, _ = t.gemv_grouped_f32(ids, x)
    finally:
        omega.lib().omega_gpu_fp8_test_set_mutant(0)
    assert rel_err(y, ref) > 0.05
    y, _ = t.gemv_grouped_f32(ids, x)
    assert rel_err(y, ref) <= TOL
    t.free()


def test_no_fold_upload_mutant_is_caught(omega, oracle):
    w, s = oracle.synth_fp8(15, 3, 1, 256, 256)
    x = np.random.default_rng(4).standard_normal(256).astype(np.float32)
    ref = oracle.fp8_grouped(w, s, [0], x)[0]
    omega.lib().omega_gpu_fp8_test_set_no_fold(1)
    try:
        t = omega.Fp8Tensor.upload(1, 256, 256, w, s)
    finally:
        omega.lib().omega_gpu_fp8_test_set_no_fold(0)
    assert rel_err(t.gemv_f32(0, x)[0], ref) > 0.5
    t.free()


def test_nan_weights_and_bad_shapes_are_refused(omega):
    w = np.zeros((1, 128, 128), np.uint8)
    s = np.full((1, 1, 1), 0x3F80, np.uint16)
    w[0, 5, 77] = 0xFF
    with pytest.raises(omega.OmegaGpuError) as e:
        omega.Fp8Tensor.upload(1, 128, 128, w, s)
    assert "NAN_WEIGHT" in str(e.value)
    w[0, 5, 77] = 0x7F
    with pytest.raises(omega.OmegaGpuError):
        omega.Fp8Tensor.upload(1, 128, 128, w, s)
    import ctypes as C
    h = C.c_void_p()
    assert omega.lib().omega_gpu_fp8_tensor_upload(1, 100, 128, omega.ptr(w), omega.ptr(s),
                                                   C.byref(h)) == -1
    assert not h.value


def test_grouped_dev_reads_the_router_table(omega, oracle):
    # the router writes x' * 2^64 and the group table; the GEMV reads both on the device
    E, H = 128, 2048
    gu_w, gu_s = oracle.synth_fp8(16, 1, E, 1536, H)
    dn_w, dn_s = oracle.synth_fp8(16, 2, E, 2048, 768)
    gu = omega.Fp8Tensor.upload(E, 1536, H, gu_w, gu_s)
    dn = omega.Fp8Tensor.upload(E, 2048, 768, dn_w, dn_s)
    r = omega.Router(1)
    rng = np.random.default_rng(5)
    gate = oracle.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    norm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    r.set_layer(0, gate, norm)
    r.set_directory(0, np.array([gu.entry(e) for e in range(E)], np.uint64),
                    np.array([dn.entry(e) for e in range(E)], np.uint64))
    x = rng.standard_normal(H).astype(np.float32)
    ids, wts, _ = r.route(0, x, 1e-6)
    xout_va, tab_gu, tab_dn = r.device_outputs()
    y, _ = gu.gemv_grouped_dev(8, tab_gu, xout_va)
    want_ids, _, post, _ = oracle.route(gate, norm, x, 1e-6)
    np.testing.assert_array_equal(ids, want_ids)
    ref = oracle.fp8_grouped(gu_w, gu_s, want_ids, post, threads=8)
    assert rel_err(y, ref) <= TOL
    r.free()
    gu.free()
    dn.free()


def test_gemm_is_bit_identical_to_the_gemv_per_row(omega, oracle):
    experts, n, k = 8, 1536, 2048
    w, s = oracle.synth_fp8(17, 4, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, k)).astype(np.float32)
    eids = np.sort(rng.integers(0, experts, 70)).astype(np.uint32)
    rows = rng.integers(0, 5, 70).astype(np.uint32)
    y, info = t.gemm_f32(eids, rows, x)
    for i in range(70):
        yi, _ = t.gemv_f32(int(eids[i]), x[rows[i]])
        np.testing.assert_array_equal(y[i], yi)
    assert info.rows == 70 and info.segments == len(set(eids.tolist()))
    with pytest.raises(omega.OmegaGpuError):
        t.gemm_f32(eids[::-1].copy(), rows, x)     # unsorted
    t.free()


def config2_rows(rng, tokens, experts):
    """The row table of a batched MoE step: each token's 8 distinct experts, sorted by expert
    (stable: rows of one expert keep token order)."""
    eids = np.concatenate([rng.choice(experts, 8, replace=False) for _ in range(tokens)]).astype(np.uint32)
    toks = np.repeat(np.arange(tokens, dtype=np.uint32), 8)
    order = np.argsort(eids, kind="stable")
    return eids[order], toks[order]


@pytest.mark.parametrize("n,k", [(1536, 2048), (2048, 768)])
def test_gemm_config2_row_table_against_the_oracle(omega, oracle, n, k):
    # configuration 2 at T = 32: 256 rows over ~112 of the 128 experts (gate|up, then down);
    # one launch that reads each segment's weights once
    experts = 128
    w, s = oracle.synth_fp8(23, n + k, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(n * 3 + k)
    eids, toks = config2_rows(rng, 32, experts)
    x = np.stack([bf16_row(rng, k, oracle) for _ in range(32)])
    y, info = t.gemm_f32(eids, toks, x)
    segs = len(set(eids.tolist()))
    assert 90 <= segs <= 128 and info.segments == segs and info.rows == 256
    assert info.passes_max == 1
    assert info.weight_bytes == segs * n * k and info.streamed_bytes == info.weight_bytes
    ref = oracle.fp8_grouped(w, s, eids, x[toks], threads=8)
    for i in range(256):
        assert rel_err(y[i], ref[i]) <= TOL, (i, int(eids[i]), rel_err(y[i], ref[i]))
    for i in np.random.default_rng(1).choice(256, 12, replace=False):
        yi, _ = t.gemv_f32(int(eids[i]), x[toks[i]])
        np.testing.assert_array_equal(y[i], yi)
    t.free()


def test_gemm_other_width_takes_passes_of_eight_rows(omega, oracle):
    # k = 384 runs the runtime-shaped kernel: segments of 19, 1, 8 and 9 rows take 3, 1, 1 and 2
    # passes over their weights
    experts, n, k = 4, 256, 384
    w, s = oracle.synth_fp8(24, 9, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(9)
    eids = np.repeat(np.arange(4, dtype=np.uint32), [19, 1, 8, 9])
    x = np.stack([bf16_row(rng, k, oracle) for _ in range(6)])
    toks = rng.integers(0, 6, eids.size).astype(np.uint32)
    y, info = t.gemm_f32(eids, toks, x)
    assert info.passes_max == 3 and info.streamed_bytes == 7 * n * k and info.weight_bytes == 4 * n * k
    ref = oracle.fp8_grouped(w, s, eids, x[toks], threads=8)
    for i in range(eids.size):
        assert rel_err(y[i], ref[i]) <= TOL, (i, rel_err(y[i], ref[i]))
        yi, _ = t.gemv_f32(int(eids[i]), x[toks[i]])
        np.testing.assert_array_equal(y[i], yi)
    t.free()


@pytest.mark.parametrize("k", [2048, 384])
@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_gemm_mutants_are_caught(omega, oracle, mutant, k):
    # crates/aien-omega-fp8/src/lib.rs:644-645: 1 scale dropped, 2 scale pointer never advances,
    # 3 neighbour row's x
    experts, n = 3, 256
    w, s = oracle.synth_fp8(25, k, experts, n, k)
    t = omega.Fp8Tensor.upload(experts, n, k, w, s)
    rng = np.random.default_rng(k + mutant)
    eids = np.array([0, 0, 1, 1, 1, 2], np.uint32)
    x = np.stack([bf16_row(rng, k, oracle) for _ in range(6)])
    toks = np.arange(6, dtype=np.uint32)
    ref = oracle.fp8_grouped(w, s, eids, x, threads=8)
    omega.lib().omega_gpu_fp8gemm_test_set_mutant(mutant)
    try:
        y, _ = t.gemm_f32(eids, toks, x)
    finally:
        omega.lib().omega_gpu_fp8gemm_test_set_mutant(0)
    assert rel_err(y, ref) > TOL, mutant
    y, _ = t.gemm_f32(eids, toks, x)
    assert rel_err(y, ref) <= TOL
    t.free()
