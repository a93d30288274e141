"""Pins of the W8A8 activation quantiser (fake_quant.rs) against the reference's golden table.

Reference: crates/aien-inference-abi/src/qwen3_moe_omega_prefill/fake_quant.rs:130-226 and the
golden file pq_golden.txt (tests/golden/pq_golden.txt).
"""
import os
import struct

import numpy as np

from conftest import GOLDEN


def bits_f32(u):
    return struct.unpack("<f", struct.pack("<I", u))[0]


def test_e4m3_edges(oracle):
    # fake_quant.rs:135-166
    L = oracle.lib()
    assert L.oref_e4m3_rne_sat(448.0) == 0x7E
    assert L.oref_e4m3_rne_sat(1000.0) == 0x7E
    assert L.oref_e4m3_rne_sat(-1000.0) == 0xFE
    assert L.oref_e4m3_rne_sat(0.0) == 0x00
    assert L.oref_e4m3_rne_sat(1.0) == 0x38
    assert L.oref_e4m3_rne_sat(2.0 ** -6) == 0x08
    assert L.oref_e4m3_rne_sat(2.0 ** -9) == 0x01
    assert L.oref_e4m3_rne_sat(1.0625) == 0x38
    assert L.oref_e4m3_rne_sat(1.1875) == 0x3A
    for c in range(256):
        if c & 0x7F == 0x7F:
            continue
        want = 0x80 if c == 0x80 else c
        assert L.oref_e4m3_rne_sat(L.oref_fq_e4m3_to_f32(c)) == want, hex(c)


def test_quantiser_encoder_agrees_with_the_model_encoder(oracle):
    # Two restated encoders (qwen3_moe.rs binary search, fake_quant.rs f64 arithmetic) agree on
    # every value that does not saturate above 448 (where both clamp to 0x7e).
    L = oracle.lib()
    rng = np.random.default_rng(11)
    for v in np.concatenate([rng.standard_normal(5000) * 40, rng.standard_normal(2000) * 0.01]):
        v = float(np.float32(v))
        assert L.oref_e4m3_rne_sat(v) == L.oref_f32_to_e4m3(v), v


def test_block_scale_rounds_amax_up_above_1_75(oracle):
    # fake_quant.rs:168-179
    L = oracle.lib()
    import ctypes as C

    def bs(m):
        s, i = C.c_float(), C.c_float()
        L.oref_block_scale(m, C.byref(s), C.byref(i))
        return s.value, i.value

    assert bs(1.0) == (2.0 ** -8, 256.0)
    assert bs(1.75) == (2.0 ** -8, 256.0)
    assert bs(1.8) == (2.0 ** -7, 128.0)
    assert bs(3.0e4) == (2.0 ** 7, 2.0 ** -7)
    row = np.full(128, 0.3, dtype=np.float32)
    row[0] = 1.0
    L.oref_fake_quant_row(oracle.ptr(row), 128)
    assert row[0] == 1.0
    assert row[1] == 0.3125


def test_quant_row_matches_the_c_reference_golden(oracle):
    # fake_quant.rs:181-226 over tests/golden/pq_golden.txt
    k, rows = 256, 6
    x = np.zeros(rows * k, dtype=np.float32)
    want_q = np.zeros(rows * k, dtype=np.uint8)
    want_s = np.zeros(rows * 2, dtype=np.float32)
    nq = ns = 0
    with open(os.path.join(GOLDEN, "pq_golden.txt")) as f:
        for line in f:
            p = line.split()
            if p[0] == "S":
                r, b = int(p[1]), int(p[2])
                want_s[r * 2 + b] = bits_f32(int(p[3], 16))
                ns += 1
            elif p[0] == "Q":
                x[nq] = bits_f32(int(p[1], 16))
                want_q[nq] = int(p[2], 16)
                nq += 1
            else:
                raise AssertionError(line)
    assert (nq, ns) == (rows * k, rows * 2)
    q = np.zeros(rows * k, dtype=np.uint8)
    s = np.zeros(rows * 2, dtype=np.float32)
    L = oracle.lib()
    for r in range(rows):
        L.oref_quant_row(oracle.ptr(x[r * k:(r + 1) * k]), k,
                         oracle.ptr(q[r * k:(r + 1) * k]), oracle.ptr(s[r * 2:(r + 1) * 2]))
    assert int((q != want_q).sum()) == 0
    assert int((s.view(np.uint32) != want_s.view(np.uint32)).sum()) == 0


def test_a_planted_quantiser_mistake_is_caught_by_the_golden(oracle):
    # The golden table discriminates: flooring instead of round-to-nearest-even changes codes.
    k = 256
    with open(os.path.join(GOLDEN, "pq_golden.txt")) as f:
        lines = [l.split() for l in f if l.startswith("Q")]
    x = np.array([bits_f32(int(p[1], 16)) for p in lines[:k]], dtype=np.float32)
    want = np.array([int(p[2], 16) for p in lines[:k]], dtype=np.uint8)
    L = oracle.lib()
    import ctypes as C
    bad = 0
    for b in range(2):
        blk = x[b * 128:(b + 1) * 128]
        m = max(float(np.abs(blk).max()), 2.0 ** -100)
        s, inv = C.c_float(), C.c_float()
        L.oref_block_scale(m, C.byref(s), C.byref(inv))
        for j, v in enumerate(blk):
            a = abs(float(np.float32(v * inv.value)))
            # the mutant: truncate the mantissa instead of rounding
            if a >= 2.0 ** -6:
                e = int(np.floor(np.log2(a)))
                mm = int((a / 2.0 ** e - 1) * 8)
                code = ((e + 7) << 3) | mm
            else:
                code = int(a * 512)
            code = min(code, 0x7E) | (0x80 if v < 0 else 0)
            bad += code != want[b * 128 + j]
    assert bad > 10
