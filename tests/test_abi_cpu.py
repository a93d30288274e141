"""The C-ABI boundary without a GPU: the library loads, exports every symbol the header
declares (the shared library for dlopen / ctypes users and the static archive the reference's
crates link with -lomega_gpu), the struct mirrors have the byte layouts the header asserts, and
the checks that run before any device work refuse bad arguments with the reference's codes.
A C program built by gcc against the header and linked to the static archive the way the
crates link it (no hipcc) runs without a GPU: every hot entry answers CHIP_FAIL with a message.

Reference: crates/*/build.rs detect the archive by `nm` lines ending " T <symbol>"
(crates/aien-omega-fp8/build.rs:51-70, router/build.rs:45-52, dattn/build.rs:45-47,
bf16/build.rs:45-47, dgraph/build.rs:44-46); return codes crates/aien-omega-gpu/src/ffi.rs:32-37;
layouts fp8/src/lib.rs:787-810, router/src/lib.rs:494-508, dattn/src/lib.rs:445-456,
dgraph/src/lib.rs:531-548, omega-gpu/src/ffi.rs:318-400.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "omega_gpu.h")
BUILD = os.path.join(REPO, "aien-sovereign-core-mv_amd", "_build")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omega_gpu_\w+)\s*\(", text)))


def exported(path):
    out = subprocess.run(["nm", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_header_declares_the_hot_path_families():
    syms = declared_symbols()
    assert len(syms) > 90
    # the detection symbols of every crate's build script
    for s in ("omega_gpu_fp8_gemv_grouped_f32", "omega_gpu_fp8_gemv_grouped_dev",
              "omega_gpu_fp8_tensor_entry", "omega_gpu_fp8gemm_f32",
              "omega_gpu_fp8_grouped_ctas_auto", "omega_gpu_router", "omega_gpu_decode_attn",
              "omega_gpu_bf16_gemv_f32", "omega_gpu_decode_graph_create",
              "omega_gpu_paged_attention_bf16", "omega_gpu_paged_attention_batch_bf16"):
        assert s in syms, s


@pytest.mark.parametrize("name", ["libomega_gpu.so", "libomega_gpu.a"])
def test_every_declared_symbol_is_exported(name):
    path = os.path.join(BUILD, name)
    assert os.path.exists(path), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    missing = [s for s in declared_symbols() if s not in exported(path)]
    assert not missing, missing


ROCM_LIB = "/opt/rocm/lib"


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="this host has a GPU driver")
def test_static_archive_links_from_c_and_answers_chip_fail_without_a_gpu(tmp_path):
    archive = os.path.join(BUILD, "libomega_gpu.a")
    assert os.path.exists(archive), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    exe = str(tmp_path / "static_link_driver")
    # the reference's build.rs link line: -lomega_gpu, the HIP runtime, -lstdc++ -lpthread -lm
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.dirname(HEADER),
                    os.path.join(REPO, "tests", "c", "static_link_driver.c"), archive,
                    "-L" + ROCM_LIB, "-Wl,-rpath," + ROCM_LIB, "-lamdhip64", "-lstdc++",
                    "-lpthread", "-lm", "-o", exe], check=True, capture_output=True, text=True)
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    lines = run.stdout.splitlines()
    assert run.returncode == 0, run.stdout + run.stderr
    assert lines[-1] == "0 failed"
    chip = [ln for ln in lines if "(CHIP_FAIL)" in ln]
    assert len(chip) == 7 and all(ln.startswith("ok ") and "no HIP device" in ln for ln in chip), lines


def test_library_loads_without_a_gpu_and_mirrors_match_the_header():
    import omega_amd as om

    lib = om.lib()
    assert lib is not None
    sizes = {om.Fp8Info: 160, om.GemmInfo: 80, om.RouterInfo: 48, om.DecodeAttnInfo: 64,
             om.Bf16Info: 136, om.GraphStats: 40, om.GraphConfig: 40, om.AttnInfo: 176,
             om.KvLayout: 64}
    for t, n in sizes.items():
        assert C.sizeof(t) == n, t.__name__
    assert om.Fp8Info.weight_bytes.offset == 48
    assert om.Fp8Info.kernel_cache_hit.offset == 84
    assert om.Fp8Info.sm_architecture.offset == 152
    assert om.GraphConfig.router.offset == 16 and om.GraphConfig.lm_head.offset == 32
    assert om.AttnInfo.kv_source.offset == 168 and om.KvLayout.block_size.offset == 56


def test_host_checks_refuse_before_touching_the_device():
    import omega_amd as om

    lib = om.lib()
    # return-code names (ffi.rs:32-37)
    assert om._s(lib.omega_gpu_fp8_rc_name(0)) == "OK"
    assert om._s(lib.omega_gpu_fp8_rc_name(-1)) == "BAD_ARGS"
    assert om._s(lib.omega_gpu_attention_rc_name(-5)) == "UNWRITTEN"
    # shape rules run before any HIP call
    assert lib.omega_gpu_fp8_prepare(100) == -1
    assert lib.omega_gpu_fp8_prepare(4096) == 0
    assert lib.omega_gpu_bf16_prepare(100) == -1
    assert lib.omega_gpu_fp8gemm_prepare(0) == -1
    # a graph with zero layers is refused before any handle is read (dgraph/src/lib.rs:552-576)
    cfg = om.GraphConfig(layers=0, vocab=10, eps=1e-6, norm_topk=1, router=None, attn=None,
                         lm_head=None)
    out = C.c_void_p(123)
    assert lib.omega_gpu_decode_graph_create(C.byref(cfg), C.byref(out)) == -1
    assert out.value is None
    assert "layers" in om._s(lib.omega_gpu_session_last_error())
    # serving bounds are checked before the device is opened (head_dim 64, a block of 12)
    for bad in (dict(head_dim=64), dict(kv_block_size=12), dict(max_seqs=0), dict(kernel_slots=129)):
        kw = dict(max_context=640, max_seqs=4, num_q_heads=32, num_kv_heads=4, head_dim=128, kv_block_size=16,
                  max_rows=1, max_k=2048, max_n=2048, max_n_one_row=0, kernel_slots=8)
        kw.update(bad)
        with pytest.raises(om.OmegaGpuError, match="serving bounds refused"):
            om.reserve_serving(**kw)
    assert C.sizeof(om.ServingBounds) == 44 and C.sizeof(om.AllocStats) == 40
    # NULL handles
    assert lib.omega_gpu_fp8_tensor_entry(None, 0, None, None) == -1


def test_kv_layout_helper_matches_the_oracle(oracle):
    import omega_amd

    for args in ((100, 16, 48, 4, 128), (7, 16, 2, 4, 128), (3, 8, 1, 2, 64)):
        a, b = omega_amd.kv_layout(*args), oracle.kv_layout(*args)
        assert [getattr(a, f) for f, _ in a._fields_] == [getattr(b, f) for f, _ in b._fields_]
