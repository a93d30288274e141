"""ABI qualification against the reference's Omega manifest (CPU).

tests/golden/omega_gpu.manifest is crates/aien-omega-gpu/abi/omega_gpu.manifest unchanged: the
facts the reference's build checks an Omega archive against before it links it
(aien-abi-conformance src/build.rs:166-239, src/probe.rs:40-140). omega_amd.qualify runs the same
three checks against include/omega_gpu.h and the built libomega_gpu.a / .so: struct fields in
manifest order and function prototypes of the manifest's signatures, a C layout probe compiled
against the header, and the archive's defined symbols. Planted mistakes on either side must be
reported, so the check cannot pass vacuously.
"""
import os
import re
import shutil
import tempfile

import pytest

from omega_amd import qualify

MANIFEST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "omega_gpu.manifest")


@pytest.fixture(scope="module")
def text():
    return open(MANIFEST).read()


def test_library_qualifies_against_the_reference_manifest(text):
    report, errs = qualify.check(text)
    assert errs == [], "\n".join(errs)
    m = qualify.Manifest(text)
    assert len(m.structs) == 6 and len(m.fns) == 34 and len(m.consts) == 23, report


@pytest.mark.parametrize("old,new,needle", [
    ("field OmegaGpuKvLayout num_layers 52 4 u32 1", "field OmegaGpuKvLayout num_layers 56 4 u32 1",
     "layout: C `field OmegaGpuKvLayout num_layers 52 4 u32 1`"),
    ("struct OmegaGpuAttnInfo 176 8", "struct OmegaGpuAttnInfo 184 8", "struct OmegaGpuAttnInfo"),
    ("field OmegaGpuMatmulInfo target_chip 65 64 c_char 64", "field OmegaGpuMatmulInfo target_chip 65 64 u8 64",
     "field OmegaGpuMatmulInfo target_chip"),
    ("field OmegaGpuAllocStats frees 24 8 u64 1", "field OmegaGpuAllocStats freed 24 8 u64 1",
     "struct OmegaGpuAllocStats: C fields"),  # the probe does not compile either
    ("const OMEGA_GPU_ATTN_TOO_LARGE -2", "const OMEGA_GPU_ATTN_TOO_LARGE -3", "const OMEGA_GPU_ATTN_TOO_LARGE"),
    ("fn omega_gpu_session_set_spin_us fn(u32) -> i32", "fn omega_gpu_session_set_spin_us fn(u64) -> i32",
     "fn omega_gpu_session_set_spin_us: C signature"),
    ("fn omega_gpu_attention_pool_alloc fn(usize, *mut *mut c_void) -> i32",
     "fn omega_gpu_attention_pool_alloc fn(usize, *mut c_void) -> i32", "fn omega_gpu_attention_pool_alloc"),
    ("fn omega_gpu_device_close fn() -> ()", "fn omega_gpu_device_close fn() -> ()\nfn omega_gpu_not_there fn() -> ()",
     "symbol omega_gpu_not_there: not defined in libomega_gpu.a"),
])
def test_manifest_side_mistakes_are_reported(text, old, new, needle):
    assert old in text
    _, errs = qualify.check(text.replace(old, new))
    assert any(needle in e for e in errs), errs


def test_header_side_mistakes_are_reported(text):
    """Two fields of the KV layout swapped in a copy of the header: the field-order check and the
    probe's offsets both report it."""
    src = open(qualify.HEADER).read()
    a = "    uint32_t num_blocks, num_layers, block_size;"
    assert a in src
    with tempfile.TemporaryDirectory() as d:
        h = os.path.join(d, "omega_gpu.h")
        open(h, "w").write(src.replace(a, "    uint32_t num_layers, num_blocks, block_size;"))
        _, errs = qualify.check(text, header=h)
    assert any(e.startswith("struct OmegaGpuKvLayout: C fields") for e in errs), errs
    assert any("field OmegaGpuKvLayout num_blocks 52" in e for e in errs), errs


def test_prototype_conversion():
    src = "int f0(void); const char *omega_gpu_x(int rc); void omega_gpu_y(void);\n" \
          "int omega_gpu_z(const float *a, void **b, const OmegaGpuKvLayout *l, size_t n, uint32_t k);"
    fns = qualify.header_fns(src)
    assert fns == {"omega_gpu_x": "fn(i32) -> *const c_char", "omega_gpu_y": "fn() -> ()",
                   "omega_gpu_z": "fn(*const f32, *mut *mut c_void, *const OmegaGpuKvLayout, usize, u32) -> i32"}
