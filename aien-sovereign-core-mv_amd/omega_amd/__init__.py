"""ctypes binding of libomega_gpu (the MI355X decode-step library) for tests and the benchmark.

The classes mirror the reference's safe Rust wrappers (crates/aien-omega-fp8, -router, -dattn,
-bf16, -dgraph): the same host-side shape and length checks run before any call crosses the C
ABI, and a non-zero return code becomes OmegaGpuError carrying the rc name and last_error text.
There is no fallback: when the library is not built, loading it raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
# OMEGA_GPU_LIB selects another build of the same library (a tuning variant); default: in-tree
LIB_PATH = os.environ.get("OMEGA_GPU_LIB") or os.path.join(PKG, "_build", "libomega_gpu.so")

_lib = None


class OmegaGpuError(RuntimeError):
    def __init__(self, rc: int, name: str):
        super().__init__(f"rc {rc}: {name}")
        self.rc = rc
        self.name = name


class ShapeMismatch(ValueError):
    def __init__(self, what: str, expected: int, got: int):
        super().__init__(f"{what}: expected {expected}, got {got}")
        self.what, self.expected, self.got = what, expected, got


# ------------------------------------------------------------------ C structs (include/omega_gpu.h)
class Fp8Info(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("experts", "n", "k", "groups", "lane_bytes",
                                          "rows_per_warp", "warps_per_cta", "depth", "grid_x",
                                          "grid_y", "steps")] + [
        ("weight_bytes", C.c_uint64), ("scale_bytes", C.c_uint64), ("elapsed_ns", C.c_uint64),
        ("call_ns", C.c_uint64), ("completion_marker", C.c_uint32),
        ("kernel_cache_hit", C.c_bool), ("target_chip", C.c_char * 64),
        ("sm_architecture", C.c_uint32)]


class GemmInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("rows", "segments", "n", "k", "mt", "warps_per_cta",
                                          "lane_bytes", "grid_x", "grid_y", "passes_max")] + [
        ("weight_bytes", C.c_uint64), ("streamed_bytes", C.c_uint64), ("elapsed_ns", C.c_uint64),
        ("call_ns", C.c_uint64), ("completion_marker", C.c_uint32),
        ("kernel_cache_hit", C.c_bool)]


class RouterInfo(C.Structure):
    _fields_ = [("layer", C.c_uint32), ("warps", C.c_uint32), ("depth", C.c_uint32),
                ("threads", C.c_uint32), ("weight_bytes", C.c_uint64), ("elapsed_ns", C.c_uint64),
                ("call_ns", C.c_uint64), ("completion_marker", C.c_uint32),
                ("kernel_cache_hit", C.c_int32)]


class DecodeAttnInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("layer", "pos", "splits", "per_split", "depth",
                                          "grid_x", "grid_y", "threads")] + [
        ("kv_bytes", C.c_uint64), ("elapsed_ns", C.c_uint64), ("call_ns", C.c_uint64),
        ("completion_marker", C.c_uint32), ("kernel_cache_hit", C.c_int32)]


class Bf16Info(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n", "k", "rows_per_warp", "warps_per_cta", "depth",
                                          "grid_x", "steps")] + [
        ("weight_bytes", C.c_uint64), ("elapsed_ns", C.c_uint64), ("call_ns", C.c_uint64),
        ("completion_marker", C.c_uint32), ("kernel_cache_hit", C.c_bool),
        ("target_chip", C.c_char * 64), ("sm_architecture", C.c_uint32)]


class GraphStats(C.Structure):
    _fields_ = [("launches", C.c_uint32), ("submits", C.c_uint32), ("chip_ns", C.c_uint64),
                ("record_ns", C.c_uint64), ("total_ns", C.c_uint64), ("sems_done", C.c_uint32)]


class GraphConfig(C.Structure):
    _fields_ = [("layers", C.c_uint32), ("vocab", C.c_uint32), ("eps", C.c_float),
                ("norm_topk", C.c_int32), ("router", C.c_void_p), ("attn", C.c_void_p),
                ("lm_head", C.c_void_p)]


class AttnInfo(C.Structure):
    _fields_ = [("chip_calls", C.c_uint32), ("elapsed_ns", C.c_uint64), ("call_ns", C.c_uint64),
                ("completion_marker", C.c_uint32), ("unwritten_words", C.c_uint32),
                ("gpr_count", C.c_uint32), ("insn_count", C.c_uint32),
                ("kernel_cache_hit", C.c_bool), ("ctas_last_launch", C.c_uint32),
                ("threads_per_cta", C.c_uint32), ("target_chip", C.c_char * 64),
                ("sm_architecture", C.c_uint32), ("kv_bytes_staged", C.c_uint64),
                ("kv_bytes_naive", C.c_uint64), ("kv_blocks_logical", C.c_uint32),
                ("kv_blocks_unique", C.c_uint32), ("q_bytes", C.c_uint64),
                ("tab_bytes", C.c_uint64), ("out_bytes", C.c_uint64), ("kv_source", C.c_uint32)]


class KvLayout(C.Structure):
    _fields_ = [("block_stride_bytes", C.c_uint64), ("layer_stride_bytes", C.c_uint64),
                ("kv_plane_stride_bytes", C.c_uint64), ("token_stride_bytes", C.c_uint64),
                ("head_stride_bytes", C.c_uint64), ("pool_bytes", C.c_uint64),
                ("num_blocks", C.c_uint32), ("num_layers", C.c_uint32),
                ("block_size", C.c_uint32)]


class BatchDecodeConfig(C.Structure):
    """OmegaGpuBatchDecodeConfig (include/omega_gpu.h), 136 bytes."""
    _fields_ = [("layers", C.c_uint32), ("vocab", C.c_uint32), ("max_seqs", C.c_uint32),
                ("max_blocks_per_seq", C.c_uint32), ("max_pos", C.c_uint32), ("eps", C.c_float),
                ("norm_topk", C.c_int32), ("rope_theta", C.c_double), ("router", C.c_void_p),
                ("lm_head", C.c_void_p), ("embed", C.c_void_p), ("pool", C.c_void_p),
                ("layout", KvLayout)]


class ServingBounds(C.Structure):
    """OmegaGpuServingBounds (include/omega_gpu.h), 44 bytes."""
    _fields_ = [(n, C.c_uint32) for n in ("max_context", "max_seqs", "num_q_heads", "num_kv_heads", "head_dim",
                                          "kv_block_size", "max_rows", "max_k", "max_n", "max_n_one_row",
                                          "kernel_slots")]


class AllocStats(C.Structure):
    """OmegaGpuAllocStats (include/omega_gpu.h), 40 bytes."""
    _fields_ = [(n, C.c_uint64) for n in ("allocs", "alloc_bytes", "alloc_failures", "frees", "stale_refusals")]


P = C.c_void_p
U8P, U16P, U32P, U64P, F32P = (C.POINTER(C.c_uint8), C.POINTER(C.c_uint16),
                                C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_float))
u32, i32, u64, f32, f64 = C.c_uint32, C.c_int32, C.c_uint64, C.c_float, C.c_double
cstr = C.c_char_p

SIGNATURES = {
    # FP8 (crates/aien-omega-fp8/src/lib.rs:132-207)
    "omega_gpu_fp8_tensor_upload": (i32, [u32, u32, u32, P, P, C.POINTER(P)]),
    "omega_gpu_fp8_tensor_free": (None, [P]),
    "omega_gpu_fp8_gemv_f32": (i32, [P, u32, P, P, C.POINTER(Fp8Info)]),
    "omega_gpu_fp8_gemv_grouped_f32": (i32, [P, u32, P, P, u32, P, C.POINTER(Fp8Info)]),
    "omega_gpu_fp8_gemv_grouped_dev": (i32, [P, u32, u64, u64, P, C.POINTER(Fp8Info)]),
    "omega_gpu_fp8_tensor_entry": (i32, [P, u32, U64P, U64P]),
    "omega_gpu_fp8gemm_f32": (i32, [P, u32, P, P, P, u32, P, C.POINTER(GemmInfo)]),
    "omega_gpu_fp8gemm_prepare": (i32, [u32]),
    "omega_gpu_fp8gemm_rc_name": (cstr, [i32]),
    "omega_gpu_fp8gemm_last_error": (cstr, []),
    "omega_gpu_fp8gemm_test_set_mutant": (None, [i32]),
    "omega_gpu_fp8_grouped_ctas_auto": (u32, [u32]),
    "omega_gpu_fp8_prepare": (i32, [u32]),
    "omega_gpu_fp8_seal": (None, [i32]),
    "omega_gpu_fp8_rc_name": (cstr, [i32]),
    "omega_gpu_fp8_last_error": (cstr, []),
    "omega_gpu_fp8_cache_clear": (None, []),
    "omega_gpu_fp8_set_shape": (None, [u32, u32, u32]),
    "omega_gpu_fp8_set_cta_budget": (None, [u32]),
    "omega_gpu_fp8_test_set_mutant": (None, [i32]),
    "omega_gpu_fp8_test_set_no_fold": (None, [i32]),
    # router (crates/aien-omega-router/src/lib.rs:78-132)
    "omega_gpu_router_alloc_shape": (i32, [u32, u32, u32, C.POINTER(P)]),
    "omega_gpu_router_free": (None, [P]),
    "omega_gpu_router_set_layer": (i32, [P, u32, P, P]),
    "omega_gpu_router_set_directory": (i32, [P, u32, P, P]),
    "omega_gpu_router": (i32, [P, u32, P, f32, i32, f32, P, P, C.POINTER(RouterInfo)]),
    "omega_gpu_router_device_outputs": (None, [P, U64P, U64P, U64P]),
    "omega_gpu_router_read_back": (i32, [P, P, P, P]),
    "omega_gpu_router_last_error": (cstr, []),
    "omega_gpu_router_rc_name": (cstr, [i32]),
    "omega_gpu_router_test_set_mutant": (None, [i32]),
    # decode attention (crates/aien-omega-dattn/src/lib.rs:80-136)
    "omega_gpu_decode_attn_cache_alloc": (i32, [u32, u32, f64, C.POINTER(P)]),
    "omega_gpu_decode_attn_cache_free": (None, [P]),
    "omega_gpu_decode_attn_set_norms": (i32, [P, u32, P, P]),
    "omega_gpu_decode_attn": (i32, [P, u32, u32, P, f32, f32, P, C.POINTER(DecodeAttnInfo)]),
    "omega_gpu_decode_attn_last_error": (cstr, []),
    "omega_gpu_decode_attn_rc_name": (cstr, [i32]),
    "omega_gpu_decode_attn_set_depth": (None, [u32]),
    "omega_gpu_decode_attn_set_per_split": (None, [u32]),
    "omega_gpu_decode_attn_test_set_mutant": (None, [i32]),
    "omega_gpu_paged_attention_set_folded": (None, [i32]),
    "omega_gpu_decode_attn_cache_write": (i32, [P, u32, u32, u32, u32, P, P]),
    "omega_gpu_decode_attn_cache_read": (i32, [P, u32, u32, u32, P, P]),
    "omega_gpu_decode_attn_cache_payload_len": (u64, [P, u32]),
    "omega_gpu_decode_attn_cache_export": (i32, [P, u32, u32, P, u64, P]),
    "omega_gpu_decode_attn_cache_export_dev": (i32, [P, u32, u32, P, u64, P]),
    "omega_gpu_decode_attn_cache_import": (i32, [P, u32, u32, P, u64, P]),
    "omega_gpu_decode_attn_cache_import_dev": (i32, [P, u32, u32, P, u64, P]),
    # bf16 (crates/aien-omega-bf16/src/lib.rs:70-101)
    "omega_gpu_bf16_tensor_upload": (i32, [u32, u32, P, C.POINTER(P)]),
    "omega_gpu_bf16_tensor_free": (None, [P]),
    "omega_gpu_bf16_gemv_f32": (i32, [P, P, P, C.POINTER(Bf16Info)]),
    "omega_gpu_bf16_gemv_bf16": (i32, [P, P, P, C.POINTER(Bf16Info)]),
    "omega_gpu_bf16_prepare": (i32, [u32]),
    "omega_gpu_bf16_rc_name": (cstr, [i32]),
    "omega_gpu_bf16_last_error": (cstr, []),
    "omega_gpu_bf16_test_set_mutant": (None, [i32]),
    # decode graph (crates/aien-omega-dgraph/src/lib.rs:113-165)
    "omega_gpu_decode_graph_create": (i32, [C.POINTER(GraphConfig), C.POINTER(P)]),
    "omega_gpu_decode_graph_free": (None, [P]),
    "omega_gpu_decode_graph_set_layer": (i32, [P, u32, P, P, P, P, P]),
    "omega_gpu_decode_graph_set_final_norm": (i32, [P, P]),
    "omega_gpu_decode_graph_token": (i32, [P, P, u32, U32P, C.POINTER(GraphStats)]),
    "omega_gpu_decode_graph_read": (i32, [P, P, P, P]),
    "omega_gpu_decode_graph_set_flush_each": (None, [P, i32]),
    "omega_gpu_decode_graph_test_set_mutant": (None, [P, i32]),
    "omega_gpu_decode_graph_set_stamps": (None, [P, i32]),
    "omega_gpu_decode_graph_stamps": (i32, [P, U64P, U8P, u32]),
    "omega_gpu_decode_graph_kind_name": (cstr, [C.c_uint8]),
    "omega_gpu_session_last_error": (cstr, []),
    "omega_gpu_reserve_serving": (i32, [C.POINTER(ServingBounds)]),
    "omega_gpu_matmul_last_error": (cstr, []),
    "omega_gpu_serving_seal": (None, []),
    "omega_gpu_serving_release": (None, []),
    "omega_gpu_session_alloc_stats": (None, [C.POINTER(AllocStats)]),
    # base ABI (crates/aien-omega-gpu/src/ffi.rs)
    "omega_gpu_session_set_spin_us": (i32, [u32]),
    "omega_gpu_session_spin_us": (u32, []),
    "omega_gpu_attention_pool_alloc": (i32, [C.c_size_t, C.POINTER(P)]),
    "omega_gpu_attention_pool_free": (None, []),
    "omega_gpu_paged_attention_bf16": (i32, [P, P, C.POINTER(KvLayout), P, u32, u32, u32, u32,
                                             u32, u32, P, C.POINTER(AttnInfo)]),
    "omega_gpu_paged_attention_batch_bf16": (i32, [P, P, C.POINTER(KvLayout), P, P, u32, u32,
                                                   u32, u32, u32, u32, P, C.POINTER(AttnInfo)]),
    "omega_gpu_attention_rc_name": (cstr, [i32]),
    "omega_gpu_attention_last_error": (cstr, []),
    # device-resident extensions
    "omega_gpu_fp8_tensor_synth": (i32, [u32, u32, u32, u64, u64, f32, C.POINTER(P)]),
    "omega_gpu_bf16_tensor_synth": (i32, [u32, u32, u64, u64, f32, C.POINTER(P)]),
    "omega_gpu_synth_bf16_host": (None, [u64, u64, C.c_size_t, f32, i32, P]),
    "omega_gpu_synth_bf16_dev": (i32, [P, u64, u64, u64, f32]),
    "omega_gpu_moe_batch_f32": (i32, [P, u32, P, P, u32, P, f32, i32, P, P, P]),
    "omega_gpu_moe_batch_dev": (i32, [P, u32, P, P, u32, P, f32, i32, P, P, P, P]),
    "omega_gpu_moe_test_set_mutant": (None, [i32]),
    "omega_gpu_batch_decode_create": (i32, [C.POINTER(BatchDecodeConfig), C.POINTER(P)]),
    "omega_gpu_batch_decode_free": (None, [P]),
    "omega_gpu_batch_decode_set_layer": (i32, [P, u32, P, P, P, P, P, P, P]),
    "omega_gpu_batch_decode_set_final_norm": (i32, [P, P]),
    "omega_gpu_batch_decode_set_tables": (i32, [P, u32, P]),
    "omega_gpu_batch_decode_set_keep_logits": (None, [P, i32]),
    "omega_gpu_batch_decode_set_eager": (None, [P, i32]),
    "omega_gpu_batch_decode_step": (i32, [P, u32, P, P, P]),
    "omega_gpu_batch_decode_read": (i32, [P, u32, P, P, P, P]),
    "omega_gpu_fp8_gemv_dev": (i32, [P, u32, P, P]),
    "omega_gpu_paged_attention_batch_dev": (i32, [P, P, C.POINTER(KvLayout), P, P, u32, u32, u32,
                                                  u32, u32, u32, u32, P]),
    "omega_gpu_paged_attention_batch_dev_noalloc": (i32, [P, P, C.POINTER(KvLayout), P, P, u32, u32, u32,
                                                          u32, u32, u32, u32, P]),
    "omega_gpu_paged_attention_items_dev": (i32, [P, P, C.POINTER(KvLayout), P, u32, P, u32, u32, P]),
    # whole-prompt prefill (crates/aien-omega-pf/src/lib.rs:384-456, :542-571)
    "omega_gpu_pf_rc_name": (cstr, [i32]),
    "omega_gpu_pf_alloc_dev": (i32, [C.c_size_t, P]),
    "omega_gpu_pf_alloc_host": (i32, [C.c_size_t, P]),
    "omega_gpu_pf_free": (None, [P]),
    "omega_gpu_pf_copy_va": (i32, [u64, u64, C.c_size_t]),
    "omega_gpu_pf_stats": (None, [P, P]),
    "omega_gpu_pf_stats_reset": (None, []),
    "omega_gpu_pf_quant": (i32, [u32, u32, u32, u64, u64, u64, P]),
    "omega_gpu_pf_qgemm_bm": (u32, []),
    "omega_gpu_pf_qgemm_tiles_va": (u32, [u32, P, P, P, P, u32]),
    "omega_gpu_pf_qgemm": (i32, [u32, u32, u32, u64, u32, u64, u64, u64, u64, P]),
    "omega_gpu_pf_router_rows": (u32, []),
    "omega_gpu_pf_router_pack": (None, [u32, u32, P, P]),
    "omega_gpu_pf_router_logits": (i32, [u32, u32, u32, u64, u64, u64, P]),
    "omega_gpu_pf_moe_combine": (i32, [u32, u32, u32, u64, u64, u64, u64, P]),
    "omega_gpu_prefill_attn": (i32, [P, u32, u32, u32, P, f32, f32, P, P]),
    "omega_gpu_prefill_attn_dev": (i32, [P, u32, u32, u32, u64, f32, f32, u64, P]),
    "omega_gpu_pf_residual_norm": (i32, [u32, u32, u64, u64, u64, f32, u64, P]),
    "omega_gpu_pf_moe_plan": (i32, [u32, u32, u32, P, P, P, P, P, P, P]),
    "omega_gpu_decode_graph_read_routes": (i32, [P, P, P]),
    "omega_gpu_decode_graph_test_force_routes": (i32, [P, P]),
    "omega_gpu_decode_graph_test_set_trace": (i32, [P, P, u32]),
    "omega_gpu_decode_graph_test_read_trace": (i32, [P, u32, P, P, P, P, P, P, P, P]),
    "omega_gpu_decode_graph_kernel_ns": (i32, [P, U64P, u32]),
    "omega_gpu_decode_graph_set_persistent": (i32, [P, i32]),
    "omega_gpu_decode_graph_set_stage_stamps": (None, [P, i32]),
    "omega_gpu_decode_graph_stage_ns": (i32, [P, U64P, u32]),
    "omega_gpu_decode_graph_set_embedding": (i32, [P, P]),
    "omega_gpu_decode_graph_token_id": (i32, [P, u32, u32, U32P, C.POINTER(GraphStats)]),
    "omega_gpu_stream": (P, []),
    "omega_gpu_sync": (i32, []),
}


def lib():
    """The loaded library. Raises when it is not built: there is no fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libomega_gpu is not built ({LIB_PATH} missing): run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def gpu_count() -> int:
    try:
        hip = C.CDLL("libamdhip64.so")
    except OSError:
        return 0
    n = C.c_int(0)
    if hip.hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def require_gpu():
    """Raises when no GPU is visible or the library is not built: a caller that needs the device
    fails loudly rather than passing without it."""
    if gpu_count() == 0:
        raise RuntimeError("no HIP device is visible: the MI355X path needs a GPU")
    lib()


def ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def _s(b):
    return b.decode() if b else ""


def _check(rc, family):
    if rc != 0:
        L = lib()
        name = _s(getattr(L, f"omega_gpu_{family}_rc_name")(rc))
        err = _s(getattr(L, f"omega_gpu_{family}_last_error")())
        raise OmegaGpuError(rc, f"{name}: {err}" if err else name)


def check_len(what, expected, got):
    if expected != got:
        raise ShapeMismatch(what, expected, got)


# ------------------------------------------------------------------ FP8 (aien-omega-fp8)
BLOCK, MAX_GROUPS, MAX_K = 128, 64, 32768
GEMM_MAX_ROWS, GEMM_MAX_SEGMENTS = 1024, 256


def fp8_check_shape(experts, n, k):
    """crates/aien-omega-fp8/src/lib.rs:246-259"""
    if experts == 0 or n == 0 or n % BLOCK or k % BLOCK or not (BLOCK <= k <= MAX_K):
        raise OmegaGpuError(-1, f"fp8 shape experts={experts} n={n} k={k} refused")


class Fp8Tensor:
    """crates/aien-omega-fp8/src/lib.rs:263-604"""

    def __init__(self, handle, experts, n, k):
        self.h, self.experts, self.n, self.k = handle, experts, n, k

    @classmethod
    def upload(cls, experts, n, k, w, scale_inv_bf16):
        fp8_check_shape(experts, n, k)
        w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
        s = np.ascontiguousarray(scale_inv_bf16, dtype=np.uint16).reshape(-1)
        check_len("fp8 weight bytes", experts * n * k, w.size)
        check_len("fp8 scale words", experts * (n // BLOCK) * (k // BLOCK), s.size)
        h = C.c_void_p()
        rc = lib().omega_gpu_fp8_tensor_upload(experts, n, k, ptr(w), ptr(s), C.byref(h))
        _check(rc, "fp8")
        return cls(h, experts, n, k)

    @classmethod
    def synth(cls, experts, n, k, seed, tensor_id, sigma=0.02):
        fp8_check_shape(experts, n, k)
        h = C.c_void_p()
        _check(lib().omega_gpu_fp8_tensor_synth(experts, n, k, seed, tensor_id, sigma,
                                                C.byref(h)), "fp8")
        return cls(h, experts, n, k)

    def as_raw(self):
        return self.h

    def resident_bytes(self):
        return self.experts * self.n * self.k + self.experts * (self.n // BLOCK) * (self.k // BLOCK) * 4

    def gemv_f32(self, expert, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        check_len("fp8 x", self.k, x.size)
        if expert >= self.experts:
            raise OmegaGpuError(-1, f"fp8 expert {expert} >= experts {self.experts}")
        y = np.empty(self.n, dtype=np.float32)
        info = Fp8Info()
        _check(lib().omega_gpu_fp8_gemv_f32(self.h, expert, ptr(x), ptr(y), C.byref(info)), "fp8")
        return y, info

    def gemv_grouped_f32(self, ids, x):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        g = ids.size
        if g == 0 or g > MAX_GROUPS:
            raise OmegaGpuError(-1, f"fp8 groups {g} outside 1..={MAX_GROUPS}")
        if (ids >= self.experts).any():
            raise OmegaGpuError(-1, "fp8 expert id out of range")
        x_rows = 1 if x.size == self.k else g
        check_len("fp8 x (k or groups*k)", x_rows * self.k, x.size)
        y = np.empty((g, self.n), dtype=np.float32)
        info = Fp8Info()
        _check(lib().omega_gpu_fp8_gemv_grouped_f32(self.h, g, ptr(ids), ptr(x), x_rows, ptr(y),
                                                    C.byref(info)), "fp8")
        return y, info

    def entry(self, expert):
        if expert >= self.experts:
            raise OmegaGpuError(-1, f"fp8 expert {expert} >= experts {self.experts}")
        w, s = C.c_uint64(), C.c_uint64()
        _check(lib().omega_gpu_fp8_tensor_entry(self.h, expert, C.byref(w), C.byref(s)), "fp8")
        return w.value, s.value

    def gemv_grouped_dev(self, groups, tab_va, x_va):
        if groups == 0 or groups > MAX_GROUPS:
            raise OmegaGpuError(-1, f"fp8 groups {groups} outside 1..={MAX_GROUPS}")
        if tab_va == 0 or x_va == 0:
            raise OmegaGpuError(-1, "fp8 device table or row address is 0")
        y = np.empty((groups, self.n), dtype=np.float32)
        info = Fp8Info()
        _check(lib().omega_gpu_fp8_gemv_grouped_dev(self.h, groups, tab_va, x_va, ptr(y),
                                                    C.byref(info)), "fp8")
        return y, info

    def gemm_f32(self, expert_ids, token_rows, x):
        """crates/aien-omega-fp8/src/lib.rs:514-593"""
        e = np.ascontiguousarray(expert_ids, dtype=np.uint32)
        t = np.ascontiguousarray(token_rows, dtype=np.uint32)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        m = e.size
        if m == 0 or m > GEMM_MAX_ROWS:
            raise OmegaGpuError(-1, f"fp8 gemm rows {m} outside 1..={GEMM_MAX_ROWS}")
        check_len("fp8 gemm token rows", m, t.size)
        if x.size == 0 or x.size % self.k:
            raise OmegaGpuError(-1, "fp8 gemm x length is not a positive multiple of k")
        x_rows = x.size // self.k
        y = np.empty((m, self.n), dtype=np.float32)
        info = GemmInfo()
        rc = lib().omega_gpu_fp8gemm_f32(self.h, m, ptr(e), ptr(t), ptr(x), x_rows, ptr(y),
                                         C.byref(info))
        _check(rc, "fp8gemm")
        return y, info

    def free(self):
        if self.h:
            lib().omega_gpu_fp8_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ router (aien-omega-router)
EXPERTS, HIDDEN, TOP_K, ROUTER_MAX_LAYERS = 128, 2048, 8, 64
OUT_SCALE_FP8 = float(2.0 ** 64)


class Router:
    """crates/aien-omega-router/src/lib.rs:182-459"""

    def __init__(self, layers, experts=128, shared=0):
        if layers == 0 or layers > ROUTER_MAX_LAYERS:
            raise OmegaGpuError(-1, f"router layers={layers} refused")
        if experts not in (128, 256) or shared > 1:
            raise OmegaGpuError(-1, f"router shape experts {experts} shared {shared}")
        self.layers, self.rows, self.slots = layers, experts + shared, TOP_K + shared
        h = C.c_void_p()
        _check(lib().omega_gpu_router_alloc_shape(layers, experts, shared, C.byref(h)), "router")
        self.h = h

    def set_layer(self, layer, gate_bf16, norm_w):
        g = np.ascontiguousarray(gate_bf16, dtype=np.uint16).reshape(-1)
        w = np.ascontiguousarray(norm_w, dtype=np.float32)
        check_len("router gate words", self.rows * HIDDEN, g.size)
        check_len("router norm weight", HIDDEN, w.size)
        _check(lib().omega_gpu_router_set_layer(self.h, layer, ptr(g), ptr(w)), "router")

    def set_directory(self, layer, gu, dn):
        gu = np.ascontiguousarray(gu, dtype=np.uint64).reshape(-1)
        dn = np.ascontiguousarray(dn, dtype=np.uint64).reshape(-1)
        check_len("router gate|up directory", self.rows * 2, gu.size)
        check_len("router down directory", self.rows * 2, dn.size)
        _check(lib().omega_gpu_router_set_directory(self.h, layer, ptr(gu), ptr(dn)), "router")

    def route(self, layer, x, eps, norm_topk=True, out_scale=OUT_SCALE_FP8):
        x = np.ascontiguousarray(x, dtype=np.float32)
        check_len("router x", HIDDEN, x.size)
        ids = np.zeros(self.slots, dtype=np.uint32)
        w = np.zeros(self.slots, dtype=np.float32)
        info = RouterInfo()
        _check(lib().omega_gpu_router(self.h, layer, ptr(x), eps, int(norm_topk), out_scale,
                                      ptr(ids), ptr(w), C.byref(info)), "router")
        return ids, w, info

    def device_outputs(self):
        a, b, c = C.c_uint64(), C.c_uint64(), C.c_uint64()
        lib().omega_gpu_router_device_outputs(self.h, C.byref(a), C.byref(b), C.byref(c))
        return a.value, b.value, c.value

    def read_back(self):
        xout = np.zeros(HIDDEN, dtype=np.float32)
        gu = np.zeros(2 * self.slots, dtype=np.uint64)
        dn = np.zeros(2 * self.slots, dtype=np.uint64)
        _check(lib().omega_gpu_router_read_back(self.h, ptr(xout), ptr(gu), ptr(dn)), "router")
        return xout, gu, dn

    def as_raw(self):
        return self.h

    def free(self):
        if self.h:
            lib().omega_gpu_router_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ decode attention (aien-omega-dattn)
Q_HEADS, KV_HEADS, HEAD_DIM, QKV_WORDS, OUT_WORDS = 32, 4, 128, 5120, 4096
POS_ROUND, MAX_POS, DATTN_MAX_LAYERS = 256, 131072, 64


def round_max_pos(max_context):
    """crates/aien-omega-dattn/src/lib.rs:178-184"""
    return min(max(-(-max_context // POS_ROUND), 1), MAX_POS // POS_ROUND) * POS_ROUND


class DecodeAttnCache:
    """crates/aien-omega-dattn/src/lib.rs:205-382 and rows.rs:26-130"""

    def __init__(self, layers, max_pos, rope_theta):
        if (layers == 0 or layers > DATTN_MAX_LAYERS or max_pos == 0 or max_pos > MAX_POS
                or max_pos % POS_ROUND):
            raise OmegaGpuError(-1, f"decode attn cache layers={layers} max_pos={max_pos} refused")
        if not rope_theta > 0:
            raise OmegaGpuError(-1, f"decode attn rope_theta {rope_theta} must be positive")
        self.layers, self.max_pos = layers, max_pos
        h = C.c_void_p()
        _check(lib().omega_gpu_decode_attn_cache_alloc(layers, max_pos, rope_theta, C.byref(h)),
               "decode_attn")
        self.h = h

    def set_norms(self, layer, q_norm, k_norm):
        q = np.ascontiguousarray(q_norm, dtype=np.float32)
        k = np.ascontiguousarray(k_norm, dtype=np.float32)
        check_len("decode attn q_norm", HEAD_DIM, q.size)
        check_len("decode attn k_norm", HEAD_DIM, k.size)
        _check(lib().omega_gpu_decode_attn_set_norms(self.h, layer, ptr(q), ptr(k)), "decode_attn")

    def attend(self, layer, pos, qkv, eps, out_scale=1.0):
        qkv = np.ascontiguousarray(qkv, dtype=np.float32)
        check_len("decode attn qkv", QKV_WORDS, qkv.size)
        if pos >= self.max_pos:
            raise OmegaGpuError(-1, f"decode attn pos {pos} >= max_pos {self.max_pos}")
        out = np.empty(OUT_WORDS, dtype=np.float32)
        info = DecodeAttnInfo()
        _check(lib().omega_gpu_decode_attn(self.h, layer, pos, ptr(qkv), eps, out_scale,
                                           ptr(out), C.byref(info)), "decode_attn")
        return out, info

    def read_row(self, layer, kv_head, pos):
        k = np.empty(HEAD_DIM, dtype=np.uint16)
        v = np.empty(HEAD_DIM, dtype=np.uint16)
        _check(lib().omega_gpu_decode_attn_cache_read(self.h, layer, kv_head, pos, ptr(k), ptr(v)),
               "decode_attn")
        return k, v

    def write_rows(self, layer, kv_head, pos, k, v):
        k = np.ascontiguousarray(k, dtype=np.uint16).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.uint16).reshape(-1)
        if k.size == 0 or k.size % HEAD_DIM:
            raise OmegaGpuError(-1, "decode attn write: not a whole number of rows")
        check_len("decode attn write v", k.size, v.size)
        _check(lib().omega_gpu_decode_attn_cache_write(self.h, layer, kv_head, pos,
                                                       k.size // HEAD_DIM, ptr(k), ptr(v)),
               "decode_attn")

    def payload_len(self, length):
        """bytes of the HostPagedPoolV1 payload of `length` positions"""
        return int(lib().omega_gpu_decode_attn_cache_payload_len(self.h, length))

    def export_kv(self, start, length):
        """the HostPagedPoolV1 payload of positions start .. start + length (qwen3_moe_omega_kvio.rs
        rows_to_blocks) as a uint8 array; returns (payload, chip ns)"""
        out = np.empty(self.payload_len(length), np.uint8)
        ns = C.c_uint64()
        _check(lib().omega_gpu_decode_attn_cache_export(self.h, start, length, out.ctypes.data, out.nbytes,
                                                        C.addressof(ns)), "decode_attn")
        return out, ns.value

    def export_kv_dev(self, start, length, out_dev, nbytes):
        ns = C.c_uint64()
        _check(lib().omega_gpu_decode_attn_cache_export_dev(self.h, start, length, out_dev, nbytes,
                                                            C.addressof(ns)), "decode_attn")
        return ns.value

    def import_kv(self, start, length, payload):
        """writes positions start .. start + length from a HostPagedPoolV1 payload (blocks_to_rows);
        a payload of the wrong size or with non-zero padding rows is refused before any write"""
        b = np.ascontiguousarray(payload, np.uint8)
        ns = C.c_uint64()
        _check(lib().omega_gpu_decode_attn_cache_import(self.h, start, length, b.ctypes.data, b.nbytes,
                                                        C.addressof(ns)), "decode_attn")
        return ns.value

    def import_kv_dev(self, start, length, bytes_dev, nbytes):
        ns = C.c_uint64()
        _check(lib().omega_gpu_decode_attn_cache_import_dev(self.h, start, length, bytes_dev, nbytes,
                                                            C.addressof(ns)), "decode_attn")
        return ns.value

    def as_raw(self):
        return self.h

    def free(self):
        if self.h:
            lib().omega_gpu_decode_attn_cache_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ bf16 lm_head (aien-omega-bf16)
class Bf16Tensor:
    """crates/aien-omega-bf16/src/lib.rs:150-270"""

    def __init__(self, handle, n, k):
        self.h, self.n, self.k = handle, n, k

    @staticmethod
    def check_shape(n, k):
        if n == 0 or k % 256 or not (256 <= k <= 16384):
            raise OmegaGpuError(-1, f"bf16 gemv shape n={n} k={k} refused")

    @classmethod
    def upload(cls, n, k, w_bf16):
        cls.check_shape(n, k)
        w = np.ascontiguousarray(w_bf16, dtype=np.uint16).reshape(-1)
        check_len("bf16 gemv weight words", n * k, w.size)
        h = C.c_void_p()
        _check(lib().omega_gpu_bf16_tensor_upload(n, k, ptr(w), C.byref(h)), "bf16")
        return cls(h, n, k)

    @classmethod
    def synth(cls, n, k, seed, tensor_id, sigma=0.02):
        cls.check_shape(n, k)
        h = C.c_void_p()
        _check(lib().omega_gpu_bf16_tensor_synth(n, k, seed, tensor_id, sigma, C.byref(h)), "bf16")
        return cls(h, n, k)

    def gemv_f32(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        check_len("bf16 gemv x", self.k, x.size)
        y = np.empty(self.n, dtype=np.float32)
        info = Bf16Info()
        _check(lib().omega_gpu_bf16_gemv_f32(self.h, ptr(x), ptr(y), C.byref(info)), "bf16")
        return y, info

    def gemv_bf16(self, x_bits):
        x = np.ascontiguousarray(x_bits, dtype=np.uint16)
        check_len("bf16 gemv x", self.k, x.size)
        y = np.empty(self.n, dtype=np.float32)
        info = Bf16Info()
        _check(lib().omega_gpu_bf16_gemv_bf16(self.h, ptr(x), ptr(y), C.byref(info)), "bf16")
        return y, info

    def as_raw(self):
        return self.h

    def free(self):
        if self.h:
            lib().omega_gpu_bf16_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ decode graph (aien-omega-dgraph)
DGRAPH_HIDDEN, DGRAPH_MAX_LAYERS, MAX_VOCAB = 2048, 64, 2048 * 2048
DGRAPH_RANK = 0xFFFFFFFF  # force_routes: this layer ranks its own logits
KIND_NAMES = ["norm", "qkv", "attn", "o_proj", "res_add", "router", "gate_up", "swiglu", "down",
              "combine_norm", "lm_head", "argmax"]


class DecodeGraph:
    """crates/aien-omega-dgraph/src/lib.rs:230-491"""

    def __init__(self, layers, vocab, eps, router, attn, lm_head, norm_topk=True):
        if layers == 0 or layers > DGRAPH_MAX_LAYERS:
            raise OmegaGpuError(-1, f"decode graph: {layers} layers, 1..={DGRAPH_MAX_LAYERS}")
        if vocab == 0 or vocab > MAX_VOCAB:
            raise OmegaGpuError(-1, f"decode graph: vocab {vocab} outside 1..={MAX_VOCAB}")
        cfg = GraphConfig(layers, vocab, eps, int(norm_topk), router.as_raw(), attn.as_raw(),
                          lm_head.as_raw())
        self._keep = (router, attn, lm_head)
        self.layers, self.vocab = layers, vocab
        h = C.c_void_p()
        rc = lib().omega_gpu_decode_graph_create(C.byref(cfg), C.byref(h))
        if rc != 0:
            raise OmegaGpuError(rc, _s(lib().omega_gpu_session_last_error()))
        self.h = h
        self._tensors = []

    def _rc(self, rc, stage):
        if rc != 0:
            raise OmegaGpuError(rc, f"decode graph {stage}: {_s(lib().omega_gpu_session_last_error())}")

    def set_layer(self, layer, qkv, o, gate_up, down, input_norm):
        w = np.ascontiguousarray(input_norm, dtype=np.float32)
        check_len("decode graph input_norm", DGRAPH_HIDDEN, w.size)
        self._tensors.append((qkv, o, gate_up, down))
        self._rc(lib().omega_gpu_decode_graph_set_layer(self.h, layer, qkv.as_raw(), o.as_raw(),
                                                        gate_up.as_raw(), down.as_raw(), ptr(w)),
                 "set_layer")

    def set_final_norm(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        check_len("decode graph final_norm", DGRAPH_HIDDEN, w.size)
        self._rc(lib().omega_gpu_decode_graph_set_final_norm(self.h, ptr(w)), "set_final_norm")

    def token(self, x_embed, pos):
        x = np.ascontiguousarray(x_embed, dtype=np.float32)
        check_len("decode graph x_embed", DGRAPH_HIDDEN, x.size)
        tok = C.c_uint32()
        st = GraphStats()
        self._rc(lib().omega_gpu_decode_graph_token(self.h, ptr(x), pos, C.byref(tok),
                                                    C.byref(st)), "token")
        return tok.value, st

    def set_embedding(self, embed):
        self._keep_embed = embed
        self._rc(lib().omega_gpu_decode_graph_set_embedding(self.h, embed.as_raw()), "set_embedding")

    def token_id(self, token_in, pos):
        tok = C.c_uint32()
        st = GraphStats()
        self._rc(lib().omega_gpu_decode_graph_token_id(self.h, token_in, pos, C.byref(tok),
                                                       C.byref(st)), "token_id")
        return tok.value, st

    def read(self, x=False, hidden=False, logits=False):
        xs = np.empty(DGRAPH_HIDDEN, np.float32) if x else None
        hs = np.empty(DGRAPH_HIDDEN, np.float32) if hidden else None
        ls = np.empty(self.vocab, np.float32) if logits else None
        self._rc(lib().omega_gpu_decode_graph_read(self.h, ptr(xs), ptr(hs), ptr(ls)), "read")
        return xs, hs, ls

    def read_routes(self):
        ids = np.zeros((self.layers, 8), np.uint32)
        w = np.zeros((self.layers, 8), np.float32)
        self._rc(lib().omega_gpu_decode_graph_read_routes(self.h, ptr(ids), ptr(w)), "read_routes")
        return ids, w

    def force_routes(self, ids):
        """Teacher forcing for parity tests: [layers][8] expert ids in place of the ranking, or
        None to turn it off; a row starting with DGRAPH_RANK (0xFFFFFFFF) leaves that layer's own
        ranking in place."""
        if ids is None:
            self._rc(lib().omega_gpu_decode_graph_test_force_routes(self.h, None), "force_routes")
            return
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        check_len("decode graph forced routes", self.layers * 8, a.size)
        self._rc(lib().omega_gpu_decode_graph_test_force_routes(self.h, ptr(a)), "force_routes")

    def set_trace(self, layers):
        """Layer trace for parity tests: the following tokens run the chain as direct launches
        and record each listed layer's rows (at most 8 layers); None or [] turns it off."""
        a = np.ascontiguousarray(list(layers or []), dtype=np.uint32)
        self._rc(lib().omega_gpu_decode_graph_test_set_trace(self.h, ptr(a) if a.size else None,
                                                             a.size), "set_trace")

    def read_trace(self, i):
        """The last token's record of the i-th traced layer: a dict of x_in, attn_proj, x_mid
        (the residual after the attention), post (the router's normed row), experts, weights,
        moe_out and x_out."""
        rows = {k: np.empty(DGRAPH_HIDDEN, np.float32)
                for k in ("x_in", "attn_proj", "x_mid", "post", "moe_out", "x_out")}
        rows["experts"] = np.empty(8, np.uint32)
        rows["weights"] = np.empty(8, np.float32)
        self._rc(lib().omega_gpu_decode_graph_test_read_trace(
            self.h, i, ptr(rows["x_in"]), ptr(rows["attn_proj"]), ptr(rows["x_mid"]),
            ptr(rows["post"]), ptr(rows["experts"]), ptr(rows["weights"]), ptr(rows["moe_out"]),
            ptr(rows["x_out"])), "read_trace")
        return rows

    def set_stamps(self, on):
        lib().omega_gpu_decode_graph_set_stamps(self.h, int(on))

    def stamps(self):
        cap = DGRAPH_MAX_LAYERS * 16 + 16
        st = np.zeros(cap + 1, np.uint64)
        kinds = np.zeros(cap + 1, np.uint8)
        n = lib().omega_gpu_decode_graph_stamps(self.h, st.ctypes.data_as(U64P),
                                                kinds.ctypes.data_as(U8P), cap + 1)
        if n < 0:
            self._rc(n, "stamps")
        return st[:n + 1], kinds[:n]

    def set_persistent(self, on):
        """The graph's form: True for one persistent launch of every layer (the default where
        the device holds it), False for the chain of six launches per layer. Returns the form in
        use afterwards."""
        r = lib().omega_gpu_decode_graph_set_persistent(self.h, int(on))
        if r < 0:
            self._rc(r, "set_persistent")
        return bool(r)

    def set_stage_stamps(self, on):
        lib().omega_gpu_decode_graph_set_stage_stamps(self.h, int(on))

    def stage_ns(self):
        """[layers][5] ns since the persistent launch started at which each layer's stages
        ended (input row, attention row, residual, route inputs, down rows), last token."""
        cap = self.layers * 5
        ns = np.zeros(cap, np.uint64)
        n = lib().omega_gpu_decode_graph_stage_ns(self.h, ns.ctypes.data_as(U64P), cap)
        if n < 0:
            self._rc(n, "stage_ns")
        return ns[:n].reshape(self.layers, 5)

    def kernel_ns(self):
        """Per-launch durations (ns) of the last stamped token, as the dispatch recorded them."""
        cap = DGRAPH_MAX_LAYERS * 16 + 16
        ns = np.zeros(cap, np.uint64)
        n = lib().omega_gpu_decode_graph_kernel_ns(self.h, ns.ctypes.data_as(U64P), cap)
        if n < 0:
            self._rc(n, "kernel_ns")
        return ns[:n]

    def set_flush_each(self, on):
        lib().omega_gpu_decode_graph_set_flush_each(self.h, int(on))

    def test_set_mutant(self, m):
        lib().omega_gpu_decode_graph_test_set_mutant(self.h, m)

    def free(self):
        if self.h:
            lib().omega_gpu_decode_graph_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


QWEN3_30B = dict(layers=48, hidden=2048, q_heads=32, kv_heads=4, head_dim=128, experts=128,
                 top_k=8, inter=768, vocab=151936, eps=1e-6, rope_theta=1e6)


def synth_tensor_id(layer, kind):
    """Tensor id of the shared counter-based generator for (layer, kind): kinds 0..3 are the
    q|k|v, o, gate|up and down FP8 projections, 8 the router; the embedding is id 1 and the
    lm_head id 2 (the CPU oracle's oref_model_synth uses the same ids)."""
    return 1000 + layer * 16 + kind


class SynthDecodeModel:
    """A random-init Qwen3-MoE model made resident the way OmegaModelUploader does it
    (qwen3_moe_omega.rs:1231-1598), with every tensor synthesised on the device by the library's
    generator instead of read from a checkpoint: FP8 projections N(0, sigma) block-quantised,
    router rows bf16 N(0, sigma), bf16 embedding and lm_head N(0, 0.02), norm weights 1.0; the
    router directories, the fused decode cache and the decode graph over them. The CPU oracle's
    oref_model_synth(seed, sigma, norm_sigma = 0) builds the same values."""

    def __init__(self, seed, max_pos, cfg=None, sigma=0.02):
        c = dict(QWEN3_30B if cfg is None else cfg)
        self.cfg = c
        L, H, E, HD = c["layers"], c["hidden"], c["experts"], c["head_dim"]
        qkv_n = (c["q_heads"] + 2 * c["kv_heads"]) * HD
        self.router = Router(L, E)
        self.cache = DecodeAttnCache(L, max_pos, c["rope_theta"])
        ones = np.ones(H, np.float32)
        self.layers = []
        for l in range(L):
            qkv = Fp8Tensor.synth(1, qkv_n, H, seed, synth_tensor_id(l, 0), sigma)
            o = Fp8Tensor.synth(1, H, c["q_heads"] * HD, seed, synth_tensor_id(l, 1), sigma)
            gu = Fp8Tensor.synth(E, 2 * c["inter"], H, seed, synth_tensor_id(l, 2), sigma)
            dn = Fp8Tensor.synth(E, H, c["inter"], seed, synth_tensor_id(l, 3), sigma)
            self.layers.append((qkv, o, gu, dn))
            self.router.set_layer(l, synth_bf16_host(seed, synth_tensor_id(l, 8), (E, H), sigma), ones)
            self.router.set_directory(l, np.array([gu.entry(e) for e in range(E)], np.uint64),
                                      np.array([dn.entry(e) for e in range(E)], np.uint64))
            self.cache.set_norms(l, np.ones(HD, np.float32), np.ones(HD, np.float32))
        self.lm = Bf16Tensor.synth(c["vocab"], H, seed, 2, 0.02)
        self.embed = Bf16Tensor.synth(c["vocab"], H, seed, 1, 0.02)
        self.graph = DecodeGraph(L, c["vocab"], c["eps"], self.router, self.cache, self.lm)
        for l, (qkv, o, gu, dn) in enumerate(self.layers):
            self.graph.set_layer(l, qkv, o, gu, dn, ones)
        self.graph.set_final_norm(ones)
        self.graph.set_embedding(self.embed)

    def free(self):
        if self.graph is None:
            return
        self.graph.free()
        for ts in self.layers:
            for t in ts:
                t.free()
        for t in (self.router, self.cache, self.lm, self.embed):
            t.free()
        self.graph = None


_hip = None


def hip():
    """libamdhip64 for the device buffers and events of the device-pointer entry points."""
    global _hip
    if _hip is None:
        h = C.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [C.POINTER(P), C.c_size_t]
        h.hipFree.argtypes = [P]
        h.hipMemcpy.argtypes = [P, P, C.c_size_t, C.c_int]
        h.hipMemsetAsync.argtypes = [P, C.c_int, C.c_size_t, P]
        h.hipEventCreate.argtypes = [C.POINTER(P)]
        h.hipEventRecord.argtypes = [P, P]
        h.hipEventSynchronize.argtypes = [P]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), P, P]
        h.hipEventDestroy.argtypes = [P]
        _hip = h
    return _hip


def reserve_serving(**bounds):
    """omega_gpu_reserve_serving (aien-omega-gpu/src/lib.rs:1129-1160) with the named bounds"""
    b = ServingBounds(**bounds)
    rc = lib().omega_gpu_reserve_serving(C.byref(b))
    if rc:
        raise OmegaGpuError(rc, _s(lib().omega_gpu_matmul_last_error()))


def serving_seal():
    lib().omega_gpu_serving_seal()


def serving_release():
    lib().omega_gpu_serving_release()


def alloc_stats():
    s = AllocStats()
    lib().omega_gpu_session_alloc_stats(C.byref(s))
    return {n: getattr(s, n) for n, _ in AllocStats._fields_}


class DeviceBuffer:
    """A device allocation (hipMalloc) with host copies; `.ptr` is the device address."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = P()
        rc = hip().hipMalloc(C.byref(p), C.c_size_t(max(self.nbytes, 1)))
        if rc != 0:
            raise OmegaGpuError(-4, f"hipMalloc({self.nbytes}) failed: {rc}")
        self.ptr = p

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        sync()
        assert hip().hipMemcpy(self.ptr, a.ctypes.data_as(P), C.c_size_t(a.nbytes), 1) == 0

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        sync()
        assert hip().hipMemcpy(out.ctypes.data_as(P), self.ptr, C.c_size_t(out.nbytes), 2) == 0
        return out

    def free(self):
        if self.ptr:
            sync()
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class StreamTimer:
    """HIP events on the library's stream: the GPU time between start() and stop()."""

    def __init__(self):
        self.a, self.b = P(), P()
        assert hip().hipEventCreate(C.byref(self.a)) == 0
        assert hip().hipEventCreate(C.byref(self.b)) == 0

    def start(self):
        assert hip().hipEventRecord(self.a, lib().omega_gpu_stream()) == 0

    def stop(self):
        assert hip().hipEventRecord(self.b, lib().omega_gpu_stream()) == 0

    def ms(self):
        assert hip().hipEventSynchronize(self.b) == 0
        v = C.c_float()
        assert hip().hipEventElapsedTime(C.byref(v), self.a, self.b) == 0
        return v.value


def kv_layout(num_blocks, block_size, layers, kv_heads, head_dim):
    """The aien-kv-cache bf16 page layout (crates/aien-kv-cache/src/lib.rs:247-292): element
    (block, layer, plane, token, head, dim) at block*BS + layer*LS + plane*PS + token*TS + head*HS
    + dim*2."""
    hs = head_dim * 2
    ts = kv_heads * hs
    ps = block_size * ts
    ls = 2 * ps
    bs = layers * ls
    return KvLayout(bs, ls, ps, ts, hs, num_blocks * bs, num_blocks, layers, block_size)


class BatchDecode:
    """The batched serving decode (omega_gpu_batch_decode_*) over a device KV pool."""

    def __init__(self, layers, vocab, max_seqs, max_blocks, max_pos, eps, rope_theta, router, lm_head,
                 embed, pool_ptr, layout, norm_topk=True):
        cfg = BatchDecodeConfig(layers, vocab, max_seqs, max_blocks, max_pos, eps, int(norm_topk),
                                rope_theta, router.as_raw(), lm_head.as_raw(), embed.as_raw(),
                                pool_ptr, layout)
        self.cfg = cfg
        self._keep = (router, lm_head, embed)
        h = P()
        self._rc(lib().omega_gpu_batch_decode_create(C.byref(cfg), C.byref(h)))
        self.h = h

    @staticmethod
    def _rc(rc):
        if rc:
            raise OmegaGpuError(rc, _s(lib().omega_gpu_session_last_error()))

    def set_layer(self, layer, qkv, o, gate_up, down, input_norm, q_norm, k_norm):
        args = [np.ascontiguousarray(a, dtype=np.float32) for a in (input_norm, q_norm, k_norm)]
        self._rc(lib().omega_gpu_batch_decode_set_layer(self.h, layer, qkv.as_raw(), o.as_raw(),
                                                        gate_up.as_raw(), down.as_raw(),
                                                        *[ptr(a) for a in args]))

    def set_final_norm(self, w):
        self._rc(lib().omega_gpu_batch_decode_set_final_norm(
            self.h, ptr(np.ascontiguousarray(w, dtype=np.float32))))

    def set_tables(self, tables):
        t = np.ascontiguousarray(tables, dtype=np.int32)
        self._rc(lib().omega_gpu_batch_decode_set_tables(self.h, t.shape[0], ptr(t)))

    def set_keep_logits(self, on):
        lib().omega_gpu_batch_decode_set_keep_logits(self.h, int(on))

    def set_eager(self, on):
        lib().omega_gpu_batch_decode_set_eager(self.h, int(on))

    def step(self, tokens, positions):
        tk = np.ascontiguousarray(tokens, dtype=np.uint32)
        ps = np.ascontiguousarray(positions, dtype=np.uint32)
        out = np.empty(tk.size, np.uint32)
        self._rc(lib().omega_gpu_batch_decode_step(self.h, tk.size, ptr(tk), ptr(ps), ptr(out)))
        return out

    def read(self, seqs, x=False, hidden=False, logits=False, routes=False):
        c = self.cfg
        xa = np.empty((seqs, 2048), np.float32) if x else None
        ha = np.empty((seqs, 2048), np.float32) if hidden else None
        la = np.empty((seqs, c.vocab), np.float32) if logits else None
        ra = np.empty((c.layers, seqs, 8), np.uint32) if routes else None
        self._rc(lib().omega_gpu_batch_decode_read(self.h, seqs, ptr(xa), ptr(ha), ptr(la), ptr(ra)))
        return xa, ha, la, ra

    def free(self):
        if getattr(self, "h", None):
            lib().omega_gpu_batch_decode_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def moe_batch(router, layer, gate_up, down, h, eps, norm_topk=True):
    """The batched MoE block (omega_gpu_moe_batch_f32): h [T][2048] -> (moe_out [T][2048] without
    the residual, ids [T][8], weights [T][8])."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    T = h.shape[0]
    out = np.empty((T, 2048), np.float32)
    ids = np.empty((T, 8), np.uint32)
    w = np.empty((T, 8), np.float32)
    rc = lib().omega_gpu_moe_batch_f32(router.as_raw(), layer, gate_up.as_raw(), down.as_raw(), T,
                                       ptr(h), eps, int(norm_topk), ptr(ids), ptr(w), ptr(out))
    if rc:
        raise OmegaGpuError(rc, _s(lib().omega_gpu_fp8gemm_last_error()))
    return out, ids, w


def synth_bf16_dev(buf, count, seed, tensor_id, sigma=1.0, offset_bytes=0):
    """Fill `count` bf16 values of the library's generator into a device buffer."""
    dst = P((buf.ptr.value or 0) + offset_bytes)
    rc = lib().omega_gpu_synth_bf16_dev(dst, count, seed, tensor_id, sigma)
    if rc:
        raise OmegaGpuError(rc, _s(lib().omega_gpu_bf16_last_error()))


def synth_bf16_host(seed, tensor_id, shape, sigma, one_plus=False):
    """bf16 N(0, sigma) values from the library's generator (the device generator's twin)."""
    out = np.empty(shape, dtype=np.uint16)
    lib().omega_gpu_synth_bf16_host(seed, tensor_id, out.size, sigma, int(one_plus), ptr(out))
    return out


def kind_name(kind):
    return _s(lib().omega_gpu_decode_graph_kind_name(kind))


def sync():
    rc = lib().omega_gpu_sync()
    if rc:
        raise OmegaGpuError(rc, _s(lib().omega_gpu_session_last_error()))
