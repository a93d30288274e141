"""ctypes binding of the CPU oracle (oracle/oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only
as the checker or as the timed CPU baseline. The product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_lib = None


class KvLayout(C.Structure):
    _fields_ = [
        ("block_stride_bytes", C.c_uint64),
        ("layer_stride_bytes", C.c_uint64),
        ("kv_plane_stride_bytes", C.c_uint64),
        ("token_stride_bytes", C.c_uint64),
        ("head_stride_bytes", C.c_uint64),
        ("pool_bytes", C.c_uint64),
        ("num_blocks", C.c_uint32),
        ("num_layers", C.c_uint32),
        ("block_size", C.c_uint32),
    ]


class Config(C.Structure):
    _fields_ = [
        ("layers", C.c_int),
        ("hidden", C.c_int),
        ("q_heads", C.c_int),
        ("kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("experts", C.c_int),
        ("top_k", C.c_int),
        ("inter", C.c_int),
        ("vocab", C.c_int),
        ("eps", C.c_float),
        ("rope_theta", C.c_double),
    ]


def build():
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        f32, f64, u8, u16, u32, u64, i32 = (C.c_float, C.c_double, C.c_uint8, C.c_uint16,
                                            C.c_uint32, C.c_uint64, C.c_int)
        sig = {
            "oref_bf16_to_f32": (f32, [u16]),
            "oref_f32_to_bf16": (u16, [f32]),
            "oref_kv_f32_to_bf16": (u16, [f32]),
            "oref_e4m3_to_f32": (f32, [u8]),
            "oref_f32_to_e4m3": (u8, [f32]),
            "oref_f32_to_e4m3_fast": (u8, [f32]),
            "oref_e4m3_rne_sat": (u8, [f32]),
            "oref_fq_e4m3_to_f32": (f32, [u8]),
            "oref_block_scale": (None, [f32, P, P]),
            "oref_quant_row": (None, [P, i32, P, P]),
            "oref_fake_quant_row": (None, [P, i32]),
            "oref_bf16_round_row": (None, [P, i32]),
            "oref_quantize_block128": (None, [P, i32]),
            "oref_prand": (f32, [u64, u64]),
            "oref_splitmix64": (u64, [u64]),
            "oref_synth_normal": (f32, [u64, u64, u64, f32]),
            "oref_synth_bf16": (None, [u64, u64, C.c_size_t, f32, i32, P]),
            "oref_synth_f32": (None, [u64, u64, C.c_size_t, f32, i32, P]),
            "oref_synth_fp8": (None, [u64, u64, i32, i32, i32, f32, P, P]),
            "oref_fp8_grouped": (None, [P, P, i32, i32, i32, i32, P, P, i32, P]),
            "oref_fp8_grouped_mt": (None, [P, P, i32, i32, i32, i32, P, P, i32, P, i32]),
            "oref_dequant_matvec": (None, [P, P, i32, i32, P, P]),
            "oref_bf16_gemv": (None, [P, i32, i32, P, P]),
            "oref_bf16_gemv_mt": (None, [P, i32, i32, P, P, i32]),
            "oref_argmax": (u32, [P, i32]),
            "oref_rmsnorm": (None, [P, P, i32, f32, P]),
            "oref_rmsnorm_per_head": (None, [P, P, f32, i32, i32, P]),
            "oref_rope_cos_sin": (None, [f64, i32, i32, P, P]),
            "oref_apply_rope": (None, [P, P, i32, i32, i32, i32, f64]),
            "oref_sdpa": (None, [P, P, P, i32, i32, i32, i32, P]),
            "oref_router_logits": (None, [P, P, i32, i32, P]),
            "oref_router_logits_f64": (None, [P, P, i32, i32, P]),
            "oref_moe_plan": (i32, [P, i32, i32, i32, P, P, P, P, P, P]),
            "oref_reduce_grouped": (None, [P, P, i32, i32, P, i32, P]),
            "oref_swiglu": (None, [P, i32, P]),
            "oref_route": (i32, [P, P, i32, i32, i32, P, f32, i32, P, P, P, P]),
            "oref_moe_forward": (None, [P, P, P, P, i32, i32, i32, i32, P, P, P, i32, P]),
            "oref_moe_block": (None, [P, P, P, P, i32, i32, i32, i32, P, P, P, i32, P]),
            "oref_kv_layout_bf16": (None, [u32, u32, u32, u32, u32, P]),
            "oref_kv_element_offset": (u64, [P, u32, u32, i32, u32, u32, u32]),
            "oref_kv_write_token": (None, [P, P, u32, u32, u32, i32, P, P]),
            "oref_kv_read_token": (None, [P, P, u32, u32, u32, i32, P, P]),
            "oref_paged_attention": (None, [P, P, P, P, i32, i32, i32, i32, i32, P]),
            "oref_fnv1a64": (u64, [P, C.c_size_t]),
            "oref_dattn_alloc": (P, [i32, i32, f64]),
            "oref_dattn_free": (None, [P]),
            "oref_dattn_set_norms": (None, [P, i32, P, P]),
            "oref_dattn_attend": (None, [P, i32, i32, P, f32, f32, P]),
            "oref_dattn_read_row": (None, [P, i32, i32, i32, P, P]),
            "oref_dattn_write_rows": (None, [P, i32, i32, i32, i32, P, P]),
            "oref_set_mutant": (None, [i32]),
            "oref_model_synth": (P, [P, u64, f32, f32, i32]),
            "oref_model_synth_layers": (P, [P, u64, f32, f32, i32, P]),
            "oref_model_free": (None, [P]),
            "oref_model_tensor": (P, [P, i32, i32, P]),
            "oref_model_embed": (P, [P]),
            "oref_model_lm_head": (P, [P]),
            "oref_model_final_norm": (P, [P]),
            "oref_engine_new": (P, [P, i32, i32, i32]),
            "oref_engine_free": (None, [P]),
            "oref_engine_step": (i32, [P, u32, P]),
            "oref_engine_logits": (None, [P, P, P]),
            "oref_engine_pos": (i32, [P]),
            "oref_engine_seek": (i32, [P, i32]),
            "oref_engine_kv": (P, [P]),
            "oref_engine_last_routes": (None, [P, P, P, P]),
            "oref_engine_last_x": (None, [P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be contiguous"
    return a.ctypes.data_as(C.c_void_p)


# --------------------------------------------------------------------------- helpers
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """RNE f32 -> bf16 bits (finite inputs), the rule of qwen3_moe.rs:486-493."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def e4m3_table() -> np.ndarray:
    L = lib()
    return np.array([L.oref_e4m3_to_f32(b) for b in range(256)], dtype=np.float32)


def synth_fp8(seed: int, tensor: int, experts: int, n: int, k: int, sigma: float = 0.02):
    w = np.empty((experts, n, k), dtype=np.uint8)
    s = np.empty((experts, n // 128, k // 128), dtype=np.uint16)
    lib().oref_synth_fp8(seed, tensor, experts, n, k, sigma, ptr(w), ptr(s))
    return w, s


def synth_bf16(seed: int, tensor: int, shape, sigma: float, one_plus: bool = False):
    out = np.empty(shape, dtype=np.uint16)
    lib().oref_synth_bf16(seed, tensor, out.size, sigma, int(one_plus), ptr(out))
    return out


def synth_f32(seed: int, tensor: int, shape, sigma: float, one_plus: bool = False):
    out = np.empty(shape, dtype=np.float32)
    lib().oref_synth_f32(seed, tensor, out.size, sigma, int(one_plus), ptr(out))
    return out


def fp8_grouped(w, s, ids, x, threads: int = 1):
    experts, n, k = w.shape
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    groups = ids.size
    x_rows = 1 if x.size == k else groups
    y = np.empty((groups, n), dtype=np.float32)
    lib().oref_fp8_grouped_mt(ptr(w), ptr(s), experts, n, k, groups, ptr(ids), ptr(x), x_rows,
                              ptr(y), threads)
    return y


def dequant_matvec(w, s, v):
    rows, cols = w.shape
    out = np.empty(rows, dtype=np.float32)
    lib().oref_dequant_matvec(ptr(np.ascontiguousarray(w)), ptr(np.ascontiguousarray(s)), rows,
                              cols, ptr(np.ascontiguousarray(v, dtype=np.float32)), ptr(out))
    return out


def bf16_gemv(w, x, threads: int = 1):
    n, k = w.shape
    y = np.empty(n, dtype=np.float32)
    lib().oref_bf16_gemv_mt(ptr(w), n, k, ptr(np.ascontiguousarray(x, dtype=np.float32)),
                            ptr(y), threads)
    return y


def argmax(logits) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().oref_argmax(ptr(logits), logits.size))


def rmsnorm(x, w, eps: float):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oref_rmsnorm(ptr(x), ptr(np.ascontiguousarray(w, dtype=np.float32)), x.size, eps,
                       ptr(out))
    return out


def rmsnorm_per_head(x, w, eps: float, heads: int, hd: int):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oref_rmsnorm_per_head(ptr(x), ptr(np.ascontiguousarray(w, dtype=np.float32)), eps,
                                heads, hd, ptr(out))
    return out


def rope_cos_sin(theta: float, hd: int, pos: int):
    c = np.empty(hd // 2, dtype=np.float32)
    s = np.empty(hd // 2, dtype=np.float32)
    lib().oref_rope_cos_sin(theta, hd, pos, ptr(c), ptr(s))
    return c, s


def apply_rope(q, k, pos: int, qh: int, kvh: int, hd: int, theta: float):
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    lib().oref_apply_rope(ptr(q), ptr(k), pos, qh, kvh, hd, theta)
    return q, k


def sdpa(q, K, V, qh: int, kvh: int, hd: int):
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    ctx = K.shape[0] if K.ndim > 1 else K.size // (kvh * hd)
    out = np.empty(qh * hd, dtype=np.float32)
    lib().oref_sdpa(ptr(np.ascontiguousarray(q, dtype=np.float32)), ptr(K), ptr(V), ctx, qh, kvh,
                    hd, ptr(out))
    return out


def router_logits(gate_bf16, post, refined: bool = False):
    experts, hidden = gate_bf16.shape
    out = np.empty(experts, dtype=np.float32)
    fn = lib().oref_router_logits_f64 if refined else lib().oref_router_logits
    fn(ptr(np.ascontiguousarray(gate_bf16)), ptr(np.ascontiguousarray(post, dtype=np.float32)),
       experts, hidden, ptr(out))
    return out


def moe_plan(logits, tokens: int, experts: int, top_k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    a = tokens * top_k
    te = np.zeros(a, dtype=np.uint32)
    tw = np.zeros(a, dtype=np.float32)
    off = np.zeros(experts + 1, dtype=np.uint32)
    g2a = np.zeros(a, dtype=np.uint32)
    a2g = np.zeros(a, dtype=np.uint32)
    gt = np.zeros(a, dtype=np.uint32)
    rc = lib().oref_moe_plan(ptr(logits), tokens, experts, top_k, ptr(te), ptr(tw), ptr(off),
                             ptr(g2a), ptr(a2g), ptr(gt))
    if rc != 0:
        raise ValueError(f"moe plan refused: rc {rc}")
    return dict(topk_experts=te, topk_weights=tw, expert_offsets=off, grouped_to_assignment=g2a,
                assignment_to_grouped=a2g, grouped_token_ids=gt)


def route(gate_bf16, norm_w, x, eps: float, top_k: int = 8, refined: bool = True):
    experts, hidden = gate_bf16.shape
    ids = np.zeros(top_k, dtype=np.uint32)
    w = np.zeros(top_k, dtype=np.float32)
    post = np.zeros(hidden, dtype=np.float32)
    logits = np.zeros(experts, dtype=np.float32)
    rc = lib().oref_route(ptr(np.ascontiguousarray(gate_bf16)),
                          ptr(np.ascontiguousarray(norm_w, dtype=np.float32)), experts, hidden,
                          top_k, ptr(np.ascontiguousarray(x, dtype=np.float32)), eps, int(refined),
                          ptr(ids), ptr(w), ptr(post), ptr(logits))
    if rc != 0:
        raise ValueError(f"route refused: rc {rc}")
    return ids, w, post, logits


def moe_block(gu_w, gu_s, dn_w, dn_s, ids, weights, post, w8a8: bool = False):
    """The engine's FP8 MoE arm for one token (oref_moe_block): moe_out without the residual."""
    experts, n2, h = gu_w.shape
    out = np.zeros(h, dtype=np.float32)
    lib().oref_moe_block(ptr(gu_w), ptr(gu_s), ptr(dn_w), ptr(dn_s), experts, h, n2 // 2, len(ids),
                         ptr(np.ascontiguousarray(ids, dtype=np.uint32)),
                         ptr(np.ascontiguousarray(weights, dtype=np.float32)),
                         ptr(np.ascontiguousarray(post, dtype=np.float32)), int(w8a8), ptr(out))
    return out


def swiglu(gu, i: int):
    act = np.empty(i, dtype=np.float32)
    lib().oref_swiglu(ptr(np.ascontiguousarray(gu, dtype=np.float32)), i, ptr(act))
    return act


def kv_layout(num_blocks, block_size, layers, kv_heads, head_dim) -> KvLayout:
    lay = KvLayout()
    lib().oref_kv_layout_bf16(num_blocks, block_size, layers, kv_heads, head_dim, C.byref(lay))
    return lay


def fnv1a64(b: bytes | np.ndarray) -> int:
    arr = np.frombuffer(bytes(b), dtype=np.uint8) if isinstance(b, (bytes, bytearray)) else \
        np.ascontiguousarray(b).view(np.uint8).reshape(-1)
    return int(lib().oref_fnv1a64(ptr(arr), arr.size))


# ------------------------------------------------------------------ KV park / restore payload
class PoolBlockGeometry:
    """One HostPagedPoolV1 block for bf16 elements (qwen3_moe_omega_kvio.rs:42-100): per block
    [layer][K plane | V plane][token][kv head][dim]."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, block_size: int):
        self.layers, self.kv_heads, self.head_dim, self.block_size = layers, kv_heads, head_dim, block_size

    @property
    def head_stride(self):
        return self.head_dim * 2

    @property
    def token_stride(self):
        return self.kv_heads * self.head_stride

    @property
    def kv_plane_stride(self):
        return self.block_size * self.token_stride

    @property
    def layer_stride(self):
        return 2 * self.kv_plane_stride

    @property
    def block_stride(self):
        return self.layers * self.layer_stride

    def payload_len(self, length: int) -> int:
        return -(-length // self.block_size) * self.block_stride

    def row_offset(self, rel: int, layer: int, value: bool, head: int) -> int:
        return ((rel // self.block_size) * self.block_stride + layer * self.layer_stride
                + int(value) * self.kv_plane_stride + (rel % self.block_size) * self.token_stride
                + head * self.head_stride)

    def check(self, start: int, length: int):
        if min(self.layers, self.kv_heads, self.head_dim, self.block_size) == 0:
            raise ValueError("kv export geometry has a zero dimension")
        if length == 0:
            raise ValueError("kv export of zero positions")
        if start % self.block_size:
            raise ValueError(f"kv export start {start} is not a multiple of the block size")


def kv_rows_to_blocks(g: PoolBlockGeometry, start: int, length: int, read_row) -> np.ndarray:
    """rows_to_blocks (qwen3_moe_omega_kvio.rs:102-122): read_row(layer, head, pos) -> (k, v) of
    head_dim uint16 each, placed little-endian at row_offset; the rest of the payload is zero."""
    g.check(start, length)
    out = np.zeros(g.payload_len(length), np.uint8)
    for layer in range(g.layers):
        for head in range(g.kv_heads):
            for rel in range(length):
                k, v = read_row(layer, head, start + rel)
                for value, row in ((False, k), (True, v)):
                    at = g.row_offset(rel, layer, value, head)
                    out[at:at + 2 * g.head_dim] = np.asarray(row, "<u2").view(np.uint8)
    return out


def kv_check_payload(g: PoolBlockGeometry, length: int, payload) -> None:
    """check_payload (qwen3_moe_omega_kvio.rs:162-186): exact size, zero padding rows."""
    b = np.asarray(payload, np.uint8)
    if b.size != g.payload_len(length):
        raise ValueError(f"kv payload of {b.size} bytes, {length} positions need {g.payload_len(length)}")
    tail = length % g.block_size
    if tail:
        last = length - tail
        for layer in range(g.layers):
            for value in (False, True):
                lo = g.row_offset(last + tail, layer, value, 0)
                hi = g.row_offset(last, layer, value, 0) + g.kv_plane_stride
                if b[lo:hi].any():
                    raise ValueError(f"kv payload: padding rows past position {length} of layer {layer} are not zero")


def kv_blocks_to_rows(g: PoolBlockGeometry, start: int, length: int, payload, write_rows) -> None:
    """blocks_to_rows (qwen3_moe_omega_kvio.rs:124-160): refuses a damaged payload before any
    write, then write_rows(layer, head, k_rows, v_rows) with [length][head_dim] uint16 each."""
    g.check(start, length)
    kv_check_payload(g, length, payload)
    b = np.asarray(payload, np.uint8)
    for layer in range(g.layers):
        for head in range(g.kv_heads):
            k = np.empty((length, g.head_dim), np.uint16)
            v = np.empty((length, g.head_dim), np.uint16)
            for rel in range(length):
                for value, dst in ((False, k), (True, v)):
                    at = g.row_offset(rel, layer, value, head)
                    dst[rel] = b[at:at + 2 * g.head_dim].view("<u2")
            write_rows(layer, head, k, v)


def kv_zero_padding(g: PoolBlockGeometry, length: int, payload: np.ndarray) -> None:
    """zero_padding (qwen3_moe_omega_kvio.rs:188-202), in place"""
    tail = length % g.block_size
    if not tail:
        return
    last = length - tail
    for layer in range(g.layers):
        for value in (False, True):
            payload[g.row_offset(last + tail, layer, value, 0):
                    g.row_offset(last, layer, value, 0) + g.kv_plane_stride] = 0


class Dattn:
    """The fused decode-attention cache oracle (bf16 rows, f64 attention)."""

    def __init__(self, layers: int, max_pos: int, theta: float):
        self.h = lib().oref_dattn_alloc(layers, max_pos, theta)

    def set_norms(self, layer, qn, kn):
        lib().oref_dattn_set_norms(self.h, layer, ptr(np.ascontiguousarray(qn, dtype=np.float32)),
                                   ptr(np.ascontiguousarray(kn, dtype=np.float32)))

    def attend(self, layer, pos, qkv, eps, out_scale=1.0):
        out = np.empty(4096, dtype=np.float32)
        lib().oref_dattn_attend(self.h, layer, pos,
                                ptr(np.ascontiguousarray(qkv, dtype=np.float32)), eps, out_scale,
                                ptr(out))
        return out

    def read_row(self, layer, head, pos):
        k = np.empty(128, dtype=np.uint16)
        v = np.empty(128, dtype=np.uint16)
        lib().oref_dattn_read_row(self.h, layer, head, pos, ptr(k), ptr(v))
        return k, v

    def write_rows(self, layer, head, pos, k, v):
        k = np.ascontiguousarray(k, dtype=np.uint16).reshape(-1, 128)
        v = np.ascontiguousarray(v, dtype=np.uint16).reshape(-1, 128)
        lib().oref_dattn_write_rows(self.h, layer, head, pos, k.shape[0], ptr(k), ptr(v))

    def __del__(self):
        if getattr(self, "h", None):
            lib().oref_dattn_free(self.h)
            self.h = None


def quant_row(x):
    """oref_quant_row (fake_quant.rs:85-104): e4m3 codes and power-of-two block scales of one row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.uint8)
    s = np.empty(x.size // 128, dtype=np.float32)
    lib().oref_quant_row(ptr(x), x.size, ptr(q), ptr(s))
    return q, s


def fake_quant(x):
    """oref_fake_quant_row (fake_quant.rs:107-115): quantise then dequantise one row."""
    x = np.array(x, dtype=np.float32, copy=True)
    lib().oref_fake_quant_row(ptr(x), x.size)
    return x


def bf16_round(x):
    """oref_bf16_round_row (fake_quant.rs bf16_round_row): each value rounded to bf16 (RNE), kept
    as f32."""
    x = np.array(x, dtype=np.float32, copy=True)
    lib().oref_bf16_round_row(ptr(x), x.size)
    return x


def prefill_w8a8(model, tokens, pos0: int = 0, cache=None, max_pos: int = 4096, forced=None,
                 forced_qkv=None, forced_att=None, w8a8: bool = True):
    """The whole-prompt prefill's arithmetic (qwen3_moe_omega_prefill.rs:483-760, W8A8: every
    GEMM input row fake-quantised per 128-block, the SwiGLU act rounded to bf16 first), layer by
    layer over the prompt: input RMSNorm, q|k|v, the decode attention of each token at its
    position (oref_dattn), o, residual, post RMSNorm, router logits (sequential f32), the routing
    plan (oref_moe_plan), the W8A8 MoE block (oref_moe_block) and the residual. Returns the last
    token's final-normed hidden row and per layer the residual rows after attention and after
    the MoE, the router logits and the routed ids. `forced` (per layer the [T][hidden] rows to
    use as that layer's input instead of the oracle's own, layer 0 included) checks one layer at
    a time on another implementation's inputs; `forced_qkv` (per layer [T][5120]) gives the rows
    the attention takes (its K / V rows are bf16-rounded, so an f32 difference of the projection
    flips one now and then), and `forced_att` (per layer [T][4096]) replaces the
    attention rows that enter the o projection (the W8A8 quantiser maps an f32 rounding difference
    of its input to a whole e4m3 step now and then), while the oracle's own attention rows are
    still returned for comparison. With w8a8 False every quantiser is the identity (the OFF
    path's f32 activations)."""
    c = model.cfg
    eps = c.eps
    fq = fake_quant if w8a8 else (lambda v: np.asarray(v, dtype=np.float32))
    if cache is None:
        cache = Dattn(c.layers, max_pos, c.rope_theta)
        for l in range(c.layers):
            cache.set_norms(l, model.tensor(l, 7), model.tensor(l, 8))
    emb = model.embed()
    x = np.stack([bf16_to_f32(emb[t]) for t in tokens]).astype(np.float32)
    T = len(tokens)
    out = dict(x_mid=[], x_out=[], logits=[], ids=[], qkv=[], att=[])
    for l in range(c.layers):
        if forced is not None:
            x = np.array(forced[l], dtype=np.float32, copy=True)
        qw, qs = model.tensor(l, 0)
        ow, os_ = model.tensor(l, 1)
        gw, gs = model.tensor(l, 2)
        dw, ds = model.tensor(l, 3)
        gate, in_norm, post_norm = model.tensor(l, 4), model.tensor(l, 5), model.tensor(l, 6)
        qkvs, atts = [], []
        for t in range(T):
            xn = fq(rmsnorm(x[t], in_norm, eps))
            qkv = dequant_matvec(qw[0], qs[0], xn)
            q_in = qkv if forced_qkv is None else np.asarray(forced_qkv[l][t], dtype=np.float32)
            att = cache.attend(l, pos0 + t, q_in, eps)
            qkvs.append(qkv)
            atts.append(att)
            a_in = att if forced_att is None else np.asarray(forced_att[l][t], dtype=np.float32)
            x[t] = x[t] + dequant_matvec(ow[0], os_[0], fq(a_in))
        out["qkv"].append(np.stack(qkvs))
        out["att"].append(np.stack(atts))
        out["x_mid"].append(x.copy())
        posts = np.stack([rmsnorm(x[t], post_norm, eps) for t in range(T)])
        logits = np.stack([router_logits(gate, posts[t], refined=False) for t in range(T)])
        plan = moe_plan(logits, T, c.experts, c.top_k)
        ids = plan["topk_experts"].reshape(T, c.top_k)
        wts = plan["topk_weights"].reshape(T, c.top_k)
        for t in range(T):
            x[t] = x[t] + moe_block(gw, gs, dw, ds, ids[t], wts[t], posts[t], w8a8=w8a8)
        out["x_out"].append(x.copy())
        out["logits"].append(logits)
        out["ids"].append(ids.copy())
    return rmsnorm(x[-1], model.final_norm(), eps), out


def paged_step(model, pool, lay, table, pos: int, token: int, threads: int = 1):
    """One token of one sequence through every layer with a paged KV pool as the KV store: the
    engine step (oref_engine_step, qwen3_moe_omega.rs:4096-4345) on the HostPoolKv arm
    (qwen3_moe_omega.rs:2925-2941): the token's bf16 K/V row is written at page table[pos / 16],
    slot pos % 16 (write_token_kv, aien-kv-cache/src/lib.rs:586-622), then paged attention over
    positions 0..=pos (gather_layer_kv then the f64 SDPA). pool (the aien-kv-cache bytes, uint8)
    is updated in place. Returns (final-normed hidden, routed ids [layers][top_k], the smallest
    gap between consecutive ranks of each layer's top top_k + 1 router logits [layers])."""
    c = model.cfg
    qh, kvh, hd, eps = c.q_heads, c.kv_heads, c.head_dim, c.eps
    table = np.ascontiguousarray(table, dtype=np.int32)
    x = bf16_to_f32(model.embed()[token % c.vocab]).astype(np.float32)
    routes = np.zeros((c.layers, c.top_k), np.uint32)
    gaps = np.zeros(c.layers, np.float32)
    for l in range(c.layers):
        xn = rmsnorm(x, model.tensor(l, 5), eps)
        w, s = model.tensor(l, 0)
        qkv = fp8_grouped(w, s, [0], xn, threads)[0]
        q = rmsnorm_per_head(qkv[:qh * hd], model.tensor(l, 7), eps, qh, hd)
        k = rmsnorm_per_head(qkv[qh * hd:(qh + kvh) * hd], model.tensor(l, 8), eps, kvh, hd)
        v = np.ascontiguousarray(qkv[(qh + kvh) * hd:])
        q, k = apply_rope(q, k, pos, qh, kvh, hd, c.rope_theta)
        lib().oref_kv_write_token(ptr(pool), C.byref(lay), int(table[pos // lay.block_size]), l,
                                  pos % lay.block_size, kvh * hd, ptr(k), ptr(v))
        att = np.empty(qh * hd, np.float32)
        lib().oref_paged_attention(ptr(q), ptr(pool), C.byref(lay), ptr(table), pos + 1, l, qh, kvh,
                                   hd, ptr(att))
        w, s = model.tensor(l, 1)
        x = x + fp8_grouped(w, s, [0], att, threads)[0]
        ids, wts, post, rl = route(model.tensor(l, 4), model.tensor(l, 6), x, eps, c.top_k)
        routes[l] = ids
        top = np.sort(rl)[::-1][:c.top_k + 1]
        gaps[l] = float(np.min(top[:-1] - top[1:]))
        gw, gs = model.tensor(l, 2)
        dw, ds = model.tensor(l, 3)
        x = x + moe_block(gw, gs, dw, ds, ids, wts, post)
    return rmsnorm(x, model.final_norm(), eps), routes, gaps


class Model:
    """Synthetic random-init model and the whole-step engine of the oracle."""

    def __init__(self, cfg: dict, seed: int, sigma: float = 0.02, norm_sigma: float = 0.0,
                 threads: int = 1, layer_ids=None):
        """layer_ids: hold only those layers of the model cfg describes (cfg["layers"] is the
        full model's count; layer i of this object is its layer layer_ids[i])."""
        cfg = dict(cfg)
        if layer_ids is not None:
            ids = np.ascontiguousarray(layer_ids, dtype=np.int32)
            if ids.size == 0 or ids.min() < 0 or ids.max() >= cfg["layers"]:
                raise ValueError(f"layer_ids {list(ids)} outside 0..{cfg['layers'] - 1}")
            cfg["layers"] = int(ids.size)
        self.cfg = Config(**cfg)
        if layer_ids is None:
            self.h = lib().oref_model_synth(C.byref(self.cfg), seed, sigma, norm_sigma, threads)
        else:
            self.h = lib().oref_model_synth_layers(C.byref(self.cfg), seed, sigma, norm_sigma,
                                                   threads, ptr(ids))

    def tensor(self, layer: int, kind: int):
        """kind 0..3: (w, s) of qkv, o, gate_up, down; 4: router bf16; 5..8: norms."""
        c = self.cfg
        hd, h = c.head_dim, c.hidden
        sp = C.c_void_p()
        p = lib().oref_model_tensor(self.h, layer, kind, C.byref(sp))
        qkv_n = (c.q_heads + 2 * c.kv_heads) * hd
        shapes = {0: (1, qkv_n, h), 1: (1, h, c.q_heads * hd), 2: (c.experts, 2 * c.inter, h),
                  3: (c.experts, h, c.inter)}
        if kind in shapes:
            e, n, k = shapes[kind]
            w = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(e, n, k))
            s = np.ctypeslib.as_array(C.cast(sp, C.POINTER(C.c_uint16)),
                                      shape=(e, n // 128, k // 128))
            return w, s
        if kind == 4:
            return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(c.experts, h))
        n = {5: h, 6: h, 7: hd, 8: hd}[kind]
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n,))

    def embed(self):
        c = self.cfg
        p = lib().oref_model_embed(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(c.vocab, c.hidden))

    def lm_head(self):
        c = self.cfg
        p = lib().oref_model_lm_head(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(c.vocab, c.hidden))

    def final_norm(self):
        p = lib().oref_model_final_norm(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(self.cfg.hidden,))

    def __del__(self):
        if getattr(self, "h", None):
            lib().oref_model_free(self.h)
            self.h = None


class Engine:
    def __init__(self, model: Model, max_pos: int, refined_router: bool = True,
                 threads: int = 1):
        self.model = model
        self.h = lib().oref_engine_new(model.h, max_pos, int(refined_router), threads)

    def step(self, token: int) -> np.ndarray:
        out = np.empty(self.model.cfg.hidden, dtype=np.float32)
        rc = lib().oref_engine_step(self.h, token, ptr(out))
        if rc != 0:
            raise RuntimeError(f"oracle step failed: {rc}")
        return out

    def logits(self, hidden) -> np.ndarray:
        out = np.empty(self.model.cfg.vocab, dtype=np.float32)
        lib().oref_engine_logits(self.h, ptr(np.ascontiguousarray(hidden, dtype=np.float32)),
                                 ptr(out))
        return out

    def last_routes(self):
        c = self.model.cfg
        ids = np.empty((c.layers, c.top_k), dtype=np.uint32)
        w = np.empty((c.layers, c.top_k), dtype=np.float32)
        m = np.empty(c.layers, dtype=np.float32)
        lib().oref_engine_last_routes(self.h, ptr(ids), ptr(w), ptr(m))
        return ids, w, m

    def last_x(self):
        x = np.empty(self.model.cfg.hidden, dtype=np.float32)
        lib().oref_engine_last_x(self.h, ptr(x))
        return x

    def write_kv_rows(self, layer: int, head: int, pos0: int, k, v):
        """Cache rows pos0 .. pos0 + len(k) - 1 of (layer, kv head): [n][head_dim] bf16 K and V."""
        k = np.ascontiguousarray(k, dtype=np.uint16).reshape(-1, self.model.cfg.head_dim)
        v = np.ascontiguousarray(v, dtype=np.uint16).reshape(-1, self.model.cfg.head_dim)
        lib().oref_dattn_write_rows(lib().oref_engine_kv(self.h), layer, head, pos0, k.shape[0], ptr(k), ptr(v))

    def seek(self, pos: int):
        """The next step runs at position pos over cache rows 0 .. pos - 1 as they stand
        (oref_engine_seek)."""
        if lib().oref_engine_seek(self.h, pos) != 0:
            raise ValueError(f"seek to {pos} past the cache")

    def fill_random(self, pos: int, seed: int = 0):
        """Benchmark support: seeded bf16 N(0, 1) K/V rows at positions 0 .. pos - 1 of every layer,
        then seek(pos)."""
        c = self.model.cfg
        rng = np.random.default_rng(seed)
        for layer in range(c.layers):
            for head in range(c.kv_heads):
                k = f32_to_bf16(rng.standard_normal((pos, c.head_dim)).astype(np.float32))
                v = f32_to_bf16(rng.standard_normal((pos, c.head_dim)).astype(np.float32))
                self.write_kv_rows(layer, head, 0, k, v)
        self.seek(pos)

    def __del__(self):
        if getattr(self, "h", None):
            lib().oref_engine_free(self.h)
            self.h = None
