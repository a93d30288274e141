"""Whole-prompt prefill over libomega_gpu's omega_gpu_pf_* / omega_gpu_prefill_attn entries.

Mirrors crates/aien-omega-pf (the safe wrappers: PfMem, OmegaPfDevice, OmegaPrefillAttention,
build_tiles, pack_router) and the driver WholePromptPrefill (crates/aien-inference-abi/src/
qwen3_moe_omega_prefill.rs:483-760) in its device-host form (qwen3_moe_omega_prefill/devhost.rs:
router logits and the MoE combine on the chip). The host steps stay on the host as in the
reference: the RMSNorms (f64 sum of squares), the residual adds, the routing plan
(MoeBatchPlan::from_logits, moe_plan.rs:86-171) and the expert sort.

The whole prompt goes through every layer with a fixed launch count per layer: quantise x, the
q|k|v GEMM, the prefill attention, quantise the attention rows, the o GEMM, the router logits,
quantise the post-norm rows, the gate|up GEMM with the SwiGLU epilogue (rows gathered by token),
quantise the act rows (bf16), the down GEMM and the combine.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import OmegaGpuError, _s, lib

PLAIN, SWIGLU_NAT = 0, 2
IN_F32, IN_BF16 = 0, 1
TILE_BYTES = 32
MAX_TILES = 65535
BLOCK = 128

TILE_DTYPE = np.dtype([("w_va", "<u8"), ("s_va", "<u8"), ("row0", "<u4"), ("cnt", "<u4"), ("pad", "<u8")])


class OmegaGpuMem(C.Structure):
    _fields_ = [("handle_index", C.c_uint32), ("handle_generation", C.c_uint32), ("kind", C.c_uint32),
                ("cpu", C.c_void_p), ("va", C.c_uint64), ("size", C.c_uint64)]


class PrefillAttnInfo(C.Structure):
    _fields_ = [("layer", C.c_uint32), ("pos0", C.c_uint32), ("m", C.c_uint32), ("chunks", C.c_uint32),
                ("grid_x", C.c_uint32), ("grid_y", C.c_uint32), ("threads", C.c_uint32),
                ("splits", C.c_uint32), ("per_split", C.c_uint32), ("elapsed_ns", C.c_uint64),
                ("call_ns", C.c_uint64), ("kernel_cache_hit", C.c_int32)]


def _pf_check(rc, what):
    if rc != 0:
        L = lib()
        raise OmegaGpuError(rc, f"{what}: {_s(L.omega_gpu_pf_rc_name(rc))}: {_s(L.omega_gpu_session_last_error())}")


def _attn_check(rc, what):
    if rc != 0:
        L = lib()
        raise OmegaGpuError(rc, f"{what}: {_s(L.omega_gpu_decode_attn_rc_name(rc))}: "
                                f"{_s(L.omega_gpu_decode_attn_last_error())}")


class PfMem:
    """A session buffer (aien-omega-pf/src/lib.rs:610-693): device-private, or host-visible with a
    CPU view (`host` gives it as a numpy array of the requested dtype)."""

    def __init__(self, nbytes, host=False):
        if nbytes <= 0:
            raise OmegaGpuError(-1, "pf alloc of 0 bytes")
        self.mem = OmegaGpuMem()
        fn = lib().omega_gpu_pf_alloc_host if host else lib().omega_gpu_pf_alloc_dev
        _pf_check(fn(nbytes, C.addressof(self.mem)), "pf alloc")
        if self.mem.va == 0 or self.mem.size < nbytes or (host and not self.mem.cpu):
            self.free()
            raise OmegaGpuError(-1, f"pf alloc of {nbytes} bytes returned no usable view")
        self.nbytes, self.is_host = nbytes, host

    @property
    def va(self):
        return self.mem.va

    def host(self, dtype=np.uint8):
        if not self.is_host:
            raise OmegaGpuError(-1, "device-private buffer has no CPU view")
        buf = (C.c_uint8 * self.nbytes).from_address(self.mem.cpu)
        return np.frombuffer(buf, dtype=np.uint8).view(dtype)

    def free(self):
        if self.mem.va:
            lib().omega_gpu_pf_free(C.addressof(self.mem))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ the device calls
def _va(p):
    """a device address as an integer (ints, ctypes pointers and buffers with .ptr / .va)"""
    if p is None:
        return 0
    if isinstance(p, int):
        return p
    if isinstance(p, C.c_void_p):
        return p.value or 0
    return _va(getattr(p, "va", None) if hasattr(p, "va") else p.ptr)


def quant(k, in_type, rows, x_va, q_va, s_va):
    """omega_gpu_pf_quant: chip ns"""
    ns = C.c_uint64()
    _pf_check(lib().omega_gpu_pf_quant(k, in_type, rows, _va(x_va), _va(q_va), _va(s_va), C.addressof(ns)),
              "pf quant")
    return ns.value


def qgemm_bm():
    return int(lib().omega_gpu_pf_qgemm_bm())


def qgemm(n, k, layout, tiles_va, ntiles, rowidx_va, xq_va, xs_va, y_va):
    ns = C.c_uint64()
    _pf_check(lib().omega_gpu_pf_qgemm(n, k, layout, _va(tiles_va), ntiles, _va(rowidx_va), _va(xq_va), _va(xs_va),
                                       _va(y_va), C.addressof(ns)), "pf qgemm")
    return ns.value


def build_tiles(bm, w_va, s_va, counts):
    """aien-omega-pf/src/lib.rs:122-160: experts in order, tiles of up to bm rows, row0 counting
    over all experts."""
    tiles = []
    row = 0
    for e, c in enumerate(counts):
        r = 0
        while r < c:
            cnt = min(c - r, bm)
            tiles.append((w_va[e], s_va[e], row + r, cnt, 0))
            r += cnt
        row += c
    if len(tiles) > MAX_TILES:
        raise OmegaGpuError(-1, f"pf tiles: {len(tiles)} tiles > {MAX_TILES}")
    return np.array(tiles, dtype=TILE_DTYPE)


def tiles_va_c(w_va, s_va, counts):
    """The C tile builder (omega_gpu_pf_qgemm_tiles_va)."""
    e = len(counts)
    w = np.ascontiguousarray(w_va, np.uint64)
    s = np.ascontiguousarray(s_va, np.uint64)
    c = np.ascontiguousarray(counts, np.uint32)
    tab = np.zeros(MAX_TILES, TILE_DTYPE)
    n = lib().omega_gpu_pf_qgemm_tiles_va(e, w.ctypes.data, s.ctypes.data, c.ctypes.data, tab.ctypes.data,
                                          MAX_TILES)
    return tab[:n]


def router_rows():
    return int(lib().omega_gpu_pf_router_rows())


def router_packed_len(e, k):
    return (k // 4 + 1) * e * 4


def pack_router(w):
    """omega_gpu_pf_router_pack: f32 [e][k] -> the packed layout wq[g][ex][q] = w[ex][4 g + q]
    plus one zero pad group."""
    e, k = w.shape
    w = np.ascontiguousarray(w, np.float32)
    wq = np.full(router_packed_len(e, k), np.nan, np.float32)
    lib().omega_gpu_pf_router_pack(e, k, w.ctypes.data, wq.ctypes.data)
    return wq


def router_logits(k, e, rows, x_va, wq_va, logits_va):
    ns = C.c_uint64()
    _pf_check(lib().omega_gpu_pf_router_logits(k, e, rows, _va(x_va), _va(wq_va), _va(logits_va), C.addressof(ns)),
              "pf router logits")
    return ns.value


def moe_combine(h, top_k, rows, down_va, inv_va, wt_va, out_va):
    ns = C.c_uint64()
    _pf_check(lib().omega_gpu_pf_moe_combine(h, top_k, rows, _va(down_va), _va(inv_va), _va(wt_va), _va(out_va),
                                             C.addressof(ns)), "pf moe combine")
    return ns.value


def residual_norm(k, rows, x_va, add_va, w_va, eps, out_va):
    """omega_gpu_pf_residual_norm: x += add (add_va 0: no add), out = rmsnorm(x) * w; chip ns"""
    ns = C.c_uint64()
    _pf_check(lib().omega_gpu_pf_residual_norm(k, rows, _va(x_va), _va(add_va), _va(w_va), float(eps), _va(out_va),
                                               C.addressof(ns)), "pf residual norm")
    return ns.value


def copy_va(dst_va, src_va, nbytes):
    _pf_check(lib().omega_gpu_pf_copy_va(_va(dst_va), _va(src_va), nbytes), "pf copy")


def stats():
    ns, n = C.c_uint64(), C.c_uint64()
    lib().omega_gpu_pf_stats(C.addressof(ns), C.addressof(n))
    return ns.value, n.value


def stats_reset():
    lib().omega_gpu_pf_stats_reset()


class PrefillAttention:
    """aien-omega-pf/src/lib.rs:978-1100 over a DecodeAttnCache: the host and device entries."""

    def __init__(self, cache):
        self.cache = cache

    def attend(self, layer, pos0, m, qkv, eps, out_scale):
        qkv = np.ascontiguousarray(qkv, np.float32).reshape(-1)
        if qkv.size != m * 5120:
            raise OmegaGpuError(-1, f"prefill attn: qkv {qkv.size} words, want {m * 5120}")
        out = np.empty(m * 4096, np.float32)
        info = PrefillAttnInfo()
        _attn_check(lib().omega_gpu_prefill_attn(self.cache.as_raw(), layer, pos0, m, qkv.ctypes.data, eps,
                                                 out_scale, out.ctypes.data, C.addressof(info)), "prefill attn")
        return out.reshape(m, 4096), info

    def attend_dev(self, layer, pos0, m, qkv_va, eps, out_scale, out_va):
        info = PrefillAttnInfo()
        _attn_check(lib().omega_gpu_prefill_attn_dev(self.cache.as_raw(), layer, pos0, m, _va(qkv_va), eps, out_scale,
                                                     _va(out_va), C.addressof(info)), "prefill attn dev")
        return info


# ------------------------------------------------------------------ host steps
def rmsnorm_rows(x, w, eps):
    """tensor.rs:94-110 per row: f64 sum of squares, scale (1 / sqrt(mean + eps)) as f32,
    out = x * scale * w in f32."""
    x = np.asarray(x, np.float32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1)
    scale = (1.0 / np.sqrt(ss / x.shape[-1] + float(eps))).astype(np.float32)
    return (x * scale[..., None]) * np.asarray(w, np.float32)


def moe_plan(logits, tokens, experts, top_k):
    """MoeBatchPlan::from_logits (moe_plan.rs:86-171) in the library (omega_gpu_pf_moe_plan): per
    token the top_k experts by total order (ties to the lower id), weights exp(l - max) / sum over
    the selected in f32, then the stable counting sort of the (token, slot) assignments by
    expert. Returns (ids [t][k], weights [t][k], counts [e], grouped_token [t*k],
    assignment_to_grouped [t*k])."""
    lg = np.ascontiguousarray(np.asarray(logits, np.float32).reshape(tokens, experts))
    ids = np.empty((tokens, top_k), np.uint32)
    wts = np.empty((tokens, top_k), np.float32)
    counts = np.empty(experts, np.uint32)
    grouped_token = np.empty(tokens * top_k, np.uint32)
    a2g = np.empty(tokens * top_k, np.uint32)
    _pf_check(lib().omega_gpu_pf_moe_plan(tokens, experts, top_k, lg.ctypes.data, ids.ctypes.data,
                                          wts.ctypes.data, counts.ctypes.data, grouped_token.ctypes.data,
                                          a2g.ctypes.data, None), "pf moe plan")
    return ids, wts, counts, grouped_token, a2g


# ------------------------------------------------------------------ the driver
class WholePromptPrefill:
    """The whole-prompt driver (qwen3_moe_omega_prefill.rs:483-760, device-host form devhost.rs)
    over the fused decode cache. `layers` holds per layer: qkv, o, gate_up, down (Fp8Tensor),
    input_norm, post_norm (f32 [hidden]) and the router gate (f32 or bf16-valued [experts][hidden]);
    `embed_row(token)` gives the f32 embedding row."""

    def __init__(self, layers, final_norm, embed_row, cache, eps, hidden=2048, q_dim=4096, qkv_n=5120,
                 experts=128, top_k=8, inter=768):
        self.h, self.qd, self.qkv_n, self.e, self.top_k, self.i, self.eps = (hidden, q_dim, qkv_n, experts, top_k,
                                                                            inter, eps)
        self.final_norm = np.asarray(final_norm, np.float32)
        self.embed_row = embed_row
        self.attn = PrefillAttention(cache)
        self.bm = qgemm_bm()
        self.t = router_rows()
        self.layers = []
        for L in layers:
            gu, dn = L["gate_up"], L["down"]
            gue = [gu.entry(x) for x in range(experts)]
            dne = [dn.entry(x) for x in range(experts)]
            ent = dict(qkv=(np.array([L["qkv"].entry(0)[0]], np.uint64), np.array([L["qkv"].entry(0)[1]], np.uint64)),
                       o=(np.array([L["o"].entry(0)[0]], np.uint64), np.array([L["o"].entry(0)[1]], np.uint64)),
                       gu=(np.array([v[0] for v in gue], np.uint64), np.array([v[1] for v in gue], np.uint64)),
                       dn=(np.array([v[0] for v in dne], np.uint64), np.array([v[1] for v in dne], np.uint64)))
            wq = pack_router(np.asarray(L["router"], np.float32))
            wq_dev = PfMem(wq.nbytes)
            host = PfMem(wq.nbytes, host=True)
            host.host(np.float32)[:] = wq
            copy_va(wq_dev.va, host.va, wq.nbytes)  # (k / 4 + 1) x e x 16 bytes: a 16-byte multiple
            host.free()
            self.layers.append(dict(ent=ent, wq=wq_dev, input_norm=self._const(L["input_norm"]),
                                    post_norm=self._const(L["post_norm"])))
        self.final_dev = self._const(self.final_norm)
        self.bufs = None
        self.stats = {}

    @staticmethod
    def _const(v):
        """an f32 vector uploaded once to a device buffer"""
        v = np.ascontiguousarray(v, np.float32)
        nb = (v.nbytes + 15) // 16 * 16
        dev, host = PfMem(nb), PfMem(nb, host=True)
        host.host(np.float32)[:v.size] = v
        copy_va(dev.va, host.va, nb)
        host.free()
        return dev

    def _ensure(self, m):
        if self.bufs is not None and self.bufs["m"] >= m:
            return self.bufs
        self.bufs = None
        h, qd, qkv_n, i, e, bm, top_k = self.h, self.qd, self.qkv_n, self.i, self.e, self.bm, self.top_k
        g = m * top_k
        kmax = max(h, qd)
        mt = -(-m // self.t) * self.t
        max_tiles = -(-g // bm) + e
        # HOST buffers are the CPU's side (written or read in place); the kernels read and write
        # DEVICE buffers, and the copies between them are DMA (omega_gpu_pf_copy_va)
        b = dict(m=m, max_tiles=max_tiles,
                 stage=PfMem(max(mt * max(h, e), m * qkv_n, g * h) * 4 + g * 8, host=True),
                 x=PfMem(m * h * 4), xin=PfMem(mt * h * 4), xq=PfMem((m + bm) * kmax), xs=PfMem((m + bm) * (kmax // BLOCK) * 4),
                 qkv=PfMem(m * qkv_n * 4), att=PfMem(m * qd * 4), oproj=PfMem(m * h * 4),
                 logits=PfMem(mt * e * 4), rowidx=PfMem((g + bm) * 4),
                 act=PfMem(g * i * 2), aq=PfMem((g + bm) * i), a_s=PfMem((g + bm) * (i // BLOCK) * 4),
                 down=PfMem(g * h * 4), inv=PfMem(g * 4), wts=PfMem(g * 4), moe=PfMem(m * h * 4),
                 tiles=PfMem(3 * max_tiles * TILE_BYTES, host=True))
        self.bufs = b
        return b

    def _up(self, dst, arr):
        """host rows -> a device buffer through the staging buffer"""
        arr = np.ascontiguousarray(arr)
        nb = (arr.nbytes + 15) // 16 * 16
        if nb > self.bufs["stage"].nbytes or nb > dst.nbytes:
            raise OmegaGpuError(-1, f"staging copy of {nb} bytes exceeds its buffers")
        st = self.bufs["stage"].host(np.uint8)
        st[:arr.nbytes] = arr.view(np.uint8).reshape(-1)
        copy_va(dst.va, self.bufs["stage"].va, nb)

    def _down(self, src, dtype, count):
        nb = (count * np.dtype(dtype).itemsize + 15) // 16 * 16
        if nb > self.bufs["stage"].nbytes or nb > src.nbytes:
            raise OmegaGpuError(-1, f"staging copy of {nb} bytes exceeds its buffers")
        copy_va(self.bufs["stage"].va, src.va, nb)
        return self.bufs["stage"].host(dtype)[:count].copy()

    def _put_tiles(self, b, region, ws, counts):
        """the tile table of (weights, scales) addresses `ws` over `counts` rows per expert, built
        by the library's builder straight into the pinned table region"""
        w, sc = ws
        c = np.ascontiguousarray(counts, np.uint32)
        off = region * b["max_tiles"] * TILE_BYTES
        n = lib().omega_gpu_pf_qgemm_tiles_va(len(c), w.ctypes.data, sc.ctypes.data, c.ctypes.data,
                                              b["tiles"].host(np.uint8)[off:].ctypes.data, b["max_tiles"])
        if n == 0:
            raise OmegaGpuError(-1, f"tile table larger than its region of {b['max_tiles']} entries")
        return b["tiles"].va + off, n

    def run(self, tokens, pos0, trace=None):
        """Tokens at positions pos0 .. pos0 + m - 1 through every layer; returns the last token's
        final-normed hidden row. `trace` (a dict) receives per layer the q|k|v rows, the attention
        rows, the residual rows after the attention and after the MoE, the router logits and the
        routed ids (the recorder of qwen3_moe_omega_prefill.rs WpTrace)."""
        m = len(tokens)
        if m == 0:
            raise OmegaGpuError(-1, "whole-prompt prefill of 0 tokens")
        h, qd, qkv_n, e, top_k, i, eps = self.h, self.qd, self.qkv_n, self.e, self.top_k, self.i, self.eps
        g = m * top_k
        b = self._ensure(m)
        self._up(b["x"], np.stack([np.asarray(self.embed_row(t), np.float32) for t in tokens]))
        chip = 0
        dense = [m]
        add = 0  # the previous layer's MoE rows, added to the residual by the next norm
        for l, L in enumerate(self.layers):
            ent = L["ent"]
            chip += residual_norm(h, m, b["x"].va, add, L["input_norm"].va, eps, b["xin"].va)
            if trace is not None and l > 0:
                trace.setdefault("x_out", []).append(self._down(b["x"], np.float32, m * h).reshape(m, h))
            chip += quant(h, IN_F32, m, b["xin"].va, b["xq"].va, b["xs"].va)
            tv, nt = self._put_tiles(b, 0, ent["qkv"], dense)
            chip += qgemm(qkv_n, h, PLAIN, tv, nt, 0, b["xq"].va, b["xs"].va, b["qkv"].va)
            info = self.attn.attend_dev(l, pos0, m, b["qkv"].va, eps, 1.0, b["att"].va)
            chip += info.elapsed_ns
            if trace is not None:
                trace.setdefault("qkv", []).append(self._down(b["qkv"], np.float32, m * qkv_n).reshape(m, qkv_n))
                trace.setdefault("att", []).append(self._down(b["att"], np.float32, m * qd).reshape(m, qd))
            chip += quant(qd, IN_F32, m, b["att"].va, b["xq"].va, b["xs"].va)
            tv, nt = self._put_tiles(b, 1, ent["o"], dense)
            chip += qgemm(h, qd, PLAIN, tv, nt, 0, b["xq"].va, b["xs"].va, b["oproj"].va)
            # x += o_proj, then the post-norm rows: the quantiser's and the router's input
            chip += residual_norm(h, m, b["x"].va, b["oproj"].va, L["post_norm"].va, eps, b["xin"].va)
            chip += router_logits(h, e, m, b["xin"].va, L["wq"].va, b["logits"].va)
            logits = self._down(b["logits"], np.float32, m * e)
            ids, wts, counts, grouped_token, a2g = moe_plan(logits, m, e, top_k)
            if trace is not None:
                trace.setdefault("x_mid", []).append(self._down(b["x"], np.float32, m * h).reshape(m, h))
                trace.setdefault("post", []).append(self._down(b["xin"], np.float32, m * h).reshape(m, h))
                trace.setdefault("ids", []).append(ids.copy())
                trace.setdefault("wts", []).append(wts.copy())
                trace.setdefault("a2g", []).append(a2g.copy())
                trace.setdefault("logits", []).append(logits.reshape(m, e).copy())
            chip += quant(h, IN_F32, m, b["xin"].va, b["xq"].va, b["xs"].va)
            self._up(b["rowidx"], grouped_token)
            tv, nt = self._put_tiles(b, 2, ent["gu"], counts)
            chip += qgemm(2 * i, h, SWIGLU_NAT, tv, nt, b["rowidx"].va, b["xq"].va, b["xs"].va, b["act"].va)
            chip += quant(i, IN_BF16, g, b["act"].va, b["aq"].va, b["a_s"].va)
            tv, nt = self._put_tiles(b, 2, ent["dn"], counts)
            chip += qgemm(h, i, PLAIN, tv, nt, 0, b["aq"].va, b["a_s"].va, b["down"].va)
            self._up(b["inv"], a2g)
            self._up(b["wts"], wts.reshape(-1))
            chip += moe_combine(h, top_k, m, b["down"].va, b["inv"].va, b["wts"].va, b["moe"].va)
            if trace is not None:
                trace.setdefault("act", []).append(self._down(b["act"], np.uint16, g * i).reshape(g, i))
                trace.setdefault("down", []).append(self._down(b["down"], np.float32, g * h).reshape(g, h))
            add = b["moe"].va
        # the last MoE add, then the final norm (over every row: one launch either way)
        chip += residual_norm(h, m, b["x"].va, add, self.final_dev.va, eps, b["xin"].va)
        if trace is not None:
            trace.setdefault("x_out", []).append(self._down(b["x"], np.float32, m * h).reshape(m, h))
        self.stats = dict(tokens=m, chip_ns=chip)
        return self._down(b["xin"], np.float32, m * h)[(m - 1) * h:].copy()

    def free(self):
        self.bufs = None
        for L in self.layers:
            L["wq"].free()
            L["input_norm"].free()
            L["post_norm"].free()
        self.final_dev.free()
