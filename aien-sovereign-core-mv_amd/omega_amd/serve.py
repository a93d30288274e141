"""Many conversations at once over one upload of the weights: a beat scheduler around the batched
serving decode (omega_gpu_batch_decode_*), the serving mode of configuration 5.

The shape follows the reference's batching door (aien-serve-http/src/qwen36_batch.rs:1-28) and
the engine's concurrency contract (aien-serve-http/src/engine.rs:125-179): `slots` conversation
rows share every weight read; every beat feeds one token of every live row (its next prompt
token while the prompt is going in, else the token it sampled last); requests join at the next
beat and leave when they stop or reach their length, and the other rows never notice. A request
beyond the free slots is refused (`SchedulerBusy`, the server's 503 server_busy).

Each row's KV lives in pages of the caller's device pool (the aien-kv-cache page layout); a
request reserves the pages of its whole length when it is admitted and returns them when it
leaves. The batched step computes every row the same way whatever the batch holds (its attention
is cut per page while a beat holds at most 512 pages, and to rounding past that), so a row's
tokens are the tokens that request gets alone.
"""
from __future__ import annotations

import ctypes as C
from collections import deque

import numpy as np

from . import OmegaGpuError


def _addr(p):
    return (p.value or 0) if isinstance(p, C.c_void_p) else int(p)


class SchedulerBusy(OmegaGpuError):
    """Every slot is taken (the server answers 503 server_busy)."""


class Request:
    """One conversation: its prompt, limits, and what it has produced so far."""

    def __init__(self, rid, prompt, max_new, stop, on_token):
        self.rid = rid
        self.prompt = [int(t) for t in prompt]
        self.max_new = int(max_new)
        self.stop = set(int(t) for t in stop)
        self.on_token = on_token
        self.tokens: list[int] = []   # generated tokens, in order
        self.fed = 0                  # positions fed so far (prompt and generated)
        self.pages: list[int] = []    # pool blocks of positions 0, 16, 32, ...
        self.finish = None            # "stop", "length", "cancelled" or "error" once it has left
        self.error = None             # the exception that ended it ("error")
        self.joined_beat = self.first_token_beat = self.left_beat = None
        self.cancelled = False

    @property
    def done(self):
        return self.finish is not None


class PromptPrefill:
    """Prompts that go in whole instead of one token per beat. Positions 0 .. n - 2 of a joining
    request run through the whole-prompt prefill `wp` (omega_amd.prefill.WholePromptPrefill) into
    its fused decode cache, leave that cache as the HostPagedPoolV1 payload
    (omega_gpu_decode_attn_cache_export_dev), whose blocks are the pool's pages byte for byte, and
    are copied into the request's pages; the last prompt token then goes through the batched step,
    which gives the first generated token. The prompt's K / V are the prefill's (W8A8) rows, as
    with the reference engine's whole-prompt mode."""

    def __init__(self, wp, cache, pool_ptr, max_positions, min_tokens=16):
        from . import DeviceBuffer

        self.wp, self.cache, self.pool_ptr, self.min_tokens = wp, cache, _addr(pool_ptr), min_tokens
        self.block_bytes = cache.payload_len(16)
        self.payload = DeviceBuffer(cache.payload_len(max_positions))
        self.max_positions = max_positions

    def fill(self, tokens, pages):
        from .prefill import copy_va

        n = len(tokens)
        if n > self.max_positions:
            raise OmegaGpuError(-1, f"schedule prefill of {n} tokens > {self.max_positions}")
        self.wp.run(tokens, 0)
        nbytes = self.cache.payload_len(n)
        self.cache.export_kv_dev(0, n, self.payload.ptr, nbytes)
        base = _addr(self.payload.ptr)
        for j in range(nbytes // self.block_bytes):
            copy_va(self.pool_ptr + pages[j] * self.block_bytes, base + j * self.block_bytes, self.block_bytes)

    def free(self):
        self.payload.free()


class BeatScheduler:
    """The beat loop over a BatchDecode whose KV pool has `num_blocks` pages of `block_size`
    tokens and whose tables hold `max_blocks` pages per row."""

    def __init__(self, bd, num_blocks, max_blocks, block_size=16, slots=None, prefill: PromptPrefill | None = None):
        self.bd = bd
        self.prefill = prefill
        self.block_size = block_size
        self.max_blocks = max_blocks
        self.slots = min(int(bd.cfg.max_seqs), int(slots or bd.cfg.max_seqs))
        self.free_pages = deque(range(num_blocks))
        self.pending: deque[Request] = deque()
        self.live: list[Request] = []
        self.beats = 0
        self.fed_tokens = 0
        self._next_id = 0

    def concurrency(self):
        """Conversations stacked on one weight read (Engine::concurrency)."""
        return self.slots

    def submit(self, prompt, max_new, stop=(), on_token=None) -> Request:
        """Queues a request for the next beat. Refuses an empty prompt, a length past the row's
        page table, too few free pages, or a full house (SchedulerBusy)."""
        if len(prompt) == 0 or max_new < 1:
            raise OmegaGpuError(-1, "schedule: an empty prompt or max_new < 1")
        length = len(prompt) + max_new
        pages = -(-length // self.block_size)
        if pages > self.max_blocks:
            raise OmegaGpuError(-1, f"schedule: {length} positions need {pages} pages, a row holds {self.max_blocks}")
        if len(self.live) + len(self.pending) >= self.slots:
            raise SchedulerBusy(-1, f"schedule: all {self.slots} slots are taken")
        if pages > len(self.free_pages):
            raise SchedulerBusy(-1, f"schedule: {pages} pages needed, {len(self.free_pages)} free")
        r = Request(self._next_id, prompt, max_new, stop, on_token)
        self._next_id += 1
        r.pages = [self.free_pages.popleft() for _ in range(pages)]
        self.pending.append(r)
        return r

    def cancel(self, r: Request):
        """The client went away: the request leaves at the next beat."""
        r.cancelled = True

    def _leave(self, r: Request, why: str):
        r.finish = why
        r.left_beat = self.beats
        self.free_pages.extend(r.pages)
        r.pages = []

    def _prefills(self, r: Request) -> bool:
        """Whether the joining request's prompt goes through the whole-prompt prefill: long enough
        to be worth it and within the prefill's capacity (a longer prompt is fed one token per
        beat like a short one)."""
        n = len(r.prompt) - 1
        return bool(self.prefill) and self.prefill.min_tokens <= n <= self.prefill.max_positions

    def beat(self):
        """One step of every live row. Returns the number of rows that stepped. A request whose
        prompt prefill fails leaves with finish "error" (its pages returned, `error` set); the
        other rows go on."""
        while self.pending:
            r = self.pending.popleft()
            r.joined_beat = self.beats
            if r.cancelled:  # left before it ever ran: no prefill for it
                self._leave(r, "cancelled")
                continue
            if self._prefills(r):
                try:
                    self.prefill.fill(r.prompt[:-1], r.pages)
                except Exception as e:  # noqa: BLE001 - the request ends, the beat goes on
                    r.error = e
                    self._leave(r, "error")
                    continue
                r.fed = len(r.prompt) - 1
            self.live.append(r)
        for r in [r for r in self.live if r.cancelled]:
            self._leave(r, "cancelled")
        self.live = [r for r in self.live if not r.done]
        if not self.live:
            return 0
        n = len(self.live)
        tables = np.full((n, self.max_blocks), -1, np.int32)
        tokens = np.empty(n, np.uint32)
        positions = np.empty(n, np.uint32)
        for i, r in enumerate(self.live):
            tables[i, :len(r.pages)] = r.pages
            p = r.fed
            tokens[i] = r.prompt[p] if p < len(r.prompt) else r.tokens[-1]
            positions[i] = p
        self.bd.set_tables(tables)
        out = self.bd.step(tokens, positions)
        self.beats += 1
        self.fed_tokens += n
        for i, r in enumerate(self.live):
            r.fed += 1
            if r.fed < len(r.prompt):
                continue  # a prompt position: its prediction is the next prompt token
            t = int(out[i])
            r.tokens.append(t)
            if r.first_token_beat is None:
                r.first_token_beat = self.beats
            keep = r.on_token(t) if r.on_token else True
            if keep is False:
                self._leave(r, "cancelled")
            elif t in r.stop:
                self._leave(r, "stop")
            elif len(r.tokens) >= r.max_new:
                self._leave(r, "length")
        self.live = [r for r in self.live if not r.done]
        return n

    def run(self, arrivals=None):
        """Beats until every request has left. `arrivals` maps a beat number to a list of
        (key, prompt, max_new, stop) submitted before that beat; an arrival that finds every slot
        taken waits for the next beat (a client retrying after server_busy). Returns
        {key: Request}."""
        waiting = deque()
        arrivals = {b: list(v) for b, v in (arrivals or {}).items()}
        out: dict = {}
        while self.live or self.pending or arrivals or waiting:
            waiting.extend(arrivals.pop(self.beats, []))
            while waiting:
                key, prompt, max_new, stop = waiting[0]
                try:
                    out[key] = self.submit(prompt, max_new, stop)
                except SchedulerBusy:
                    break
                waiting.popleft()
            if self.beat():
                continue
            if waiting:  # nothing live, yet the first waiting request cannot be admitted
                raise OmegaGpuError(-1, f"schedule: request {waiting[0][0]!r} can never be admitted")
            if arrivals:
                self.beats = min(arrivals)  # idle until the next arrival
        return out
