"""The beat scheduler's host logic on the CPU (omega_amd.serve.BeatScheduler), over a stand-in
for the batched step: a prefill failure ends only its own request and returns its pages, a
request cancelled before it joins never runs the prefill, and a prompt past the prefill's
capacity is fed one token per beat instead (the shape of the reference's batching door,
aien-serve-http/src/qwen36_batch.rs:1-28)."""
import types

import numpy as np
import pytest

from omega_amd.serve import BeatScheduler


class FakeStep:
    """Stands in for BatchDecode: the next token of a row is its position + 1000."""

    def __init__(self, max_seqs=4):
        self.cfg = types.SimpleNamespace(max_seqs=max_seqs)
        self.calls = []

    def set_tables(self, tables):
        self.tables = tables.copy()

    def step(self, tokens, positions):
        self.calls.append((tokens.copy(), positions.copy()))
        return (positions + 1000).astype(np.uint32)


class FakePrefill:
    def __init__(self, max_positions=64, min_tokens=4, fail_on=()):
        self.max_positions, self.min_tokens, self.fail_on = max_positions, min_tokens, set(fail_on)
        self.filled = []

    def fill(self, tokens, pages):
        if tokens[0] in self.fail_on:
            raise RuntimeError("device error in the prompt prefill")
        self.filled.append((list(tokens), list(pages)))


def test_prefill_failure_ends_only_that_request():
    bd, pf = FakeStep(), FakePrefill(fail_on={7})
    s = BeatScheduler(bd, num_blocks=64, max_blocks=8, prefill=pf)
    bad = s.submit([7] * 10, 3)
    good = s.submit([1] * 10, 3)
    free_before = len(s.free_pages)
    s.run()
    assert bad.finish == "error" and isinstance(bad.error, RuntimeError) and bad.tokens == []
    assert good.finish == "length" and good.tokens == [1009, 1010, 1011]
    assert len(s.free_pages) == 64 and free_before == 64 - 1 - 1  # 13 positions: one page each


def test_cancelled_before_joining_runs_no_prefill():
    bd, pf = FakeStep(), FakePrefill()
    s = BeatScheduler(bd, num_blocks=32, max_blocks=8, prefill=pf)
    r = s.submit([2] * 20, 4)
    s.cancel(r)
    assert s.beat() == 0
    assert r.finish == "cancelled" and pf.filled == [] and bd.calls == []
    assert len(s.free_pages) == 32


def test_prompt_past_the_prefill_capacity_is_fed_per_beat():
    bd, pf = FakeStep(), FakePrefill(max_positions=8)
    s = BeatScheduler(bd, num_blocks=32, max_blocks=8, prefill=pf)
    long = s.submit(list(range(20)), 2)
    short = s.submit(list(range(6)), 2)
    s.run()
    # the 6-token prompt's first 5 positions went through the prefill, the 20-token one did not
    assert [len(t) for t, _ in pf.filled] == [5]
    assert long.finish == "length" and long.tokens == [1019, 1020]
    assert short.tokens == [1005, 1006]
    # the long prompt was fed token by token: its first beat fed position 0
    assert bd.calls[0][1].tolist() == [0, 5]


def test_busy_and_bad_requests_are_refused():
    from omega_amd import OmegaGpuError
    from omega_amd.serve import SchedulerBusy

    s = BeatScheduler(FakeStep(max_seqs=1), num_blocks=4, max_blocks=2)
    with pytest.raises(OmegaGpuError):
        s.submit([], 1)
    with pytest.raises(OmegaGpuError):
        s.submit([1] * 40, 1)   # 41 positions need 3 pages, a row holds 2
    s.submit([1], 1)
    with pytest.raises(SchedulerBusy):
        s.submit([1], 1)
