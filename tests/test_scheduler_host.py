"""Host logic of BatchScheduler on the CPU, against a deterministic stand-in
for the engine that keeps the engine's contract (sequences, positions added
in order, logit rows in row order, at most two asynchronous steps in flight,
token sources resolved from the step issued just before).  Its "model" picks
the next token from a hash of the sequence's whole token history, so any
mistake in what a row feeds (wrong token, wrong position, a row fed twice or
skipped) changes every later token of that stream.

Checked: the pipelined run (step N+1 issued before step N's tokens are
collected) issues the same steps as the unpipelined run when no request
stops on EOS; with EOS it drops exactly one row per request that stops
before its last allowed token, and the streams are the same; every
sequence is released; the observer sees each step's logit-row requests in
row order; and the stand-in refuses what the engine refuses.
"""
import hashlib

import numpy as np
import pytest

from qraf_amd.engine import BatchScheduler

V = 97


def next_token(history):
    h = hashlib.blake2b(np.asarray(history, np.int64).tobytes(), digest_size=8).digest()
    return int.from_bytes(h, "little") % V


class FakeEngine:
    def __init__(self, max_batch=64):
        self.max_batch = max_batch
        self.seqs = {}        # id -> token history (position i holds the token fed at i)
        self.free_ids = []
        self.next_id = 0
        self.inflight = []    # issued, not collected: token lists
        self.last = None      # tokens of the step issued last (the token sources of the next)
        self.rows_run = 0
        self.released = []

    def seq_create(self):
        if self.free_ids:
            i = self.free_ids.pop()
        else:
            i = self.next_id
            self.next_id += 1
        self.seqs[i] = []
        return i

    def seq_release(self, i):
        assert i in self.seqs, f"release of unknown sequence {i}"
        del self.seqs[i]
        self.free_ids.append(i)
        self.released.append(i)

    def _run(self, seq_ids, tokens, positions, want_logits, token_src=None):
        n = len(seq_ids)
        assert 0 < n <= self.max_batch
        want = [True] * n if want_logits is None else [bool(w) for w in want_logits]
        out = []
        for i in range(n):
            s, p = seq_ids[i], positions[i]
            t = int(tokens[i])
            if token_src is not None and token_src[i] >= 0:
                assert self.last is not None and token_src[i] < len(self.last), "token source past the last step"
                t = self.last[token_src[i]]
            # a row of a released sequence would be a scheduler bug: no such rows are issued
            assert s in self.seqs, f"row of sequence {s}, which is not live"
            hist = self.seqs[s]
            assert p == len(hist), f"sequence {s}: position {p}, length {len(hist)}"
            hist.append(t)
            if want[i]:
                out.append(next_token(hist))
        self.rows_run += n
        self.last = out
        return out

    def step(self, seq_ids, tokens, positions, want_logits=None, logits=False, argmax=True):
        assert not self.inflight, "synchronous step while steps are in flight"
        out = self._run(seq_ids, tokens, positions, want_logits)
        return None, np.array(out, np.uint32)

    def step_async(self, seq_ids, tokens, positions, want_logits=None, token_src=None):
        assert len(self.inflight) < 2, "a third step in flight"
        self.inflight.append(self._run(seq_ids, tokens, positions, want_logits, token_src))

    def collect(self):
        assert self.inflight, "nothing in flight"
        return np.array(self.inflight.pop(0), np.uint32)


def workload(seed, n, plen=(1, 40), olen=(0, 30)):
    rng = np.random.default_rng(seed)
    return [(rng.integers(0, V, int(rng.integers(*plen))).tolist(), int(rng.integers(*olen))) for _ in range(n)]


def run(work, pipeline, eos=None, max_batch=4, max_rows=16, chunk=5, observe=False):
    e = FakeEngine(max_batch=max_rows)
    s = BatchScheduler(e, max_batch=max_batch, max_rows=max_rows, prefill_chunk=chunk, pipeline=pipeline)
    seen = []
    if observe:
        s.observer = lambda sc, lrows, nx: seen.append(([r.id for r in lrows], [int(t) for t in nx]))
    ids = [s.submit(p, o, eos=eos) for p, o in work]
    done = {r.id: r for r in s.run()}
    assert not e.seqs, "every sequence is released"
    assert not e.inflight
    return [done[i].generated for i in ids], s.steps, s.rows, e, seen, [done[i] for i in ids]


def reference_stream(prompt, max_tokens, eos=None):
    hist, out = list(prompt), []
    while len(out) < max_tokens:
        t = next_token(hist)
        if eos is not None and t == eos:
            break
        out.append(t)
        hist.append(t)
    return out


@pytest.mark.parametrize("max_batch,max_rows,chunk", [(1, 1, 1), (3, 3, 1), (4, 16, 5), (8, 64, 64), (5, 7, 3)])
def test_pipelined_equals_unpipelined_without_eos(max_batch, max_rows, chunk):
    work = workload(1, 23)
    a = run(work, False, max_batch=max_batch, max_rows=max_rows, chunk=chunk)
    b = run(work, True, max_batch=max_batch, max_rows=max_rows, chunk=chunk)
    assert a[0] == b[0]
    assert (a[1], a[2]) == (b[1], b[2]), "the same steps, row for row"
    for (p, o), g in zip(work, a[0]):
        assert g == reference_stream(p, o)


@pytest.mark.parametrize("seed", [2, 3, 4])
def test_pipelined_eos_drops_one_row_per_early_stop(seed):
    work = workload(seed, 19, olen=(5, 40))
    full = [reference_stream(p, o) for p, o in work]
    # the token (past the first) that most streams contain
    counts = {}
    for f in full:
        for t in set(f[1:]):
            counts[t] = counts.get(t, 0) + 1
    eos = max(sorted(counts), key=lambda t: counts[t])
    want = [reference_stream(p, o, eos) for p, o in work]
    a = run(work, False, eos=eos)
    b = run(work, True, eos=eos)
    assert a[0] == want and b[0] == want
    dropped = sum(len(w) < o - 1 for w, (_, o) in zip(want, work))
    assert dropped >= 1
    assert b[2] == a[2] + dropped


def test_zero_max_tokens_and_single_token_prompts():
    work = [([5], 0), ([7], 1), ([1, 2, 3], 0), ([9], 2)]
    for pipeline in (False, True):
        got = run(work, pipeline, max_batch=2, max_rows=2, chunk=1)[0]
        assert got == [reference_stream(p, o) for p, o in work]


def test_observer_sees_logit_rows_in_order():
    work = workload(5, 9)
    _, _, _, _, seen_a, _ = run(work, False, observe=True)
    _, _, _, _, seen_b, _ = run(work, True, observe=True)
    assert seen_a == seen_b
    assert all(len(ids) == len(toks) for ids, toks in seen_a)


def test_inflight_counts_return_to_zero():
    work = workload(6, 12)
    *_, reqs = run(work, True)
    assert all(r.inflight == 0 and r.state == "DONE" for r in reqs)


def test_stand_in_refuses_what_the_engine_refuses():
    e = FakeEngine()
    s = e.seq_create()
    e.step_async([s], [1], [0])
    e.step_async([s], [0], [1], token_src=[0])
    with pytest.raises(AssertionError):
        e.step_async([s], [0], [2], token_src=[0])  # a third step in flight
    with pytest.raises(AssertionError):
        e.step([s], [0], [2])  # synchronous step while steps are in flight
    e.collect()
    e.collect()
    with pytest.raises(AssertionError):
        e.collect()
    with pytest.raises(AssertionError):
        e.step_async([s], [0], [2], token_src=[1])  # the last step left one logit row
