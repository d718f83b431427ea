"""Continuous-batching scheduler (velox_amd/csrc/sched.cpp) on the CPU,
through the C ABI, driving a toy engine written in Python
(`vx_sched_create_with_backend`).

The toy engine keeps token ids in its KV "pages" and predicts the next token
from the context it reads back through the block tables, so a wrong block
table, a wrongly shared prefix page or a write into a shared page changes
the output.  Expected outputs are the greedy continuations computed straight
from the token sequences; speculative rounds must commit exactly these
(spec.rs:266-301: accepted draft prefix plus the target's token).

Reference behaviour covered (scheduler.rs, prefix_cache.rs, request.rs):
FCFS admission bounded by max_running_requests and by free pages with the
request left at the head of the queue, the max_batch_tokens budget walked in
request-id order, EOS ("stop") and max_tokens ("length") with the
finish-reason rule, "Empty prompt", prefix-cache hits and refcounts, LRU
eviction that frees pages, cancel.
"""
import zlib

import numpy as np
import pytest

from velox_amd._lib import VeloxError
from velox_amd.scheduler import BatchScheduler, PyBackend, RequestStatus, SchedulerConfig

V = 1000


def target_next(ctx):
    return zlib.crc32(np.asarray(ctx, np.uint32).tobytes()) % V


def draft_next(ctx):
    t = target_next(ctx)
    return t if zlib.crc32(np.asarray(ctx[-3:], np.uint32).tobytes()) % 3 else (t + 1) % V


def greedy(prompt, max_new, eos=()):
    ctx, out = list(prompt), []
    while len(out) < max_new:
        t = target_next(ctx)
        out.append(t)
        ctx.append(t)
        if t in eos:
            break
    return out


class Pool:
    def __init__(self, n, ps):
        self.free = list(range(n - 1, -1, -1))
        self.ref = [0] * n
        self.slots = np.full((n, ps), -1, np.int64)

    def alloc(self, n):
        assert len(self.free) >= n
        out = [self.free.pop() for _ in range(n)]
        for p in out:
            self.ref[p] = 1
        return out

    def incref(self, pages):
        for p in pages:
            assert self.ref[p] >= 1
            self.ref[p] += 1

    def decref(self, pages):
        for p in pages:
            assert self.ref[p] >= 1
            self.ref[p] -= 1
            if self.ref[p] == 0:
                self.free.append(p)


class ToyEngine(PyBackend):
    def __init__(self, pages=64, ps=8):
        super().__init__(ps)
        self.ps = ps
        self.pools = [Pool(pages, ps), Pool(pages, ps)]
        self.states = {}
        self.next_id = 0
        self.calls = []  # ("prefill", {state: n}) / ("step", [states])

    # --- helpers
    def write(self, which, st, pos, tok):
        bt = st["bt"][which]
        page = bt[pos // self.ps]
        assert self.pools[which].ref[page] == 1, f"write into shared page {page}"
        self.pools[which].slots[page, pos % self.ps] = tok

    def read(self, which, st, n):
        bt = st["bt"][which]
        return [int(self.pools[which].slots[bt[p // self.ps], p % self.ps]) for p in range(n)]

    # --- backend interface
    def add_state(self, prompt, cached, tp, dp, reserve, stream_id, temperature):
        need = -(-max(reserve, len(prompt) - 1) // self.ps)
        extra = need - len(tp)
        if extra > min(len(self.pools[0].free), len(self.pools[1].free)):
            raise MemoryError("not enough free pages")
        st = dict(prompt=list(prompt), kv=cached, bt=[tp + self.pools[0].alloc(extra), dp + self.pools[1].alloc(extra)],
                  stream=stream_id, temp=temperature, ready=cached == len(prompt) - 1, gen=[])
        sid = self.next_id
        self.next_id += 1
        self.states[sid] = st
        return sid

    def prefill_chunk(self, states, n_tokens):
        self.calls.append(("prefill", dict(zip(states, n_tokens))))
        for s, n in zip(states, n_tokens):
            st = self.states[s]
            assert not st["ready"] and st["kv"] + n <= len(st["prompt"]) - 1
            for p in range(st["kv"], st["kv"] + n):
                for w in (0, 1):
                    self.write(w, st, p, st["prompt"][p])
            st["kv"] += n
            st["ready"] = st["kv"] == len(st["prompt"]) - 1

    def step(self, states, k):
        self.calls.append(("step", list(states)))
        assert len({self.states[s]["temp"] for s in states}) == 1, "mixed temperatures in one round"
        res = []
        for s in states:
            st = self.states[s]
            assert st["ready"]
            kv = st["kv"]
            ctx_t = self.read(0, st, kv)
            ctx_d = self.read(1, st, kv)
            assert ctx_t == ctx_d == (st["prompt"] + st["gen"])[:kv], "KV does not hold the sequence"
            last = (st["prompt"] + st["gen"])[kv]
            # draft: k tokens, writing its KV at kv .. kv+k-1
            ctx = ctx_d + [last]
            cand = []
            for i in range(k):
                self.write(1, st, kv + i, ctx[-1])
                c = draft_next(ctx)
                cand.append(c)
                ctx.append(c)
            # verify rows kv .. kv+k: [last, c0 .. c_{k-1}]
            rows = [last] + cand
            for j, t in enumerate(rows):
                self.write(0, st, kv + j, t)
            ctx = ctx_t + [last]
            acc, out = 0, []
            for j in range(k):
                t = target_next(ctx)
                if cand[j] != t:
                    break
                out.append(t)
                ctx.append(t)
                acc += 1
            out.append(target_next(ctx))
            if acc == k:  # fill the draft's slot kv + k (the engine's fix_draft_hole)
                self.write(1, st, kv + k, cand[k - 1])
            st["gen"] += out
            st["kv"] += acc + 1
            res.append((acc, out))
        return res

    def state_pages(self, s, which):
        return list(self.states[s]["bt"][which])

    def free_state(self, s):
        st = self.states.pop(s)
        for w in (0, 1):
            self.pools[w].decref(st["bt"][w])

    def incref(self, which, pages):
        self.pools[which].incref(pages)

    def decref(self, which, pages):
        self.pools[which].decref(pages)

    def free_pages(self):
        return [len(p.free) for p in self.pools]


def make(pages=64, ps=8, eos=(), **cfg):
    eng = ToyEngine(pages, ps)
    c = dict(max_running_requests=64, max_batch_tokens=512, prefix_cache_capacity=0, draft_k=4)
    c.update(cfg)
    return eng, BatchScheduler(eng, eos, SchedulerConfig(**c))


def prompt(seed, n):
    return list(np.random.default_rng(seed).integers(0, V, n))


def test_generates_greedy_continuations_and_returns_pages():
    eng, s = make()
    ps_ = [prompt(i, n) for i, n in enumerate((5, 17, 30))]
    ids = [s.submit(p, 12) for p in ps_]
    assert ids == [1, 2, 3]
    steps = s.run(100)
    for rid, p in zip(ids, ps_):
        r = s.poll(rid)
        assert r.status == RequestStatus.FINISHED and r.finish_reason == "length"
        assert r.tokens == greedy(p, 12)
    st = s.stats()
    assert st["requests_completed"] == 3 and st["steps"] == steps
    assert st["tokens_generated"] == 36
    assert st["prefill_tokens"] == sum(len(p) - 1 for p in ps_)
    assert st["draft_tokens_proposed"] == 4 * sum(len(a) for kind, a in eng.calls if kind == "step")
    assert 0 < st["draft_tokens_accepted"] < st["draft_tokens_proposed"]
    assert eng.free_pages() == [64, 64] and not eng.errors
    # the stream of a request defaults to its id
    s.release(1)
    with pytest.raises(VeloxError, match="unknown request"):
        s.poll(1)


def test_max_running_requests():
    eng, s = make(max_running_requests=2)
    ps_ = [prompt(10 + i, 9) for i in range(5)]
    ids = [s.submit(p, 6) for p in ps_]
    while s.num_waiting() + s.num_running():
        s.step()
        assert s.num_running() <= 2
    for rid, p in zip(ids, ps_):
        assert s.poll(rid).tokens == greedy(p, 6)


def test_admission_waits_for_pages_fcfs():
    """A request that does not fit stays at the head of the queue
    (scheduler.rs:283-293); later, smaller requests do not overtake it."""
    eng, s = make(pages=6, ps=8)
    big = prompt(20, 30)   # 30 + 8 + 4 = 42 positions -> 6 pages
    small = prompt(21, 5)  # 5 + 8 + 4 -> 3 pages
    r1 = s.submit(small, 8)
    r2 = s.submit(big, 8)
    r3 = s.submit(small, 8)
    s.step()
    assert s.num_running() == 1 and s.num_waiting() == 2  # big blocks small #3
    order = []
    while s.num_waiting() + s.num_running():
        s.step()
        for rid in (r1, r2, r3):
            if s.poll(rid).status == RequestStatus.FINISHED and rid not in order:
                order.append(rid)
    assert order == [r1, r2, r3]
    assert s.poll(r2).tokens == greedy(big, 8)
    assert eng.free_pages() == [6, 6]


def test_budget_chunks_prefill_and_defers_decodes():
    eng, s = make(max_batch_tokens=16, draft_k=4)
    a = prompt(30, 50)
    r1 = s.submit(prompt(31, 6), 20)
    r2 = s.submit(a, 5)
    s.run(200)
    assert s.poll(r2).tokens == greedy(a, 5)
    for kind, arg in eng.calls:
        if kind == "prefill":
            assert all(1 <= n <= 16 for n in arg.values())
    # per step: prefill tokens + 5 per decoding request stay within 16
    chunks = [sum(arg.values()) for kind, arg in eng.calls if kind == "prefill"]
    assert sum(chunks) == 5 + 49 and max(chunks) <= 16
    # a budget below k+1 still runs one decode per step (the first request always runs)
    eng2, s2 = make(max_batch_tokens=3, draft_k=4)
    p = prompt(32, 4)
    rids = [s2.submit(p, 4), s2.submit(p, 4)]
    s2.run(100)
    assert all(len(arg) == 1 for kind, arg in eng2.calls if kind == "step")
    assert all(s2.poll(r).tokens == greedy(p, 4) for r in rids)


def test_eos_and_length_finish():
    p = prompt(40, 7)
    g = greedy(p, 30)
    eos = g[5]
    eng, s = make(eos=(eos, 999999))
    r = s.submit(p, 30)
    r2 = s.submit(p, 3)
    s.run(100)
    res = s.poll(r)
    assert res.finish_reason == "stop" and res.tokens == g[:g.index(eos) + 1]
    res2 = s.poll(r2)
    assert res2.finish_reason == ("stop" if eos in g[:3] else "length") and res2.tokens == greedy(p, 3, (eos,))
    assert s.poll(s.submit(p, 0)).status == RequestStatus.WAITING  # max_tokens raised to 1
    s.run(10)
    assert len(s.poll(3).tokens) == 1


def test_prefix_cache_shares_pages_between_concurrent_requests():
    """Four requests with a common 40-token prefix (5 pages of 8), submitted
    together: the first prefills it, the others wait for its pages and then
    reuse them (the same physical pages in their block tables)."""
    eng, s = make(pages=64, ps=8, prefix_cache_capacity=32, max_batch_tokens=64)
    shared = prompt(50, 40)
    ps_ = [shared + prompt(60 + i, 6 + i) for i in range(4)]
    ids = [s.submit(p, 10) for p in ps_]
    s.step()
    assert s.num_running() == 1 and s.num_waiting() == 3
    seen = {}
    while s.num_waiting() + s.num_running():
        s.step()
        for sid, st in eng.states.items():
            seen.setdefault(tuple(st["prompt"]), [list(st["bt"][0][:5]), list(st["bt"][1][:5])])
    for rid, p in zip(ids, ps_):
        assert s.poll(rid).tokens == greedy(p, 10)
    tables = list(seen.values())
    assert all(t == tables[0] for t in tables)
    st = s.stats()
    assert st["prefix_cache_hits"] == 3 and st["prefix_cache_misses"] == 1
    assert st["prefix_tokens_skipped"] == 3 * 40
    assert st["prefill_tokens"] == sum(len(p) - 1 for p in ps_) - 120
    # the cache alone holds its pages now; closing it returns them
    held = s.cache_pages()
    assert held > 0 and eng.free_pages() == [64 - held, 64 - held]
    s.close()
    assert eng.free_pages() == [64, 64]


def test_prefix_hit_never_covers_last_prompt_position():
    """A prompt of exactly k pages + 1 token can reuse all k pages; one of
    exactly k pages reuses k - 1 (position len - 1 is written by the first
    round)."""
    eng, s = make(pages=64, ps=8, prefix_cache_capacity=32)
    base = prompt(70, 24)
    r0 = s.submit(base + [7], 4)
    s.run(50)
    r1 = s.submit(base + [7], 4)  # 25 tokens: 3 whole pages before position 24
    r2 = s.submit(base, 4)        # 24 tokens: 2 whole pages before position 23
    s.run(50)
    st = s.stats()
    assert st["prefix_tokens_skipped"] == 24 + 16
    assert s.poll(r1).tokens == s.poll(r0).tokens == greedy(base + [7], 4)
    assert s.poll(r2).tokens == greedy(base, 4)
    assert not eng.errors


def test_prefix_cache_lru_eviction_frees_pages():
    eng, s = make(pages=64, ps=8, prefix_cache_capacity=2)
    for i in range(3):
        s.submit(prompt(80 + i, 17), 2)  # 2 whole pages each
        s.run(20)
        assert s.cache_pages() <= 2
    assert s.cache_pages() == 2
    assert eng.free_pages() == [62, 62]
    # the two most recent pages are the cached ones: the third prompt hits, the first misses
    r = s.submit(prompt(82, 17), 2)
    s.run(20)
    assert s.stats()["prefix_cache_hits"] == 1
    s.submit(prompt(80, 17), 2)
    s.run(20)
    assert s.stats()["prefix_cache_hits"] == 1


def test_abort_and_errors():
    eng, s = make(max_running_requests=1)
    a = s.submit(prompt(90, 9), 50)
    b = s.submit(prompt(91, 9), 50)
    s.step()
    s.abort(a)
    assert s.poll(a).status == RequestStatus.ABORTED and s.poll(a).finish_reason == "cancelled"
    s.abort(b)
    assert s.poll(b).status == RequestStatus.ABORTED
    assert s.num_running() == 0 and s.num_waiting() == 0
    assert eng.free_pages() == [64, 64]
    assert s.stats()["requests_aborted"] == 2
    with pytest.raises(VeloxError, match="Empty prompt"):
        s.submit([], 4)
    with pytest.raises(VeloxError, match="at least 2 tokens"):
        s.submit([5], 4)
    with pytest.raises(VeloxError, match="still waiting or running"):
        s.release(s.submit(prompt(92, 4), 4))
    with pytest.raises(VeloxError, match="draft_k"):
        make(draft_k=0)


def test_temperatures_run_in_separate_rounds_with_request_streams():
    eng, s = make()
    p = prompt(100, 6)
    ids = [s.submit(p, 5, temperature=t) for t in (0.0, 0.7, 0.0, 0.7)]
    seen = {}
    orig = eng.add_state

    def add_state(*a):
        sid = orig(*a)
        seen[sid] = (a[5], a[6])
        return sid

    eng.add_state = add_state
    s.run(50)
    assert all(s.poll(r).tokens == greedy(p, 5) for r in ids)
    assert sorted(v[0] for v in seen.values()) == ids  # stream = request id
    assert {round(v[1], 3) for v in seen.values()} == {0.0, 0.7}
    assert not eng.errors


def test_owner_destruction_closes_the_scheduler_first():
    """Destroying a scheduler frees its live states through the engine, so an
    engine (or page pool) that goes first must close the schedulers bound to
    it: velox_amd.engine.close_dependents, which SpecEngine and PagedKvCache
    call before destroying themselves (Python finalises one garbage cycle,
    and whatever is left at exit, in no set order)."""
    import gc

    from velox_amd.engine import close_dependents

    class OwnedToy(ToyEngine):
        def __init__(self):
            super().__init__()
            self._dependents = []

    eng = OwnedToy()
    s = BatchScheduler(eng, (), SchedulerConfig(max_batch_tokens=512, prefix_cache_capacity=0, draft_k=4))
    assert eng._dependents == [s]
    s.submit(prompt(5, 20), 30)
    s.step()
    s.step()
    assert eng.states, "the request holds a live state"
    close_dependents(eng)  # what the owner's __del__ runs first
    assert s._h is None and not eng.states and eng.free_pages() == [64, 64]
    assert eng._dependents == []
    s.close()  # closing again is a no-op
    # a scheduler and its engine that die together in one cycle, in either order
    eng2 = OwnedToy()
    s2 = BatchScheduler(eng2, (), SchedulerConfig(prefix_cache_capacity=0, draft_k=4))
    s2.submit(prompt(6, 9), 5)
    s2.step()
    del s2, eng2
    gc.collect()
