"""Continuous-batching speculative scheduler over the C ABI (vx_sched_*).

Mirrors the reference's `BatchScheduler` (src/paged/scheduler.rs:37-534):
`SchedulerConfig`, `submit`, a step loop, `stats`; requests are tokenised
prompts (the chat template and tokenizer stay with the caller).  Each step
admits waiting requests (FCFS, pages reserved for the whole sequence,
prefix-cache lookup), then runs prefill chunks and one speculative round for
the decoding requests under `max_batch_tokens`.  The policy lives in the
native library; this module only binds it.

`PyBackend` lets any Python object serve as the engine the scheduler drives
(`vx_sched_create_with_backend`): implement its methods with the semantics of
the vx_spec_* calls.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from ._lib import (ADD_STATE_FN, FREE_STATE_FN, PREFILL_CHUNK_FN, REF_FN, STATE_PAGES_FN, STEP_FN, SchedBackend,
                   SchedConfig, SchedStats, check, lib)


@dataclass
class SchedulerConfig:
    """SchedulerConfig (scheduler.rs:37-59) plus the draft length."""
    max_running_requests: int = 64
    max_batch_tokens: int = 512
    prefix_cache_capacity: int = 256
    draft_k: int = 4

    def _c(self) -> SchedConfig:
        return SchedConfig(self.max_running_requests, self.max_batch_tokens, self.prefix_cache_capacity,
                           self.draft_k)


class RequestStatus(IntEnum):
    """RequestStatus (request.rs:29-40)."""
    WAITING = 0
    RUNNING = 1
    FINISHED = 2
    ABORTED = 3


FINISH_REASONS = {0: None, 1: "stop", 2: "length", 3: "cancelled"}


@dataclass
class RequestResult:
    id: int
    tokens: list
    status: RequestStatus
    finish_reason: str | None


class BatchScheduler:
    """BatchScheduler over a SpecEngine (or a PyBackend)."""

    def __init__(self, engine, eos_token_ids=(), cfg: SchedulerConfig | None = None, stream=None):
        self.cfg = cfg or SchedulerConfig()
        eos = (C.c_uint32 * max(len(eos_token_ids), 1))(*eos_token_ids)
        h = C.c_void_p()
        c = self.cfg._c()
        if isinstance(engine, PyBackend):
            check(lib.vx_sched_create_with_backend(C.byref(engine._struct), C.byref(c), eos, len(eos_token_ids),
                                                   C.byref(h)))
        else:
            if stream is None:
                import torch

                stream = torch.cuda.current_stream().cuda_stream
            check(lib.vx_sched_create(engine._h, C.byref(c), eos, len(eos_token_ids), stream, C.byref(h)))
        self._h = h
        self._engine = engine  # the engine must outlive the scheduler
        # destroying the scheduler frees its states through the engine and
        # the engine's page pools: they close it before they go
        self._owners = [o for o in (engine, *getattr(engine, "_refs", ())) if hasattr(o, "_dependents")]
        for o in self._owners:
            o._dependents.append(self)

    def submit(self, prompt_tokens, max_tokens: int, temperature: float = 0.0, stream: int | None = None) -> int:
        """scheduler.rs:147-185; returns the request id."""
        a = np.ascontiguousarray(prompt_tokens, np.uint32)
        rid = C.c_int64()
        check(lib.vx_sched_submit(self._h, a.ctypes.data_as(C.POINTER(C.c_uint32)), a.size, max_tokens,
                                  temperature, -1 if stream is None else stream, C.byref(rid)))
        return rid.value

    def step(self) -> int:
        """One admit + step; returns the new tokens fed to the models."""
        n = C.c_int64()
        check(lib.vx_sched_step(self._h, C.byref(n)))
        return n.value

    def run(self, max_steps: int | None = None) -> int:
        """Steps until nothing waits or runs (the reference's run loop,
        scheduler.rs:189-215, without the idle sleep); returns the steps."""
        steps = 0
        while self.num_waiting() + self.num_running() > 0:
            if max_steps is not None and steps >= max_steps:
                break
            self.step()
            steps += 1
        return steps

    def poll(self, rid: int) -> RequestResult:
        n, status, fin = C.c_int64(), C.c_int(), C.c_int()
        check(lib.vx_sched_poll(self._h, rid, None, 0, C.byref(n), C.byref(status), C.byref(fin)))
        buf = (C.c_uint32 * max(n.value, 1))()
        check(lib.vx_sched_poll(self._h, rid, buf, n.value, C.byref(n), C.byref(status), C.byref(fin)))
        return RequestResult(rid, [buf[i] for i in range(n.value)], RequestStatus(status.value),
                             FINISH_REASONS[fin.value])

    def abort(self, rid: int) -> None:
        check(lib.vx_sched_abort(self._h, rid))

    def release(self, rid: int) -> None:
        check(lib.vx_sched_release(self._h, rid))

    def stats(self) -> dict:
        s = SchedStats()
        check(lib.vx_sched_get_stats(self._h, C.byref(s)))
        return {name: getattr(s, name) for name, _ in SchedStats._fields_}

    def num_waiting(self) -> int:
        return lib.vx_sched_num_waiting(self._h)

    def num_running(self) -> int:
        return lib.vx_sched_num_running(self._h)

    def cache_pages(self) -> int:
        return lib.vx_sched_cache_pages(self._h)

    def close(self, _destroy=lib.vx_sched_destroy) -> None:  # bound now: module globals may be gone at exit
        if getattr(self, "_h", None):
            _destroy(self._h)
            self._h = None
        for o in getattr(self, "_owners", ()):
            if self in o._dependents:
                o._dependents.remove(self)
        self._owners = []

    def __del__(self):
        self.close()


class PyBackend:
    """Base class for an engine written in Python.  Subclasses implement:

    add_state(prompt, cached_tokens, target_pages, draft_pages, reserve_tokens, stream_id, temperature) -> int
    prefill_chunk(states, n_tokens) -> None
    step(states, draft_k) -> list of (accepted, committed_tokens)
    state_pages(state, which) -> list of page ids
    free_state(state) -> None
    incref(which, pages) / decref(which, pages) -> None

    A raised exception becomes a non-zero return code (for add_state: "the
    pools cannot hold it")."""

    def __init__(self, page_size: int):
        self.page_size = page_size
        self.errors = []

        def guard(fn, fail):
            def w(*a):
                try:
                    return fn(*a)
                except Exception as e:  # reported to the scheduler as a return code
                    self.errors.append(e)
                    return fail
            return w

        def add_state(_, prompt, n, cached, tp, dp, reserve, stream_id, temperature, out):
            npg = cached // page_size
            s = self.add_state([prompt[i] for i in range(n)], cached, [tp[i] for i in range(npg)],
                               [dp[i] for i in range(npg)], reserve, stream_id, temperature)
            out[0] = s
            return 0

        def prefill_chunk(_, states, n_tokens, n):
            self.prefill_chunk([states[i] for i in range(n)], [n_tokens[i] for i in range(n)])
            return 0

        def step(_, states, n, k, outcomes, committed):
            res = self.step([states[i] for i in range(n)], k)
            for b, (acc, toks) in enumerate(res):
                outcomes[b].accepted = acc
                outcomes[b].n_committed = len(toks)
                outcomes[b].stop = 0
                for i, t in enumerate(toks):
                    committed[b * (k + 1) + i] = t
            return 0

        def state_pages(_, s, which, out, cap):
            pg = self.state_pages(s, which)
            for i in range(min(cap, len(pg))):
                out[i] = pg[i]
            return len(pg)

        def free_state(_, s):
            self.free_state(s)

        def incref(_, which, pages, n):
            self.incref(which, [pages[i] for i in range(n)])

        def decref(_, which, pages, n):
            self.decref(which, [pages[i] for i in range(n)])

        self._fns = (ADD_STATE_FN(guard(add_state, 1)), PREFILL_CHUNK_FN(guard(prefill_chunk, 1)),
                     STEP_FN(guard(step, 1)), STATE_PAGES_FN(guard(state_pages, -1)),
                     FREE_STATE_FN(guard(free_state, None)), REF_FN(guard(incref, None)),
                     REF_FN(guard(decref, None)))
        self._struct = SchedBackend(None, page_size, *self._fns)
