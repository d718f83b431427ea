"""Engine-level mirror of the reference's paged KV cache, Qwen3 model and
speculative-decoding engine (src/paged/pages.rs, qwen3.rs, spec.rs), driving the
C++/HIP engine through the C ABI.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import synth
from ._lib import (F16, LayerHost, QLinearHost, QwenConfig, RoundOutcome, RoundTrace, SeqSlice, StepProfile,
                   VeloxError, WeightsHost, check, lib)


def close_dependents(owner) -> None:
    """Close the native objects whose destruction reaches into `owner` (a
    scheduler frees its states' pages through the engine) before `owner`
    itself goes.  Python finalises objects of one garbage cycle in no set
    order (PEP 442), and at interpreter exit whatever is left goes that way,
    so the owner closes them first; a closed dependent is a no-op."""
    for d in list(getattr(owner, "_dependents", ())):
        d.close()


class PagedKvCache:
    """pages.rs:82-255: per-layer K/V pools [P, h_kv, page_size, d] (f16 on the
    device), LIFO free list (page 0 first), refcounts, all-or-nothing alloc."""

    def __init__(self, num_layers, num_kv_heads, head_dim, page_size, num_pages, dtype=F16):
        self._dependents = []  # native objects that touch these pools when destroyed
        h = C.c_void_p()
        check(lib.vx_pages_create(num_layers, num_kv_heads, head_dim, page_size, num_pages, dtype,
                                  C.byref(h)))
        self._h = h
        self.num_layers, self.num_kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.page_size, self.num_pages = page_size, num_pages

    @staticmethod
    def total_bytes(num_layers, num_kv_heads, head_dim, page_size, num_pages, elem_bytes=2):
        """PagedKvConfig::total_bytes (pages.rs:45-59)."""
        return num_layers * 2 * num_pages * num_kv_heads * page_size * head_dim * elem_bytes

    def alloc(self, n):
        out = (C.c_uint32 * max(n, 1))()
        if lib.vx_pages_alloc(self._h, n, out) != 0:
            return None
        return [out[i] for i in range(n)]

    def incref_pages(self, pages):
        arr = (C.c_uint32 * len(pages))(*pages)
        lib.vx_pages_incref(self._h, arr, len(pages))

    def free_pages(self, pages):
        arr = (C.c_uint32 * max(len(pages), 1))(*pages)
        lib.vx_pages_free(self._h, arr, len(pages))

    def num_free_pages(self):
        return lib.vx_pages_num_free(self._h)

    def page_refcount(self, page):
        return lib.vx_pages_refcount(self._h, page)

    def layer_pool_ptr(self, layer, kv):
        return lib.vx_pages_pool(self._h, layer, kv)

    def __del__(self, _destroy=lib.vx_pages_destroy, _close=close_dependents):  # bound now: globals may be gone at exit
        _close(self)
        if getattr(self, "_h", None):
            _destroy(self._h)
            self._h = None


class PagedQwen3:
    """PagedQwen3 (qwen3.rs:943-1037) from host weights in the MLX int4 format
    (the dict produced by velox_amd.synth.host_weights)."""

    def __init__(self, cfg: dict, weights: dict, n_layers: int | None = None):
        self.cfg = dict(cfg)
        L = cfg["layers"] if n_layers is None else n_layers
        self.cfg["layers"] = L
        keep = []

        def ptr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        def f16(a):
            return ptr(np.asarray(a, np.float16).view(np.uint16), np.uint16)

        def ql(p):
            return QLinearHost(ptr(weights[p + ".qweight"], np.uint32), f16(weights[p + ".scales"]),
                               f16(weights[p + ".biases"]))

        layers = (LayerHost * L)()
        for i in range(L):
            p = f"layers.{i}."
            layers[i] = LayerHost(f16(weights[p + "ln1"]), f16(weights[p + "ln2"]), f16(weights[p + "q_norm"]),
                                  f16(weights[p + "k_norm"]), ql(p + "q"), ql(p + "k"), ql(p + "v"),
                                  ql(p + "o"), ql(p + "gate"), ql(p + "up"), ql(p + "down"))
        w = WeightsHost(f16(weights["embed"]), C.cast(layers, C.c_void_p), f16(weights["norm"]), ql("lm_head"))
        c = self.cfg
        qc = QwenConfig(c["vocab"], c["hidden"], c["inter"], cfg["layers"], c["n_heads"], c["n_kv_heads"],
                        c["head_dim"], c["max_pos"], c["group_size"], c["rope_theta"], c["rms_eps"])
        h = C.c_void_p()
        check(lib.vx_model_create(C.byref(qc), C.byref(w), L, C.byref(h)))
        self._h = h
        del keep

    @classmethod
    def synthetic(cls, cfg: dict, seed: int, n_layers: int | None = None):
        return cls(cfg, synth.host_weights(cfg, seed, n_layers), n_layers)

    def config(self):
        return self.cfg

    def _run(self, pages, input_ids, seqs, all_rows, tree_parents, stream):
        import torch

        if tree_parents is not None:
            for nt, _, _ in seqs:
                if nt != len(tree_parents):
                    raise VeloxError(f"forward: a tree of {len(tree_parents)} nodes needs new_tokens == "
                                     f"{len(tree_parents)} in every sequence (got {nt})")

        ids = np.ascontiguousarray(input_ids, np.uint32)
        sl = (SeqSlice * len(seqs))()
        keep = []
        for i, (nt, off, bt) in enumerate(seqs):
            bt = np.ascontiguousarray(bt, np.uint32)
            keep.append(bt)
            sl[i] = SeqSlice(nt, off, bt.ctypes.data, bt.size)
        rows = ids.size if all_rows else len(seqs)
        logits = torch.empty((rows, self.cfg["vocab"]), dtype=torch.bfloat16, device="cuda")
        tp = None
        if tree_parents is not None:
            tp_arr = (C.c_int32 * len(tree_parents))(*[int(x) for x in tree_parents])
            tp = C.cast(tp_arr, C.POINTER(C.c_int32))
        st = torch.cuda.current_stream().cuda_stream if stream is None else stream
        check(lib.vx_forward(self._h, pages._h, ids.ctypes.data_as(C.POINTER(C.c_uint32)), sl, len(seqs),
                             1 if all_rows else 0, tp, logits.data_ptr(), st))
        return logits

    def forward(self, pages, input_ids, seqs, stream=None):
        """qwen3.rs:994-1017: logits of the last new token of each sequence.
        seqs: list of (new_tokens, kv_offset, block_table)."""
        return self._run(pages, input_ids, seqs, False, None, stream)

    def forward_all(self, pages, input_ids, seqs, tree_parents=None, stream=None):
        """qwen3.rs:1023-1036: logits of every input position."""
        return self._run(pages, input_ids, seqs, True, tree_parents, stream)

    def __del__(self, _destroy=lib.vx_model_destroy):  # bound now: module globals may be gone at exit
        if getattr(self, "_h", None):
            _destroy(self._h)
            self._h = None


@dataclass
class RoundOutcome_:
    committed_tokens: list
    accepted: int
    stop: bool


@dataclass
class SpecState:
    """spec.rs:110-124 (the engine owns the block tables; `id` names the state)."""
    id: int
    engine: "SpecEngine" = field(repr=False)

    @property
    def kv_len(self):
        return lib.vx_spec_state_kv_len(self.engine._h, self.id)

    @property
    def tokens(self):
        n = lib.vx_spec_state_num_tokens(self.engine._h, self.id)
        out = (C.c_uint32 * max(n, 1))()
        check(lib.vx_spec_state_tokens(self.engine._h, self.id, out, n))
        return [out[i] for i in range(n)]


class SpecEngine:
    """SpecEngine (spec.rs:59-323).  step() runs any number of states in one
    batched round; temperature 0 is the reference's greedy mode."""

    def __init__(self, target: PagedQwen3, target_pages: PagedKvCache, draft: PagedQwen3,
                 draft_pages: PagedKvCache, temperature=0.0, sample_seed=0, fix_draft_hole=False):
        self._dependents = []
        h = C.c_void_p()
        check(lib.vx_spec_create(target._h, target_pages._h, draft._h, draft_pages._h, temperature, sample_seed,
                                 1 if fix_draft_hole else 0, C.byref(h)))
        self._h = h
        self._refs = (target, target_pages, draft, draft_pages)
        self.vocab_size = target.cfg["vocab"]

    def prefill(self, prompt):
        return self.prefill_batch([prompt])[0]

    def prefill_batch(self, prompts):
        arrs = [np.ascontiguousarray(p, np.uint32) for p in prompts]
        ptrs = (C.POINTER(C.c_uint32) * len(arrs))(*[a.ctypes.data_as(C.POINTER(C.c_uint32)) for a in arrs])
        lens = (C.c_int64 * len(arrs))(*[a.size for a in arrs])
        first = C.c_int64()
        check(lib.vx_spec_prefill(self._h, ptrs, lens, len(arrs), C.byref(first)))
        return [SpecState(first.value + i, self) for i in range(len(arrs))]

    def step(self, state, draft_k, eos_id=None):
        return self.step_batch([state], draft_k, eos_id)[0]

    def step_batch(self, states, draft_k, eos_id=None, stream=None):
        import torch

        n = len(states)
        ids = (C.c_int64 * n)(*[s.id for s in states])
        outs = (RoundOutcome * n)()
        com = (C.c_uint32 * (n * (draft_k + 1)))()
        st = torch.cuda.current_stream().cuda_stream if stream is None else stream
        check(lib.vx_spec_step(self._h, ids, n, draft_k, -1 if eos_id is None else eos_id, outs, com, st))
        res = []
        for b in range(n):
            o = outs[b]
            res.append(RoundOutcome_([com[b * (draft_k + 1) + i] for i in range(o.n_committed)], o.accepted,
                                     bool(o.stop)))
        return res

    def last_trace(self, n, draft_k):
        cand = np.zeros((n, draft_k), np.uint32)
        logits = np.zeros((n, draft_k + 1, self.vocab_size), np.float32)
        check(lib.vx_spec_last_trace(self._h, cand.ctypes.data_as(C.POINTER(C.c_uint32)),
                                     logits.ctypes.data_as(C.POINTER(C.c_float))))
        return cand, logits

    def set_tracing(self, enable: bool):
        """Keep every draft step's logits so last_round() can return them."""
        check(lib.vx_spec_set_tracing(self._h, 1 if enable else 0))

    def last_round(self) -> dict | None:
        """Everything the last step decided on: state ids, the Philox counter
        words (stream, round) of its uniforms, the candidates, the verify and
        draft logits (as f32 copies of the bf16 device values) and the
        uniforms.  None before the first step."""
        info = RoundTrace()
        check(lib.vx_spec_last_trace_info(self._h, C.byref(info), None, None, None))
        if info.serial == 0:
            return None
        n, k, v = info.n, info.draft_k, info.vocab
        ids = np.zeros(n, np.int64)
        streams = np.zeros(n, np.uint32)
        rounds = np.zeros(n, np.uint32)
        check(lib.vx_spec_last_trace_info(self._h, C.byref(info), ids.ctypes.data_as(C.POINTER(C.c_int64)),
                                          streams.ctypes.data_as(C.POINTER(C.c_uint32)),
                                          rounds.ctypes.data_as(C.POINTER(C.c_uint32))))
        cand, logits = self.last_trace(n, k)
        uni = np.zeros((n, k + 1, 4), np.float32)
        dl = np.zeros((n, k, v), np.float32) if info.has_draft_logits else None
        check(lib.vx_spec_last_trace_draft(self._h, None if dl is None else dl.ctypes.data_as(C.POINTER(C.c_float)),
                                           uni.ctypes.data_as(C.POINTER(C.c_float))))
        return {"serial": info.serial, "n": n, "k": k, "temperature": info.temperature, "state_ids": ids,
                "streams": streams, "rounds": rounds, "candidates": cand, "verify_logits": logits,
                "draft_logits": dl, "uniforms": uni}

    def set_profiling(self, enable, phases_only: bool = False):
        """Per-kernel HIP-event timing (enable), or only the draft / verify /
        accept phase boundaries (phases_only: the kernels run undisturbed)."""
        check(lib.vx_spec_set_profiling(self._h, (2 if phases_only else 1) if enable else 0))

    def last_profile(self) -> dict:
        p = StepProfile()
        check(lib.vx_spec_last_profile(self._h, C.byref(p)))
        names = ("qmm", "attention", "other")
        out = {"draft_ms": p.draft_ms, "verify_ms": p.verify_ms, "accept_ms": p.accept_ms}
        for ph in ("verify", "draft"):
            for i, nm in enumerate(names):
                out[f"{ph}_{nm}_ms"] = getattr(p, f"{ph}_kernel_ms")[i]
                out[f"{ph}_{nm}_bytes"] = getattr(p, f"{ph}_kernel_bytes")[i]
                out[f"{ph}_{nm}_launches"] = getattr(p, f"{ph}_kernel_launches")[i]
        return out

    def free(self, state):
        lib.vx_spec_free(self._h, state.id)

    def __del__(self, _destroy=lib.vx_spec_destroy, _close=close_dependents):  # bound now: globals may be gone at exit
        _close(self)
        if getattr(self, "_h", None):
            _destroy(self._h)
            self._h = None


__all__ = ["PagedKvCache", "PagedQwen3", "SpecEngine", "SpecState", "VeloxError"]
