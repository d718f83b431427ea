"""Round-by-round oracle check of the GPU spec engine ("lockstep").

The CPU oracle replays every speculative round of the GPU engine on the GPU's
own tokens (teacher forcing), so every round is compared even where the two
implementations' logits would, on their own, pick different argmaxes at a
near-tie.  Per round (src/paged/spec.rs:186-316):

* draft step i feeds [last, c0 .. c_{D-2}] at positions kv_len + i (the
  reference's draft-KV hole included, spec.rs:31-34): the oracle's draft
  logits must agree with the GPU's within 1e-2 + 1e-2|ref|;
* greedy: each candidate is the argmax (first index, spec.rs:356-366) of the
  GPU's own draft row, bit-exact; where the oracle's row picks another token
  the two must be a near-tie within that tolerance;
* stochastic: the round's uniforms equal Philox(seed; stream, round, i) and
  the candidates equal vxo.sample_draft on the GPU's draft logits, bit-exact;
* the verify forward over [last, c0 .. c_{D-1}] at kv_len: logits within
  tolerance; the accepted count and committed tokens equal vxo.accept_greedy
  (or vxo.accept_stochastic with the same uniforms) on the GPU's verify
  logits, bit-exact; greedy decisions the oracle's own logits would change
  must sit on a near-tie;
* commit: kv_len += A + 1, last = the GPU's bonus token.

Test infrastructure only (imports the oracle).
"""
from __future__ import annotations

import os

import numpy as np

import vxo
from refgen import assert_allclose_elementwise

# north_star: logits within atol 1e-2 + rtol 1e-2 (at the benchmark configs'
# logit scale, |logit| ~ 200).  Mirrors built with a looser atol say why.
ATOL = RTOL = 1e-2


def oracle_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "") or min(16, os.cpu_count() or 8))


def assert_near_tie(row: np.ndarray, chosen: int, what: str, atol: float, rtol: float) -> None:
    """The oracle's value at the GPU's choice is within the logit tolerance of
    the oracle row's maximum."""
    top = float(row.max())
    gap = top - float(row[chosen])
    assert gap <= 2 * (atol + rtol * abs(top)), f"{what}: GPU chose {chosen} ({row[chosen]}) but the oracle's " \
                                                f"max is {int(np.argmax(row))} ({top}); not a near-tie"


class Lockstep:
    """Oracle mirror of a GPU SpecEngine: same model weights (bf16 model
    semantics), its own page pools, driven by the GPU's decisions."""

    def __init__(self, cfg: dict, weights: dict, draft_layers: int, max_tokens: int, n_seqs: int, ps: int = 16,
                 temperature: float = 0.0, seed: int = 0, threads: int | None = None, fix_hole: bool = False,
                 atol: float | None = None, noise_ref: bool = False):
        from velox_amd import synth

        th = threads or oracle_threads()
        wt = synth.as_model_dtype(weights, "bf16")
        ocfg = dict(cfg, dtype=vxo.BF16)
        self.target = vxo.Model(ocfg, wt, threads=th)
        self.draft = vxo.Model(ocfg, wt, n_layers=draft_layers, threads=th)
        # noise_ref: the same weights with f32 activations (no bf16 rounding
        # at the op outputs), fed the same tokens, measure the bf16 model's
        # own rounding noise on every compared forward
        self.noise = None
        if noise_ref:
            fcfg = dict(cfg, dtype=vxo.F32)
            self.noise = (vxo.Model(fcfg, wt, threads=th), vxo.Model(fcfg, wt, n_layers=draft_layers, threads=th))
        del wt
        self.cfg = cfg
        self.ps = ps
        self.nb = (max_tokens + ps - 1) // ps
        L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
        self.tpages = vxo.Pages(L, HK, D, ps, self.nb * n_seqs + 1)
        self.dpages = vxo.Pages(draft_layers, HK, D, ps, self.nb * n_seqs + 1)
        if noise_ref:  # allocated in the same order: same page ids as the bf16 mirror
            self.noise_pages = (vxo.Pages(L, HK, D, ps, self.nb * n_seqs + 1),
                                vxo.Pages(draft_layers, HK, D, ps, self.nb * n_seqs + 1))
        self.temperature = temperature
        self.seed = seed
        self.inv_t = float(np.float32(1.0) / np.float32(temperature)) if temperature > 0 else 0.0
        self.fix_hole = fix_hole
        self.atol = ATOL if atol is None else atol
        self.seqs: list[dict] = []
        self.rounds_checked = 0

    def prefill(self, prompts, streams=None) -> None:
        """spec.rs:131-182: both models on prompt[..len-1]; logits discarded.
        streams: the Philox stream of each sequence (default: its index)."""
        ids, tsl, dsl = [], [], []
        for i, p in enumerate(prompts):
            p = np.asarray(p, np.uint32)
            s = {"tbt": self.tpages.alloc(self.nb), "dbt": self.dpages.alloc(self.nb), "kv_len": p.size - 1,
                 "last": int(p[-1]), "tokens": list(map(int, p)), "round": 0,
                 "stream": len(self.seqs) if streams is None else int(streams[i])}
            self.seqs.append(s)
            ids.append(p[:-1])
            tsl.append((p.size - 1, 0, s["tbt"]))
            dsl.append((p.size - 1, 0, s["dbt"]))
        ids = np.concatenate(ids)
        if self.noise is not None:
            for _ in prompts:
                self.noise_pages[0].alloc(self.nb)
                self.noise_pages[1].alloc(self.nb)
        self._forward(0, ids, tsl, False)
        self._forward(1, ids, dsl, False)
        print(f"[lockstep] oracle prefill of {len(prompts)} prompts done", flush=True)

    def _forward(self, which, ids, seqs, all_rows):
        """Oracle forward of the target (0) or the draft (1); with noise_ref
        also the f32-activation twin.  Returns (logits, atol): atol is the
        mirror's atol, or twice the largest bf16-vs-f32 logit gap of this
        forward if that is larger (the GPU may not stray further from the bf16
        oracle than the bf16 model strays from exact activations, with a
        factor 2 of headroom)."""
        model, pages = (self.target, self.tpages) if which == 0 else (self.draft, self.dpages)
        ref = vxo.forward(model, pages, ids, seqs, all_rows=all_rows)
        if self.noise is None:
            return ref, self.atol
        r32 = vxo.forward(self.noise[which], self.noise_pages[which], ids, seqs, all_rows=all_rows)
        return ref, max(self.atol, 2.0 * float(np.abs(ref - r32).max()))

    def check_round(self, tr: dict, outcomes, seq_index=None) -> None:
        """Replay one GPU round (tr = SpecEngine.last_round()) on the oracle
        and check it; seq_index maps the round's rows to this mirror's
        sequences (default: row b is sequence b).  outcomes: the engine's
        RoundOutcomes, or None when a caller (the scheduler) consumed them;
        its committed tokens are then checked through the token streams."""
        n, k = tr["n"], tr["k"]
        idx = list(range(n)) if seq_index is None else list(seq_index)
        S = [self.seqs[i] for i in idx]
        cand = tr["candidates"]
        r = self.rounds_checked
        stoch = tr["temperature"] > 0
        assert stoch == (self.temperature > 0)
        dl_g = tr.get("draft_logits")  # None: run the draft forwards, check nothing on them
        # ---- draft steps
        for i in range(k):
            ids = np.array([s["last"] if i == 0 else cand[b, i - 1] for b, s in enumerate(S)], np.uint32)
            ref, atol = self._forward(1, ids, [(1, s["kv_len"] + i, s["dbt"]) for s in S], False)
            if dl_g is None:
                continue
            assert_allclose_elementwise(f"round {r} draft step {i} logits", dl_g[:, i], ref, atol, RTOL)
            if not stoch:
                for b in range(n):
                    g = int(vxo.argmax(dl_g[b, i]))
                    assert cand[b, i] == g, f"round {r} seq {b} step {i}: candidate {cand[b, i]} is not the " \
                                            f"argmax {g} of the GPU's own draft row"
                    if int(vxo.argmax(ref[b])) != g:
                        assert_near_tie(ref[b], g, f"round {r} seq {b} draft step {i}", atol, RTOL)
        uni = None
        if stoch:
            for b, s in enumerate(S):
                assert int(tr["streams"][b]) == s["stream"], f"round {r} seq {b}: Philox stream {tr['streams'][b]}"
                assert int(tr["rounds"][b]) == s["round"], f"round {r} seq {b}: round counter {tr['rounds'][b]}"
            uni = np.concatenate([vxo.spec_uniforms(self.seed, int(tr["streams"][b]), int(tr["rounds"][b]), 1, k)
                                  for b in range(n)])
            if tr.get("uniforms") is not None:
                assert np.array_equal(tr["uniforms"], uni), f"round {r}: device Philox uniforms differ from the oracle's"
            if dl_g is not None:
                want = vxo.sample_draft(dl_g, uni, self.inv_t)
                assert np.array_equal(cand, want), f"round {r}: draft draws differ from the oracle on the GPU's logits"
        # ---- verify
        ids = np.concatenate([[s["last"]] + list(cand[b]) for b, s in enumerate(S)]).astype(np.uint32)
        ref, atol = self._forward(0, ids, [(k + 1, s["kv_len"], s["tbt"]) for s in S], True)
        ref = ref.reshape(n, k + 1, -1)
        vl_g = tr["verify_logits"]
        assert_allclose_elementwise(f"round {r} verify logits", vl_g, ref, atol, RTOL)
        if stoch:
            assert dl_g is not None, "a stochastic round is re-derived from its draft logits"
            acc, tok = vxo.accept_stochastic(vl_g, dl_g, cand, uni, self.inv_t)
        else:
            acc, tok = vxo.accept_greedy(vl_g, cand)
        for b in range(n if outcomes is not None else 0):
            o = outcomes[b]
            assert o.accepted == acc[b], f"round {r} seq {b}: accepted {o.accepted}, oracle on GPU logits {acc[b]}"
            assert list(o.committed_tokens) == list(map(int, tok[b, : acc[b] + 1])), \
                f"round {r} seq {b}: committed tokens differ"
        if not stoch:
            acc_o, tok_o = vxo.accept_greedy(ref, cand)
            for b in range(n):
                # the first row where the oracle's argmax departs from the GPU's
                for i in range(min(acc[b], acc_o[b]) + 1):
                    g = int(vxo.argmax(vl_g[b, i]))
                    if int(vxo.argmax(ref[b, i])) != g:
                        assert_near_tie(ref[b, i], g, f"round {r} seq {b} verify row {i}", atol, RTOL)
                        break
        # ---- commit (spec.rs:294-301)
        for b, s in enumerate(S):
            a = int(acc[b])
            if self.fix_hole and a == k:
                # opt-in draft-hole fix: c[D-1] is fed to the draft at kv_len + D
                self._forward(1, np.array([cand[b, k - 1]], np.uint32), [(1, s["kv_len"] + k, s["dbt"])], False)
            s["kv_len"] += a + 1
            s["last"] = int(tok[b, a])
            s["tokens"] += list(map(int, tok[b, : a + 1]))
            s["round"] += 1
        self.rounds_checked += 1
        print(f"[lockstep] round {r} checked: accepted {[int(a) for a in acc]}", flush=True)
