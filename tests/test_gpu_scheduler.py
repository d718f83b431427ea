"""Continuous-batching scheduler over the GPU engine (vx_sched_create on a
vx_spec): chunked prefill, prefix-shared pages and speculative rounds on a
tiny Qwen3-shaped model.

Greedy speculative decoding emits the target model's greedy continuation
(spec.rs:266-301), so every generated token is checked against the CPU
oracle's target logits over the request's own sequence (teacher forcing, one
oracle forward per request, no pages shared): the token must be the
oracle's argmax, or within the logit tolerance of it (1e-2 + 1e-2|max|, the
north_star bound; two implementations may order a near-tie differently).
A wrong block table or a wrongly shared page gives unrelated logits and
fails this at once.
"""
import numpy as np
import pytest

import vxo

pytestmark = pytest.mark.gpu

PS = 16


def build(cfg, seed, draft_layers, pages, temperature=0.0):
    from velox_amd import engine, synth

    w = synth.host_weights(cfg, seed)
    t = engine.PagedQwen3(cfg, w)
    d = engine.PagedQwen3(cfg, w, n_layers=draft_layers)
    tp = engine.PagedKvCache(cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"], PS, pages)
    dp = engine.PagedKvCache(draft_layers, cfg["n_kv_heads"], cfg["head_dim"], PS, pages)
    e = engine.SpecEngine(t, tp, d, dp, temperature=temperature, sample_seed=5, fix_draft_hole=True)
    return w, e, tp, dp


def check_greedy(cfg, w, prompt, gen):
    from velox_amd import synth

    wt = synth.as_model_dtype(w, "bf16")
    model = vxo.Model(dict(cfg, dtype=vxo.BF16), wt, threads=8)
    seq = np.concatenate([np.asarray(prompt, np.uint32), np.asarray(gen[:-1], np.uint32)])
    pages = vxo.Pages(cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"], PS, -(-seq.size // PS))
    bt = pages.alloc(-(-seq.size // PS))
    logits = vxo.forward(model, pages, seq, [(seq.size, 0, bt)], all_rows=True)
    loose = 0
    for i, t in enumerate(gen):
        row = logits[len(prompt) - 1 + i]
        top = row.max()
        if int(np.argmax(row)) != t:
            assert row[t] >= top - 2 * (1e-2 + 1e-2 * abs(top)), f"token {i}: {t} is not a greedy choice"
            loose += 1
    return loose


def test_scheduler_greedy_prefix_sharing_and_chunks(cuda):
    from velox_amd import synth
    from velox_amd.scheduler import BatchScheduler, RequestStatus, SchedulerConfig

    cfg = synth.tiny_config(layers=2)
    w, e, tp, dp = build(cfg, 21, 1, pages=256)
    rng = np.random.default_rng(3)
    shared = [rng.integers(0, cfg["vocab"], 48) for _ in range(2)]
    prompts = [np.concatenate([shared[g], rng.integers(0, cfg["vocab"], 5 + 7 * i)]) for g in range(2)
               for i in range(3)]
    prompts.append(rng.integers(0, cfg["vocab"], 70))
    s = BatchScheduler(e, (), SchedulerConfig(max_running_requests=8, max_batch_tokens=40,
                                              prefix_cache_capacity=64, draft_k=3))
    ids = [s.submit(p, 14) for p in prompts]
    steps = s.run(400)
    st = s.stats()
    print(f"[sched] steps {steps} stats {st}", flush=True)
    assert st["requests_completed"] == len(prompts)
    assert st["prefix_cache_hits"] >= 4 and st["prefix_tokens_skipped"] >= 4 * 48
    assert st["prefill_tokens"] == sum(len(p) - 1 for p in prompts) - st["prefix_tokens_skipped"]
    loose = 0
    for rid, p in zip(ids, prompts):
        r = s.poll(rid)
        assert r.status == RequestStatus.FINISHED and len(r.tokens) == 14
        loose += check_greedy(cfg, w, p, r.tokens)
    assert loose <= 2, f"{loose} tokens only within tolerance of the argmax"
    held = s.cache_pages()
    assert tp.num_free_pages() == 256 - held and dp.num_free_pages() == 256 - held
    s.close()
    assert tp.num_free_pages() == 256 and dp.num_free_pages() == 256


def test_scheduler_stochastic_lockstep(cuda):
    """Config 4's sampling path through the scheduler: T = 0.7, per-request
    Philox streams (the request id), k = 4, chunked prefill and prefix-shared
    pages.  Every speculative round the scheduler runs is replayed by the
    oracle mirror (tests/lockstep.py) on the GPU's own logits: uniforms,
    draft draws and accept / residual decisions bit-exact, logits within
    tolerance; each request's tokens equal the mirror's committed stream."""
    from velox_amd import engine, synth
    from velox_amd.scheduler import BatchScheduler, RequestStatus, SchedulerConfig

    from lockstep import Lockstep
    from test_oracle_model import zero_mean

    cfg = synth.tiny_config(layers=4)
    w = zero_mean(synth.host_weights(cfg, 23))
    t, d = engine.PagedQwen3(cfg, w), engine.PagedQwen3(cfg, w, n_layers=2)
    HK, D = cfg["n_kv_heads"], cfg["head_dim"]
    e = engine.SpecEngine(t, engine.PagedKvCache(4, HK, D, PS, 192), d, engine.PagedKvCache(2, HK, D, PS, 192),
                          temperature=0.7, sample_seed=5, fix_draft_hole=True)
    e.set_tracing(True)
    rng = np.random.default_rng(9)
    shared = rng.integers(0, cfg["vocab"], 32)
    prompts = [np.concatenate([shared, rng.integers(0, cfg["vocab"], 3 + 5 * i)]) for i in range(3)]
    prompts += [rng.integers(0, cfg["vocab"], n) for n in (9, 41)]
    new = 12
    s = BatchScheduler(e, (), SchedulerConfig(max_batch_tokens=48, prefix_cache_capacity=32, draft_k=4))
    ids = [s.submit(p, new, temperature=0.7) for p in prompts]
    # zero-mean weights: logits at |logit| ~ 1, compared against the bf16
    # model's own measured rounding noise (see test_gpu_engine.run_lockstep)
    ls = Lockstep(cfg, w, 2, max(len(p) for p in prompts) + new + 12, len(prompts), temperature=0.7, seed=5,
                  fix_hole=True, noise_ref=True)
    ls.prefill(prompts, streams=ids)
    index_of = {rid: i for i, rid in enumerate(ids)}
    serial, steps = 0, 0
    while s.num_waiting() + s.num_running() > 0 and steps < 300:
        s.step()
        steps += 1
        tr = e.last_round()
        if tr is not None and tr["serial"] != serial:
            assert tr["serial"] == serial + 1, "more than one round per scheduler step"
            serial = tr["serial"]
            ls.check_round(tr, None, seq_index=[index_of[int(x)] for x in tr["streams"]])
    st = s.stats()
    assert st["requests_completed"] == len(prompts) and st["prefix_cache_hits"] >= 2
    assert ls.rounds_checked == serial > 0
    for rid, p in zip(ids, prompts):
        r = s.poll(rid)
        assert r.status == RequestStatus.FINISHED and len(r.tokens) == new
        assert r.tokens == ls.seqs[index_of[rid]]["tokens"][len(p): len(p) + new], f"request {rid}: tokens differ"
    s.close()


def test_scheduler_stochastic_is_deterministic(cuda):
    """Temperature 0.7 with per-request Philox streams: the same submissions
    give the same tokens on a fresh engine."""
    from velox_amd import synth
    from velox_amd.scheduler import BatchScheduler, SchedulerConfig

    cfg = synth.tiny_config(layers=2)
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, cfg["vocab"], n) for n in (9, 33, 20)]
    outs = []
    for _ in range(2):
        _, e, _, _ = build(cfg, 22, 1, pages=128, temperature=0.7)
        s = BatchScheduler(e, (), SchedulerConfig(max_batch_tokens=64, prefix_cache_capacity=0, draft_k=4))
        ids = [s.submit(p, 10, temperature=0.7) for p in prompts]
        s.run(200)
        outs.append([s.poll(r).tokens for r in ids])
        s.close()
    assert outs[0] == outs[1]
    assert all(len(t) == 10 and all(0 <= x < cfg["vocab"] for x in t) for t in outs[0])
