"""CPU checks of the oracle's model forward and spec loop (oracle/vxo.c
vxo_forward / vxo_spec_*), against an independent float64 dense restatement of
Qwen3 (no paging, full causal softmax) and against invariants of speculative
decoding (spec.rs module docs: greedy spec decoding equals greedy decoding)."""
import numpy as np
import pytest

import vxo
from refgen import dequant
from velox_amd import synth


def zero_mean(w, seed=0):
    """Synthetic weights with biases -7.5*s (+ small noise) so that E[w] = 0
    and attention / token choices depend on the inputs."""
    rng = np.random.default_rng(seed)
    out = dict(w)
    for k, v in w.items():
        if k.endswith(".biases"):
            s = w[k[:-7] + ".scales"].astype(np.float32)
            out[k] = (-7.5 * s + rng.normal(0, 1e-3, size=s.shape)).astype(np.float16)
    return out


def dense_forward(cfg, w, ids):
    """float64 Qwen3 over one sequence (qwen3.rs:418-480, 932-939, 1023-1036)."""
    H, D, HQ, HK = cfg["hidden"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    eps = cfg["rms_eps"]
    n = len(ids)

    def rms(x, g):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g

    def lin(x, p):
        return x @ dequant(w[p + ".qweight"], w[p + ".scales"], w[p + ".biases"]).T

    t = np.arange(n)[:, None]
    inv = 1.0 / (cfg["rope_theta"] ** (np.arange(0, D, 2) / D))
    cos, sin = np.cos(t * inv), np.sin(t * inv)

    def rope(x):  # [n, h, D]
        x1, x2 = x[..., : D // 2], x[..., D // 2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)

    h = w["embed"][ids].astype(np.float64)
    mask = np.tril(np.ones((n, n), bool))
    for i in range(cfg["layers"]):
        p = f"layers.{i}."
        x = rms(h, w[p + "ln1"])
        q = rms(lin(x, p + "q").reshape(n, HQ, D), w[p + "q_norm"])
        k = rms(lin(x, p + "k").reshape(n, HK, D), w[p + "k_norm"])
        v = lin(x, p + "v").reshape(n, HK, D)
        q, k = rope(q), rope(k)
        att = np.zeros((n, HQ, D))
        for hh in range(HQ):
            s = q[:, hh] @ k[:, hh // (HQ // HK)].T / np.sqrt(D)
            s = np.where(mask, s, -np.inf)
            pr = np.exp(s - s.max(-1, keepdims=True))
            att[:, hh] = (pr / pr.sum(-1, keepdims=True)) @ v[:, hh // (HQ // HK)]
        h = h + lin(att.reshape(n, HQ * D), p + "o")
        x = rms(h, w[p + "ln2"])
        g, u = lin(x, p + "gate"), lin(x, p + "up")
        h = h + lin(g / (1 + np.exp(-g)) * u, p + "down")
    return rms(h, w["norm"]) @ dequant(w["lm_head.qweight"], w["lm_head.scales"], w["lm_head.biases"]).T


@pytest.fixture(scope="module")
def tiny():
    cfg = synth.tiny_config(layers=2, vocab=512)
    w = zero_mean(synth.host_weights(cfg, 0))
    return cfg, w


def test_forward_matches_dense_float64(tiny):
    cfg, w = tiny
    wf = synth.as_model_dtype(w, "f32")
    m = vxo.Model(dict(cfg, dtype=vxo.F32), wf)
    pages = vxo.Pages(cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"], 4, 16)
    ids = np.random.default_rng(1).integers(0, cfg["vocab"], 12).astype(np.uint32)
    bt = np.array([9, 2, 14, 5], np.uint32)  # scattered pages
    last = vxo.forward(m, pages, ids[:7], [(7, 0, bt)], all_rows=False)
    ver = vxo.forward(m, pages, ids[7:], [(5, 7, bt)], all_rows=True)
    ref = dense_forward(cfg, wf, ids)
    assert np.allclose(last[0], ref[6], rtol=1e-4, atol=1e-4)
    assert np.allclose(ver, ref[7:], rtol=1e-4, atol=1e-4)


def test_bf16_rounding_points_stay_within_logit_tolerance(tiny):
    """The bf16 model (every op rounded like candle's bf16 tensors) stays within
    the path's logit tolerance of the float64 model."""
    cfg, w = tiny
    m = vxo.Model(dict(cfg, dtype=vxo.BF16), synth.as_model_dtype(w, "bf16"))
    pages = vxo.Pages(cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"], 16, 4)
    ids = np.random.default_rng(2).integers(0, cfg["vocab"], 9).astype(np.uint32)
    got = vxo.forward(m, pages, ids, [(9, 0, np.array([0], np.uint32))], all_rows=True)
    ref = dense_forward(cfg, synth.as_model_dtype(w, "f32"), ids)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 0.05 * scale


def test_batched_forward_equals_per_sequence(tiny):
    cfg, w = tiny
    m = vxo.Model(dict(cfg, dtype=vxo.BF16), synth.as_model_dtype(w, "bf16"))
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    rng = np.random.default_rng(3)
    a, b = rng.integers(0, cfg["vocab"], 6).astype(np.uint32), rng.integers(0, cfg["vocab"], 3).astype(np.uint32)
    p1 = vxo.Pages(L, HK, D, 4, 8)
    both = vxo.forward(m, p1, np.concatenate([a, b]), [(6, 0, [0, 1]), (3, 0, [2])], all_rows=True)
    p2 = vxo.Pages(L, HK, D, 4, 8)
    sa = vxo.forward(m, p2, a, [(6, 0, [0, 1])], all_rows=True)
    sb = vxo.forward(m, p2, b, [(3, 0, [2])], all_rows=True)
    assert np.array_equal(both, np.concatenate([sa, sb]))


def greedy_decode(m, cfg, prompt, n_new):
    """Target-only greedy decoding (tests/spec_decode.rs:65-116)."""
    pages = vxo.Pages(cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"], 16, 16)
    bt = pages.alloc((len(prompt) + n_new + 15) // 16)
    toks = list(prompt)
    lg = vxo.forward(m, pages, np.array(prompt, np.uint32), [(len(prompt), 0, bt)], all_rows=False)
    toks.append(vxo.argmax(lg[0]))
    while len(toks) < len(prompt) + n_new:
        lg = vxo.forward(m, pages, np.array([toks[-1]], np.uint32), [(1, len(toks) - 1, bt)], all_rows=False)
        toks.append(vxo.argmax(lg[0]))
    return toks


def test_spec_greedy_equals_target_greedy(tiny):
    """spec.rs:1-49: the rolling-bonus greedy round commits exactly the tokens
    greedy target-only decoding produces (the oracle's attention reduces per
    row in position order, so the two paths are bit-identical here)."""
    cfg, w = tiny
    wb = synth.as_model_dtype(w, "bf16")
    c = dict(cfg, dtype=vxo.BF16)
    t, d = vxo.Model(c, wb), vxo.Model(c, wb, n_layers=1)
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    prompt = [5, 77, 301, 12, 9]
    e = vxo.SpecEngine(t, vxo.Pages(L, HK, D, 16, 16), d, vxo.Pages(1, HK, D, 16, 16))
    st = e.prefill([np.array(prompt, np.uint32)])
    n_new = 24
    while st[0].n_tokens < len(prompt) + n_new:
        e.step(st, 4)
    spec = vxo.SpecEngine.tokens(st[0])[: len(prompt) + n_new].tolist()
    assert spec == greedy_decode(t, cfg, prompt, n_new)


def test_draft_kv_hole_quirk_and_fix(tiny):
    """spec.rs:31-34 / :299: with all D accepted, draft KV slot kv_len+D is
    never written.  With draft == target the fixed mode accepts every
    candidate; the reference mode reads the unwritten slot and eventually
    rejects one."""
    cfg, w = tiny
    wb = synth.as_model_dtype(w, "bf16")
    c = dict(cfg, dtype=vxo.BF16)
    t, d = vxo.Model(c, wb), vxo.Model(c, wb)
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]

    def run(fix):
        e = vxo.SpecEngine(t, vxo.Pages(L, HK, D, 16, 16), d, vxo.Pages(L, HK, D, 16, 16), fix_draft_hole=fix)
        st = e.prefill([np.array([3, 1, 4, 1, 5, 9, 2, 6], np.uint32)])
        return [int(e.step(st, 3)["accepted"][0]) for _ in range(8)]

    assert run(True) == [3] * 8
    assert min(run(False)) < 3


def test_spec_errors_and_capacity(tiny):
    cfg, w = tiny
    c = dict(cfg, dtype=vxo.BF16)
    wb = synth.as_model_dtype(w, "bf16")
    t = vxo.Model(c, wb)
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    e = vxo.SpecEngine(t, vxo.Pages(L, HK, D, 16, 2), t, vxo.Pages(L, HK, D, 16, 2))
    with pytest.raises(RuntimeError, match="at least 2 tokens"):
        e.prefill([np.array([1], np.uint32)])
    st = e.prefill([np.arange(2, 20, dtype=np.uint32)])
    with pytest.raises(RuntimeError, match="draft_k"):
        e.step(st, 0)
    with pytest.raises(RuntimeError, match="grow target block table"):
        e.step(st, 16)
    e2 = vxo.SpecEngine(t, vxo.Pages(L, HK, D, 16, 2), t, vxo.Pages(L, HK, D, 8, 2))
    with pytest.raises(RuntimeError, match="page_size"):
        e2.prefill([np.arange(2, 5, dtype=np.uint32)])


def test_lockstep_mirror_replays_the_oracle_engine(tiny, monkeypatch):
    """The round-by-round mirror the GPU engine tests use (tests/lockstep.py)
    restates the spec loop's KV bookkeeping (draft fed [last, c0..c_{D-2}] at
    kv_len + i, the draft-KV hole, verify at kv_len, commit A + 1): replayed
    on the oracle engine's own rounds it reproduces their verify logits bit for
    bit and the same token streams."""
    import lockstep

    monkeypatch.setattr(lockstep, "ATOL", 0.0)
    monkeypatch.setattr(lockstep, "RTOL", 0.0)
    cfg, w = tiny
    wb = synth.as_model_dtype(w, "bf16")
    c = dict(cfg, dtype=vxo.BF16)
    t, d = vxo.Model(c, wb), vxo.Model(c, wb, n_layers=1)
    L, HK, D = cfg["layers"], cfg["n_kv_heads"], cfg["head_dim"]
    prompts = [np.array([5, 77, 301, 12, 9], np.uint32), np.array([8, 1, 400, 22, 13, 100, 7, 250, 3], np.uint32)]
    e = vxo.SpecEngine(t, vxo.Pages(L, HK, D, 16, 16), d, vxo.Pages(1, HK, D, 16, 16))
    st = e.prefill(prompts)
    ls = lockstep.Lockstep(cfg, w, 1, max_tokens=96, n_seqs=2, threads=1)
    ls.prefill(prompts)

    class Out:
        def __init__(self, a, toks):
            self.accepted, self.committed_tokens = int(a), list(map(int, toks))

    accepted = []
    for _ in range(6):
        ro = e.step(st, 4, trace=True)
        tr = {"n": 2, "k": 4, "temperature": 0.0, "candidates": ro["candidates"], "verify_logits": ro["logits"]}
        ls.check_round(tr, [Out(ro["accepted"][b], ro["committed"][b]) for b in range(2)])
        accepted += list(ro["accepted"])
    for b in range(2):
        assert ls.seqs[b]["tokens"] == vxo.SpecEngine.tokens(st[b]).tolist()
    assert min(accepted) < 4 and max(accepted) >= 1, accepted  # rejections and accepted candidates
