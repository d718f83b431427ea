"""bench.py's command-line contract, on the CPU: a run on more than one GPU is
refused with a message (this build measures one GPU), and every mode the
driver or a user names parses."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_modes_parse():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for mode in ("spec", "qmm", "continuous", "tree", "config0", "gemm"):
        assert mode in r.stdout


def test_cpu_baseline_adopts_the_prefilled_kv(monkeypatch):
    """The CPU baseline's oracle engine takes another engine's prefilled KV
    pages (bench.py copies them from the GPU) instead of prefilling itself.
    Fed an oracle prefill's pages (bf16 values, exact in the f16 snapshot),
    its rounds commit exactly what the prefilled engine commits."""
    import numpy as np

    sys.path.insert(0, ROOT)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import bench
    import vxo
    from velox_amd import synth

    cfg = synth.tiny_config(layers=4)
    w = synth.host_weights(cfg, 2)
    wt = synth.as_model_dtype(w, "bf16")
    c = dict(cfg, dtype=vxo.BF16)
    HK, D = cfg["n_kv_heads"], cfg["head_dim"]
    t, d = vxo.Model(c, wt, threads=2), vxo.Model(c, wt, n_layers=4, threads=2)
    tp, dp = vxo.Pages(4, HK, D, 16, 40), vxo.Pages(4, HK, D, 16, 40)
    e = vxo.SpecEngine(t, tp, d, dp)
    prompts = [synth.prompt(2, 21, cfg["vocab"], stream=i) for i in range(3)]
    st = e.prefill(prompts)
    snap = []
    for which, pg in ((0, tp), (1, dp)):
        tables = [np.ctypeslib.as_array(s.target_blocks if which == 0 else s.draft_blocks,
                                        shape=(s.n_target_blocks if which == 0 else s.n_draft_blocks,)).copy()
                  for s in st]
        used = np.unique(np.concatenate(tables))
        for layer in range(4):
            for kv in (0, 1):
                pool = pg.pool(layer, kv)
                snap.append((which, layer, kv, tables, {int(u): pool[u].astype(np.float16) for u in used}))
    e.step(st, 4)  # the baseline's warm-up round
    want = e.step(st, 4)
    logs = []
    monkeypatch.setattr(bench, "log", lambda *a: logs.append(" ".join(map(str, a))))
    res = bench.cpu_baseline(cfg, w, prompts, 4, snap, rounds=1)
    assert res["value"] > 0 and res["kind"] == "port" and res["cores"] >= 1
    toks = int(sum(len(x) for x in want["committed"]))
    assert f"{toks} tokens" in logs[-1], (logs[-1], toks)
