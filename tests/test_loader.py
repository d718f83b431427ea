"""MLX int4 checkpoint loader (velox_amd/loader.py) on checkpoints written here
with safetensors: Hugging Face tensor names, u32 packed codes, bf16 scales,
biases and norms, a quantized embedding table, sharding with an index file,
and the reference loader's error cases (src/paged/qwen3.rs:180-240,
:1043-1095)."""
import json

import numpy as np
import pytest
import torch

from refgen import dequant, quantize_mlx_4bit
from velox_amd import loader, synth


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def _u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).view(torch.uint32)


def write_checkpoint(path, cfg, w, *, bits=4, tie=False, quant_embed=True, shards=2, drop=None, extra=None):
    """Writes config.json + model-0000i-of-0000n.safetensors (+ index) from a
    synth host-weight dict; returns the embedding triplet written."""
    from safetensors.torch import save_file

    H, V = cfg["hidden"], cfg["vocab"]
    conf = {"vocab_size": V, "hidden_size": H, "intermediate_size": cfg["inter"],
            "num_hidden_layers": cfg["layers"], "num_attention_heads": cfg["n_heads"],
            "num_key_value_heads": cfg["n_kv_heads"], "head_dim": cfg["head_dim"],
            "max_position_embeddings": cfg["max_pos"], "rope_theta": cfg["rope_theta"],
            "rms_norm_eps": cfg["rms_eps"], "tie_word_embeddings": tie, "attention_bias": False,
            "hidden_act": "silu", "quantization": {"group_size": cfg["group_size"], "bits": bits}}
    (path / "config.json").write_text(json.dumps(conf))
    t = {}

    def ql(dst, src):
        t[dst + ".weight"] = _u32(w[src + ".qweight"])
        t[dst + ".scales"] = _bf16(w[src + ".scales"].astype(np.float32))
        t[dst + ".biases"] = _bf16(w[src + ".biases"].astype(np.float32))

    emb = None
    if quant_embed:
        qw, sc, bi = quantize_mlx_4bit(w["embed"].astype(np.float32), V, H, cfg["group_size"])
        emb = (qw, synth.round_bits(sc, "bf16"), synth.round_bits(bi, "bf16"))
        t["model.embed_tokens.weight"] = _u32(qw)
        t["model.embed_tokens.scales"] = _bf16(sc)
        t["model.embed_tokens.biases"] = _bf16(bi)
    else:
        t["model.embed_tokens.weight"] = _bf16(w["embed"].astype(np.float32))
    if not tie:
        ql("lm_head", "lm_head")
    t["model.norm.weight"] = _bf16(w["norm"].astype(np.float32))
    for i in range(cfg["layers"]):
        s, d = f"layers.{i}.", f"model.layers.{i}."
        for lin, name in loader.LINEAR_NAMES.items():
            ql(d + name, s + lin)
        t[d + "input_layernorm.weight"] = _bf16(w[s + "ln1"].astype(np.float32))
        t[d + "post_attention_layernorm.weight"] = _bf16(w[s + "ln2"].astype(np.float32))
        t[d + "self_attn.q_norm.weight"] = _bf16(w[s + "q_norm"].astype(np.float32))
        t[d + "self_attn.k_norm.weight"] = _bf16(w[s + "k_norm"].astype(np.float32))
    for k in drop or ():
        del t[k]
    t.update(extra or {})
    names = sorted(t)
    parts = [names[i::shards] for i in range(shards)]
    wmap = {}
    for j, part in enumerate(parts):
        fn = f"model-{j + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: t[k] for k in part}, str(path / fn), metadata={"format": "mlx"})
        wmap.update({k: fn for k in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    return emb


def test_dequant_embedding_known_answer():
    """Nibbles 0..15 of one row (pack known answer 0x76543210, 0xFEDCBA98,
    dyn_quant.rs:205-218) with scale 2, bias -1 dequantize to 2q - 1."""
    qw = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    out = loader.dequant_embedding(qw, np.array([[2.0]], np.float32), np.array([[-1.0]], np.float32), 16)
    assert np.array_equal(out, (2.0 * np.arange(16) - 1.0)[None].astype(np.float32))


def test_load_round_trip(tmp_path):
    cfg = synth.tiny_config(layers=2)
    w = synth.host_weights(cfg, 9)
    emb = write_checkpoint(tmp_path, cfg, w)
    got_cfg, got = loader.load_mlx_qwen3(str(tmp_path))
    for k in ("hidden", "inter", "layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "max_pos",
              "group_size", "rope_theta", "rms_eps"):
        assert got_cfg[k] == cfg[k], k
    # embedding: q * s + b in f32 (load_embedding), rounded to bf16
    want = synth.round_bits(dequant(*emb, gs=cfg["group_size"]).astype(np.float32), "bf16")
    assert np.array_equal(got["embed"].astype(np.float32), want)
    for k, v in w.items():
        if k == "embed":
            continue
        if k.endswith(".qweight"):
            assert np.array_equal(got[k], v), k
        else:
            assert np.array_equal(got[k].astype(np.float32), synth.round_bits(v.astype(np.float32), "bf16")), k


def test_tied_quantized_embedding_serves_as_lm_head(tmp_path):
    cfg = synth.tiny_config(layers=1)
    w = synth.host_weights(cfg, 2)
    emb = write_checkpoint(tmp_path, cfg, w, tie=True, shards=1)
    _, got = loader.load_mlx_qwen3(str(tmp_path))
    assert np.array_equal(got["lm_head.qweight"], emb[0])
    assert np.array_equal(got["lm_head.scales"].astype(np.float32), emb[1])


@pytest.mark.parametrize("case,msg", [
    ("bits8", "only supports 4-bit MLX quant \\(got bits=8\\)"),
    ("missing", "missing tensor model.layers.0.mlp.down_proj.scales"),
    ("shape", "model.layers.0.self_attn.q_proj.weight: shape"),
    ("tied_dense", "tied embeddings must be stored quantized"),
    ("bias", "linear bias is not supported"),
])
def test_load_errors(tmp_path, case, msg):
    cfg = synth.tiny_config(layers=1)
    w = synth.host_weights(cfg, 4)
    kw = {}
    if case == "bits8":
        kw["bits"] = 8
    elif case == "missing":
        kw["drop"] = ["model.layers.0.mlp.down_proj.scales"]
    elif case == "shape":
        kw["extra"] = {"model.layers.0.self_attn.q_proj.weight": _u32(np.zeros((3, 5), np.uint32))}
    elif case == "tied_dense":
        kw.update(tie=True, quant_embed=False)
    elif case == "bias":
        kw["extra"] = {"model.layers.0.mlp.up_proj.bias": _bf16(np.zeros(cfg["inter"], np.float32))}
    write_checkpoint(tmp_path, cfg, w, **kw)
    with pytest.raises(loader.CheckpointError, match=msg):
        loader.load_mlx_qwen3(str(tmp_path))
