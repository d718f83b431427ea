"""MLX int4 checkpoint loader: a Hugging Face-layout Qwen3 directory
(`config.json` + `*.safetensors`, optionally sharded with
`model.safetensors.index.json`) quantized by MLX to 4 bits, read into the
host-weight dict that `engine.PagedQwen3` takes.

Follows the reference's loader (src/paged/qwen3.rs):
* config fields and the `quantization` block (`:30-69`; MLX also writes it as
  `quantization_config`, read here when `quantization` is absent);
* per-linear tensors `weight` (u32 [N, K/8], eight little-endian nibbles),
  `scales` and `biases` ([N, K/group]) and the 4-bit / divisibility checks of
  `maybe_qlinear` (`:180-240`);
* tensor names `model.embed_tokens`, `model.layers.{i}.self_attn.{q,k,v,o}_proj`,
  `...self_attn.{q,k}_norm`, `...mlp.{gate,up,down}_proj`,
  `...input_layernorm`, `...post_attention_layernorm`, `model.norm`,
  `lm_head` (`:324-326`, `:387-394`, `:921-927`, `:958-976`);
* a quantized embedding table dequantized once on the host as
  `q * scale + bias` in f32, then rounded to the model dtype
  (`load_embedding`, `:1043-1095`).

The engine runs the LM head as an int4 GEMM, so a checkpoint needs either a
quantized `lm_head` or tied embeddings stored quantized (then the embedding's
own triplet serves as the LM head: the reference multiplies by the
dequantized bf16 table instead, which differs by the weight's rounding).
"""
from __future__ import annotations

import json
import os

import numpy as np

from . import synth

LINEAR_NAMES = {  # engine name -> checkpoint path below model.layers.{i}
    "q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
    "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj",
}


class CheckpointError(ValueError):
    pass


def read_config(path: str) -> dict:
    """config.json -> the engine's config dict (synth.tiny_config keys)."""
    with open(os.path.join(path, "config.json")) as f:
        c = json.load(f)
    q = c.get("quantization") or c.get("quantization_config")
    if not q:
        raise CheckpointError("velox_amd needs an MLX 4-bit checkpoint (config.json has no quantization block)")
    if int(q.get("bits", 0)) != 4:
        raise CheckpointError(f"velox only supports 4-bit MLX quant (got bits={q.get('bits')})")
    if c.get("attention_bias", False):
        raise CheckpointError("attention bias is not supported (Qwen3 has none)")
    head_dim = c.get("head_dim") or c["hidden_size"] // c["num_attention_heads"]
    return dict(hidden=int(c["hidden_size"]), inter=int(c["intermediate_size"]),
                layers=int(c["num_hidden_layers"]), n_heads=int(c["num_attention_heads"]),
                n_kv_heads=int(c["num_key_value_heads"]), head_dim=int(head_dim), vocab=int(c["vocab_size"]),
                max_pos=int(c["max_position_embeddings"]), group_size=int(q["group_size"]),
                rope_theta=float(c["rope_theta"]), rms_eps=float(c["rms_norm_eps"]),
                tie_word_embeddings=bool(c.get("tie_word_embeddings", False)))


def _files(path: str) -> list[str]:
    idx = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(idx):
        with open(idx) as f:
            return sorted({os.path.join(path, v) for v in json.load(f)["weight_map"].values()})
    files = sorted(os.path.join(path, n) for n in os.listdir(path) if n.endswith(".safetensors"))
    if not files:
        raise CheckpointError(f"no .safetensors files in {path}")
    return files


class _Tensors:
    """Name -> tensor over every safetensors file of the checkpoint (read
    lazily; only loaders that execute nothing from the file are used)."""

    def __init__(self, path: str):
        from safetensors import safe_open

        self._where = {}
        self._handles = []
        for fn in _files(path):
            h = safe_open(fn, framework="pt")
            self._handles.append(h)
            for k in h.keys():
                self._where[k] = h

    def has(self, name: str) -> bool:
        return name in self._where

    def get(self, name: str):
        if name not in self._where:
            raise CheckpointError(f"missing tensor {name}")
        return self._where[name].get_tensor(name)


def _as_u32(t) -> np.ndarray:
    import torch

    if t.dtype in (torch.uint32, torch.int32):
        return t.contiguous().view(torch.int32).numpy().view(np.uint32)
    raise CheckpointError(f"packed int4 weights must be u32, got {t.dtype}")


def _as_f32(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).contiguous().numpy()


def _qlinear(T: _Tensors, prefix: str, n: int, k: int, g: int) -> dict:
    """maybe_qlinear (qwen3.rs:180-240) for the quantized case."""
    if k % g != 0:
        raise CheckpointError(f"QLinear: in_features {k} not divisible by group_size {g}")
    if k % 8 != 0:
        raise CheckpointError(f"QLinear: in_features {k} not multiple of 8")
    qw = _as_u32(T.get(prefix + ".weight"))
    sc = _as_f32(T.get(prefix + ".scales"))
    bi = _as_f32(T.get(prefix + ".biases"))
    for name, a, shape in (("weight", qw, (n, k // 8)), ("scales", sc, (n, k // g)), ("biases", bi, (n, k // g))):
        if a.shape != shape:
            raise CheckpointError(f"{prefix}.{name}: shape {a.shape}, expected {shape}")
    if T.has(prefix + ".bias"):
        raise CheckpointError(f"{prefix}: linear bias is not supported (Qwen3 has none)")
    # the engine takes bf16 model values in f16 carriers
    return {"qweight": qw, "scales": synth.round_bits(sc, "bf16").astype(np.float16),
            "biases": synth.round_bits(bi, "bf16").astype(np.float16)}


def dequant_embedding(qw: np.ndarray, sc: np.ndarray, bi: np.ndarray, g: int) -> np.ndarray:
    """load_embedding (qwen3.rs:1074-1092): q * scale + bias in f32 per
    (row, group, nibble)."""
    n, kp = qw.shape
    k = kp * 8
    shifts = np.arange(8, dtype=np.uint32) * 4
    q = ((qw[:, :, None] >> shifts) & 0xF).astype(np.float32).reshape(n, k)
    s = np.repeat(sc.astype(np.float32), g, axis=1)
    b = np.repeat(bi.astype(np.float32), g, axis=1)
    return q * s + b


def load_mlx_qwen3(path: str, n_layers: int | None = None) -> tuple[dict, dict]:
    """Returns (cfg, weights) for engine.PagedQwen3(cfg, weights, n_layers)."""
    cfg = read_config(path)
    T = _Tensors(path)
    H, V, F, D, g = cfg["hidden"], cfg["vocab"], cfg["inter"], cfg["head_dim"], cfg["group_size"]
    HQ, HK = cfg["n_heads"], cfg["n_kv_heads"]
    L = cfg["layers"] if n_layers is None else n_layers
    w = {}
    emb = "model.embed_tokens"
    emb_quant = T.has(emb + ".scales") and H % g == 0 and H % 8 == 0
    if emb_quant:
        eq = _qlinear(T, emb, V, H, g)
        table = dequant_embedding(eq["qweight"], eq["scales"].astype(np.float32), eq["biases"].astype(np.float32), g)
    else:
        table = _as_f32(T.get(emb + ".weight"))
        if table.shape != (V, H):
            raise CheckpointError(f"{emb}.weight: shape {table.shape}, expected {(V, H)}")
    w["embed"] = synth.round_bits(table, "bf16").astype(np.float16)
    if cfg["tie_word_embeddings"]:
        if not emb_quant:
            raise CheckpointError("tied embeddings must be stored quantized: the engine's LM head is an int4 GEMM")
        lm = eq
    else:
        lm = _qlinear(T, "lm_head", V, H, g)
    for name, arr in lm.items():
        w["lm_head." + name] = arr
    w["norm"] = synth.round_bits(_as_f32(T.get("model.norm.weight")), "bf16").astype(np.float16)
    shapes = {"q": (HQ * D, H), "k": (HK * D, H), "v": (HK * D, H), "o": (H, HQ * D),
              "gate": (F, H), "up": (F, H), "down": (H, F)}
    for i in range(L):
        src = f"model.layers.{i}."
        dst = f"layers.{i}."
        for lin, path_name in LINEAR_NAMES.items():
            n, k = shapes[lin]
            for name, arr in _qlinear(T, src + path_name, n, k, g).items():
                w[dst + lin + "." + name] = arr
        for dname, sname, size in (("ln1", "input_layernorm", H), ("ln2", "post_attention_layernorm", H),
                                   ("q_norm", "self_attn.q_norm", D), ("k_norm", "self_attn.k_norm", D)):
            a = _as_f32(T.get(src + sname + ".weight"))
            if a.shape != (size,):
                raise CheckpointError(f"{src}{sname}.weight: shape {a.shape}, expected {(size,)}")
            w[dst + dname] = synth.round_bits(a, "bf16").astype(np.float16)
    return cfg, w
