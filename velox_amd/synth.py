"""Seeded synthetic Qwen3-shaped models in the MLX int4 g64 affine format.

Tensor layouts follow the reference's MLX-int4 QLinear (src/paged/qwen3.rs:134-150,
:204-211): `qweight` u32 [N, K/8] with 8 nibbles little-endian per word,
`scales` / `biases` [N, K/64].  Value distributions are the benchmark configs'
synthetic random init: codes uniform 0..15 (a uniform u32 word is 8 uniform
nibbles), scale ~ U(0.002, 0.02), bias ~ N(0, 0.01), embeddings ~ N(0, 0.02),
all stored as f16; RMSNorm weights are 1.  Every tensor draws from its own
numpy Philox stream keyed by (seed, crc32(name)), so a model truncated to its
first L layers (the draft) holds exactly the target's first L layers.
"""
from __future__ import annotations

import zlib

import numpy as np

# Qwen3 shapes (hidden, inter, layers, q heads, kv heads, head_dim); vocab 151936.
SHAPES = {
    "qwen3-0.6b": dict(hidden=1024, inter=3072, layers=28, n_heads=16, n_kv_heads=8, head_dim=128),
    "qwen3-4b": dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8, head_dim=128),
    "qwen3-8b": dict(hidden=4096, inter=12288, layers=36, n_heads=32, n_kv_heads=8, head_dim=128),
}

LINEARS = ("q", "k", "v", "o", "gate", "up", "down")


def qwen3_config(name: str, vocab: int = 151936, max_pos: int = 40960, **over) -> dict:
    cfg = dict(SHAPES[name], vocab=vocab, max_pos=max_pos, group_size=64, rope_theta=1e6,
               rms_eps=1e-6)
    cfg.update(over)
    return cfg


def tiny_config(**over) -> dict:
    """A small Qwen3-shaped config for parity tests that the CPU oracle runs in
    seconds (same structure: GQA, q/k norm, SwiGLU, untied int4 LM head)."""
    cfg = dict(hidden=256, inter=512, layers=3, n_heads=4, n_kv_heads=2, head_dim=64,
               vocab=1024, max_pos=4096, group_size=64, rope_theta=1e6, rms_eps=1e-6)
    cfg.update(over)
    return cfg


def linear_shapes(cfg: dict) -> dict:
    H, F, D = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    qw, kw = cfg["n_heads"] * D, cfg["n_kv_heads"] * D
    return {"q": (qw, H), "k": (kw, H), "v": (kw, H), "o": (H, qw), "gate": (F, H), "up": (F, H),
            "down": (H, F)}


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=[seed, zlib.crc32(name.encode())]))


def qlinear(seed: int, name: str, n: int, k: int, group_size: int = 64) -> dict:
    """One MLX int4 g64 linear: qweight u32 [n, k/8], scales/biases f16 [n, k/g]."""
    if k % group_size or k % 8:
        raise ValueError(f"{name}: K={k} must be a multiple of group_size and 8")
    rng = _rng(seed, name)
    qweight = rng.integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint32)
    scales = rng.uniform(0.002, 0.02, size=(n, k // group_size)).astype(np.float16)
    biases = rng.normal(0.0, 0.01, size=(n, k // group_size)).astype(np.float16)
    return {"qweight": qweight, "scales": scales, "biases": biases}


def host_weights(cfg: dict, seed: int, n_layers: int | None = None) -> dict:
    """Host (numpy) weights: f16 for floats, u32 packed codes."""
    L = cfg["layers"] if n_layers is None else n_layers
    H, V, D, g = cfg["hidden"], cfg["vocab"], cfg["head_dim"], cfg["group_size"]
    w = {"embed": _rng(seed, "embed").normal(0.0, 0.02, size=(V, H)).astype(np.float16),
         "norm": np.ones(H, np.float16)}
    for name, arr in qlinear(seed, "lm_head", V, H, g).items():
        w["lm_head." + name] = arr
    shapes = linear_shapes(cfg)
    for i in range(L):
        p = f"layers.{i}."
        for lin in LINEARS:
            n, k = shapes[lin]
            for name, arr in qlinear(seed, p + lin, n, k, g).items():
                w[p + lin + "." + name] = arr
        w[p + "ln1"] = np.ones(H, np.float16)
        w[p + "ln2"] = np.ones(H, np.float16)
        w[p + "q_norm"] = np.ones(D, np.float16)
        w[p + "k_norm"] = np.ones(D, np.float16)
    return w


def round_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16/f16/f32 storage (RNE), returned as float32."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), r)
        return (r << 16).astype(np.uint32).view(np.float32)
    raise ValueError(dtype)


def as_model_dtype(weights: dict, dtype: str) -> dict:
    """What the reference's VarBuilder hands the model for vb.dtype() == dtype:
    every float tensor converted to the model dtype (u32 codes untouched),
    returned as float32 arrays for the CPU oracle."""
    out = {}
    for k, v in weights.items():
        out[k] = v if v.dtype == np.uint32 else round_bits(v.astype(np.float32), dtype)
    return out


def prompt(seed: int, length: int, vocab: int, stream: int = 0) -> np.ndarray:
    rng = np.random.Generator(np.random.Philox(key=[seed, 0x70726F6D + stream]))
    return rng.integers(0, vocab, size=length, dtype=np.uint32)
