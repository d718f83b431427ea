"""ctypes binding of the CPU oracle (oracle/libvxo.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libvxo.so")

F32, F16, BF16 = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
_i64 = C.c_int64


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_LIB_PATH)
    vp = C.c_void_p
    sig = {
        "vxo_f32_to_f16": (C.c_uint16, [C.c_float]),
        "vxo_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "vxo_round_array": (None, [_f32p, _i64, C.c_int]),
        "vxo_philox4x32_10": (None, [_u32p, _u32p, _u32p]),
        "vxo_spec_uniforms": (None, [C.c_uint64, C.c_uint32, C.c_uint32, _i64, _i64, _f32p]),
        "vxo_expf": (C.c_float, [C.c_float]),
        "vxo_pack_int4": (None, [_u32p, _i64, _i64, _u32p]),
        "vxo_unpack_int4": (None, [_u32p, _i64, _i64, _u32p]),
        "vxo_qmm_4bit": (C.c_int, [_f32p, _u32p, _f32p, _f32p, vp, _f32p, _i64, _i64, _i64, _i64, C.c_int]),
        "vxo_paged_attention": (C.c_int, [_f32p, _f32p, _f32p, _u32p, _i64, _u32p, _u32p, _i64, vp,
                                          _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_uint32, _f32p]),
        "vxo_rope_tables": (None, [_i64, _i64, C.c_double, _f32p, _f32p]),
        "vxo_rope_apply": (None, [_f32p, _f32p, _f32p, _u32p, _i64, _i64, _i64, C.c_int]),
        "vxo_kv_scatter": (None, [_f32p, _f32p, _u32p, _u32p, _i64, _i64, _i64, _i64]),
        "vxo_rmsnorm": (None, [_f32p, _f32p, _f32p, _i64, _i64, C.c_float, C.c_int]),
        "vxo_argmax": (C.c_uint32, [_f32p, _i64]),
        "vxo_accept_greedy": (None, [_f32p, _i64, _u32p, _i64, _i64, _i32p, _u32p]),
        "vxo_row_softmax_stats": (None, [_f32p, _i64, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "vxo_sample_residual": (C.c_uint32, [_f32p, C.c_float, C.c_float, vp, C.c_float, C.c_float, _i64,
                                             C.c_float, C.c_float]),
        "vxo_sample_draft": (None, [_f32p, _f32p, _i64, _i64, _i64, C.c_float, _u32p]),
        "vxo_accept_stochastic": (None, [_f32p, _f32p, _u32p, _f32p, _i64, _i64, _i64, C.c_float, _i32p, _u32p]),
        "vxo_accept_tree": (None, [_f32p, _i32p, _u32p, _i64, _i64, _i64, _i32p, _i32p, _u32p]),
        "vxo_tree_masks": (None, [_i32p, _i64, _u64p, _i32p]),
        "vxo_last_error": (C.c_char_p, []),
        "vxo_model_create": (vp, [vp, vp, C.c_int]),
        "vxo_model_destroy": (None, [vp]),
        "vxo_pages_create": (vp, [_i64, _i64, _i64, _i64, _i64]),
        "vxo_pages_destroy": (None, [vp]),
        "vxo_pages_alloc": (C.c_int, [vp, _i64, _u32p]),
        "vxo_pages_free": (None, [vp, _u32p, _i64]),
        "vxo_pages_num_free": (_i64, [vp]),
        "vxo_pages_pool": (vp, [vp, _i64, C.c_int]),
        "vxo_forward": (C.c_int, [vp, vp, _u32p, vp, _i64, C.c_int, vp, _f32p]),
        "vxo_spec_prefill": (C.c_int, [vp, vp, vp, _i64, vp]),
        "vxo_spec_step": (C.c_int, [vp, vp, _i64, _i64, _i64, _i32p, _u32p, _i32p, vp, vp]),
        "vxo_spec_adopt": (C.c_int, [vp, _u32p, _i64, vp]),
        "vxo_spec_free": (None, [vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib.vxo_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ----------------------------------------------------------------- numerics
def round_to(x: np.ndarray, dtype: int) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib.vxo_round_array(y, y.size, dtype)
    return y


def philox(ctr, key) -> np.ndarray:
    out = np.zeros(4, np.uint32)
    lib.vxo_philox4x32_10(np.asarray(ctr, np.uint32), np.asarray(key, np.uint32), out)
    return out


def spec_uniforms(seed: int, stream0: int, rnd: int, batch: int, k: int) -> np.ndarray:
    out = np.zeros((batch, k + 1, 4), np.float32)
    lib.vxo_spec_uniforms(seed, stream0, rnd, batch, k, out)
    return out


def expf(x: float) -> float:
    return lib.vxo_expf(x)


# --------------------------------------------------------------------- int4
def pack_int4(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint32)
    n, k = codes.shape
    out = np.zeros((n, k // 8), np.uint32)
    lib.vxo_pack_int4(codes, n, k, out)
    return out


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint32)
    n, kp = packed.shape
    out = np.zeros((n, kp * 8), np.uint32)
    lib.vxo_unpack_int4(packed, n, kp * 8, out)
    return out


def qmm_4bit(x, qweight, scales, biases, bias=None, group_size=64, threads=1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    n = qweight.shape[0]
    y = np.zeros((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    _check(lib.vxo_qmm_4bit(x, np.ascontiguousarray(qweight, np.uint32),
                            np.ascontiguousarray(scales, np.float32),
                            np.ascontiguousarray(biases, np.float32), _ptr(b), y, m, n, k,
                            group_size, threads))
    return y


# ---------------------------------------------------------------- attention
def paged_attention(q, k_pool, v_pool, block_table, cu_seqlens, kv_offsets, scale,
                    tree_mask=None, sliding_window=0) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    total_q, h_q, d = q.shape
    _, h_kv, ps, _ = k_pool.shape
    bt = np.ascontiguousarray(block_table, np.uint32)
    n_seqs, max_blocks = bt.shape
    out = np.zeros_like(q)
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint64)
    _check(lib.vxo_paged_attention(q, np.ascontiguousarray(k_pool, np.float32),
                                   np.ascontiguousarray(v_pool, np.float32), bt, max_blocks,
                                   np.ascontiguousarray(cu_seqlens, np.uint32),
                                   np.ascontiguousarray(kv_offsets, np.uint32), n_seqs, _ptr(tm),
                                   total_q, h_q, h_kv, d, ps, scale, sliding_window, out))
    return out


def rope_tables(max_pos: int, head_dim: int, theta: float):
    c = np.zeros((max_pos, head_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib.vxo_rope_tables(max_pos, head_dim, theta, c, s)
    return c, s


def rope_apply(x, cos_t, sin_t, pos, dtype=F32) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    n, h, d = y.shape
    lib.vxo_rope_apply(y, np.ascontiguousarray(cos_t, np.float32),
                       np.ascontiguousarray(sin_t, np.float32),
                       np.ascontiguousarray(pos, np.uint32), n, h, d, dtype)
    return y


def kv_scatter(pool, values, page_ids, slots) -> np.ndarray:
    p = np.ascontiguousarray(pool, np.float32).copy()
    _, h, s, d = p.shape
    v = np.ascontiguousarray(values, np.float32)
    lib.vxo_kv_scatter(p, v, np.ascontiguousarray(page_ids, np.uint32),
                       np.ascontiguousarray(slots, np.uint32), v.shape[0], h, s, d)
    return p


def rmsnorm(x, w, eps, dtype=F32) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    rows, dim = x.reshape(-1, x.shape[-1]).shape
    lib.vxo_rmsnorm(x, np.ascontiguousarray(w, np.float32), y, rows, dim, eps, dtype)
    return y


# --------------------------------------------------------------- acceptance
def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib.vxo_argmax(v, v.size))


def accept_greedy(logits, candidates):
    logits = np.ascontiguousarray(logits, np.float32)
    b, r, v = logits.shape
    cand = np.ascontiguousarray(candidates, np.uint32)
    acc = np.zeros(b, np.int32)
    tok = np.zeros((b, r), np.uint32)
    lib.vxo_accept_greedy(logits, v, cand, b, r - 1, acc, tok)
    return acc, tok


def row_softmax_stats(row, inv_t):
    row = np.ascontiguousarray(row, np.float32)
    m, z = C.c_float(), C.c_float()
    lib.vxo_row_softmax_stats(row, row.size, inv_t, C.byref(m), C.byref(z))
    return m.value, z.value


def sample_residual(lt, mt, zt, u, inv_t, ld=None, md=0.0, zd=1.0) -> int:
    """Inverse-CDF draw from max(0, p - q) (q absent: from p) with the
    statistics (m, z) of each row, as the acceptance kernels use it."""
    lt = np.ascontiguousarray(lt, np.float32)
    ldp = None
    if ld is not None:
        ld = np.ascontiguousarray(ld, np.float32)
        ldp = ld.ctypes.data
    return int(lib.vxo_sample_residual(lt, mt, zt, ldp, md, zd, lt.size, inv_t, u))


def sample_draft(draft_logits, uniforms, inv_t):
    dl = np.ascontiguousarray(draft_logits, np.float32)
    b, k, v = dl.shape
    out = np.zeros((b, k), np.uint32)
    lib.vxo_sample_draft(dl, np.ascontiguousarray(uniforms, np.float32), b, k, v, inv_t, out)
    return out


def accept_stochastic(target_logits, draft_logits, candidates, uniforms, inv_t):
    tl = np.ascontiguousarray(target_logits, np.float32)
    b, r, v = tl.shape
    acc = np.zeros(b, np.int32)
    tok = np.zeros((b, r), np.uint32)
    lib.vxo_accept_stochastic(tl, np.ascontiguousarray(draft_logits, np.float32),
                              np.ascontiguousarray(candidates, np.uint32),
                              np.ascontiguousarray(uniforms, np.float32), b, r - 1, v, inv_t, acc,
                              tok)
    return acc, tok


def accept_tree(logits, parents, node_tokens):
    lg = np.ascontiguousarray(logits, np.float32)
    b, r, v = lg.shape
    acc = np.zeros(b, np.int32)
    path = np.zeros((b, r), np.int32)
    tok = np.zeros((b, r), np.uint32)
    lib.vxo_accept_tree(lg, np.ascontiguousarray(parents, np.int32),
                        np.ascontiguousarray(node_tokens, np.uint32), b, r, v, acc, path, tok)
    return acc, path, tok


def tree_masks(parents):
    p = np.ascontiguousarray(parents, np.int32)
    m = np.zeros(p.size, np.uint64)
    d = np.zeros(p.size, np.int32)
    lib.vxo_tree_masks(p, p.size, m, d)
    return m, d


# ---------------------------------------------------- model / pages / spec
class _Config(C.Structure):
    _fields_ = [("vocab", _i64), ("hidden", _i64), ("inter", _i64), ("layers", _i64),
                ("n_heads", _i64), ("n_kv_heads", _i64), ("head_dim", _i64),
                ("max_pos", _i64), ("group_size", _i64), ("rope_theta", C.c_double),
                ("rms_eps", C.c_double), ("dtype", C.c_int)]


class _QLin(C.Structure):
    _fields_ = [("qweight", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class _Layer(C.Structure):
    _fields_ = [("ln1", C.c_void_p), ("ln2", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("q", _QLin), ("k", _QLin), ("v", _QLin), ("o", _QLin),
                ("gate", _QLin), ("up", _QLin), ("down", _QLin)]


class _Weights(C.Structure):
    _fields_ = [("embed", C.c_void_p), ("layers", C.c_void_p), ("norm", C.c_void_p),
                ("lm_head", _QLin)]


class _Seq(C.Structure):
    _fields_ = [("new_tokens", _i64), ("kv_offset", _i64), ("block_table", C.c_void_p),
                ("n_blocks", _i64)]


class _State(C.Structure):
    _fields_ = [("target_blocks", C.POINTER(C.c_uint32)), ("draft_blocks", C.POINTER(C.c_uint32)),
                ("n_target_blocks", _i64), ("n_draft_blocks", _i64), ("kv_len", _i64),
                ("last_token", C.c_uint32), ("tokens", C.POINTER(C.c_uint32)), ("n_tokens", _i64),
                ("stream_id", C.c_uint32), ("round", C.c_uint32)]


class _Spec(C.Structure):
    _fields_ = [("target", C.c_void_p), ("draft", C.c_void_p), ("target_pages", C.c_void_p),
                ("draft_pages", C.c_void_p), ("temperature", C.c_float),
                ("sample_seed", C.c_uint64), ("fix_draft_hole", C.c_int)]


class Model:
    """Oracle PagedQwen3.  `weights` is the dict produced by
    velox_amd.synth.host_weights(..., as_float=True) (or any dict with the same
    keys): float32 arrays already rounded to cfg['dtype']."""

    def __init__(self, cfg: dict, weights: dict, n_layers: int | None = None, threads: int = 1):
        L = cfg["layers"] if n_layers is None else n_layers
        self.cfg = dict(cfg, layers=L)
        self._keep = []

        def arr(a, dt):
            a = np.ascontiguousarray(a, dt)
            self._keep.append(a)
            return a.ctypes.data

        def ql(prefix):
            return _QLin(arr(weights[prefix + ".qweight"], np.uint32),
                         arr(weights[prefix + ".scales"], np.float32),
                         arr(weights[prefix + ".biases"], np.float32))

        layers = (_Layer * L)()
        for i in range(L):
            p = f"layers.{i}."
            layers[i] = _Layer(arr(weights[p + "ln1"], np.float32), arr(weights[p + "ln2"], np.float32),
                               arr(weights[p + "q_norm"], np.float32),
                               arr(weights[p + "k_norm"], np.float32),
                               ql(p + "q"), ql(p + "k"), ql(p + "v"), ql(p + "o"), ql(p + "gate"),
                               ql(p + "up"), ql(p + "down"))
        self._layers = layers
        self._w = _Weights(arr(weights["embed"], np.float32), C.addressof(layers),
                           arr(weights["norm"], np.float32), ql("lm_head"))
        c = self.cfg
        self._c = _Config(c["vocab"], c["hidden"], c["inter"], L, c["n_heads"], c["n_kv_heads"],
                          c["head_dim"], c["max_pos"], c["group_size"], c["rope_theta"],
                          c["rms_eps"], c["dtype"])
        self.h = lib.vxo_model_create(C.byref(self._c), C.byref(self._w), threads)

    def __del__(self):
        if getattr(self, "h", None):
            lib.vxo_model_destroy(self.h)
            self.h = None


class Pages:
    def __init__(self, layers, kv_heads, head_dim, page_size, num_pages):
        self.page_size = page_size
        self.layers, self.kv_heads, self.head_dim, self.num_pages = layers, kv_heads, head_dim, num_pages
        self.h = lib.vxo_pages_create(layers, kv_heads, head_dim, page_size, num_pages)
        if not self.h:
            raise RuntimeError(lib.vxo_last_error().decode())

    def alloc(self, n):
        out = np.zeros(n, np.uint32)
        if lib.vxo_pages_alloc(self.h, n, out) != 0:
            return None
        return out

    def free(self, pages):
        p = np.ascontiguousarray(pages, np.uint32)
        lib.vxo_pages_free(self.h, p, p.size)

    def pool(self, layer, kv):
        """Writable view of one layer's K (kv=0) or V (kv=1) pool
        [num_pages, kv_heads, page_size, head_dim]."""
        ptr = lib.vxo_pages_pool(self.h, layer, kv)
        shape = (self.num_pages, self.kv_heads, self.page_size, self.head_dim)
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=shape)

    def num_free(self):
        return lib.vxo_pages_num_free(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib.vxo_pages_destroy(self.h)
            self.h = None


def forward(model: Model, pages: Pages, ids, seqs, all_rows=True, tree_parents=None):
    """seqs: list of (new_tokens, kv_offset, block_table array)."""
    ids = np.ascontiguousarray(ids, np.uint32)
    arr = (_Seq * len(seqs))()
    keep = []
    for i, (nt, off, bt) in enumerate(seqs):
        bt = np.ascontiguousarray(bt, np.uint32)
        keep.append(bt)
        arr[i] = _Seq(nt, off, bt.ctypes.data, bt.size)
    rows = ids.size if all_rows else len(seqs)
    out = np.zeros((rows, model.cfg["vocab"]), np.float32)
    tp = None if tree_parents is None else np.ascontiguousarray(tree_parents, np.int32)
    _check(lib.vxo_forward(model.h, pages.h, ids, C.cast(arr, C.c_void_p), len(seqs),
                           1 if all_rows else 0, _ptr(tp), out))
    return out


class SpecEngine:
    def __init__(self, target: Model, target_pages: Pages, draft: Model, draft_pages: Pages,
                 temperature=0.0, sample_seed=0, fix_draft_hole=False):
        self._refs = (target, target_pages, draft, draft_pages)
        self._s = _Spec(target.h, draft.h, target_pages.h, draft_pages.h, temperature,
                        sample_seed, 1 if fix_draft_hole else 0)
        self.vocab = target.cfg["vocab"]

    def prefill(self, prompts):
        n = len(prompts)
        ps = [np.ascontiguousarray(p, np.uint32) for p in prompts]
        ptrs = (C.c_void_p * n)(*[p.ctypes.data for p in ps])
        lens = np.array([p.size for p in ps], np.int64)
        states = (_State * n)()
        _check(lib.vxo_spec_prefill(C.byref(self._s), C.cast(ptrs, C.c_void_p),
                                    lens.ctypes.data_as(C.c_void_p), n, C.cast(states, C.c_void_p)))
        return states

    def adopt(self, prompts):
        """States as prefill would leave them, with the KV pages left for the
        caller to fill (see vxo_spec_adopt)."""
        n = len(prompts)
        states = (_State * n)()
        for b, p in enumerate(prompts):
            p = np.ascontiguousarray(p, np.uint32)
            _check(lib.vxo_spec_adopt(C.byref(self._s), p, p.size, C.byref(states[b])))
        return states

    def step(self, states, draft_k, eos=-1, trace=False):
        n = len(states)
        acc = np.zeros(n, np.int32)
        com = np.zeros((n, draft_k + 1), np.uint32)
        stop = np.zeros(n, np.int32)
        tc = np.zeros((n, draft_k), np.uint32) if trace else None
        tl = np.zeros((n, draft_k + 1, self.vocab), np.float32) if trace else None
        _check(lib.vxo_spec_step(C.byref(self._s), C.cast(states, C.c_void_p), n, draft_k, eos, acc,
                                 com, stop, _ptr(tc), _ptr(tl)))
        out = {"accepted": acc, "committed": [com[b, : acc[b] + 1].copy() for b in range(n)],
               "stop": stop.astype(bool)}
        if trace:
            out["candidates"] = tc
            out["logits"] = tl
        return out

    @staticmethod
    def tokens(state) -> np.ndarray:
        return np.ctypeslib.as_array(state.tokens, shape=(state.n_tokens,)).copy()

    def free(self, states):
        for i in range(len(states)):
            lib.vxo_spec_free(C.byref(self._s), C.byref(states[i]))
