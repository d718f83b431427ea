"""CPU checks that pin the oracle (oracle/vxo.c) to the reference's known
answers and to what the mathematics fixes: closed forms, independent dense
restatements (float64 numpy), invariants and exact special cases.  Each test
names what would fail if the oracle dropped a term, transposed an operand or
mis-indexed a page."""
import math

import numpy as np
import pytest

import vxo
from refgen import quantize_mlx_4bit, rand_vec, dequant, assert_close


# ------------------------------------------------------------------- packing
def test_pack_known_answer():
    # dyn_quant.rs:205-218: ramp 0..15 packs to [0x76543210, 0xFEDCBA98]
    p = vxo.pack_int4(np.arange(16, dtype=np.uint32).reshape(1, 16))
    assert p.tolist() == [[0x76543210, 0xFEDCBA98]]
    codes = np.random.default_rng(0).integers(0, 16, size=(5, 64)).astype(np.uint32)
    assert np.array_equal(vxo.unpack_int4(vxo.pack_int4(codes)), codes)


def test_pages_total_bytes_and_allocator():
    from velox_amd.engine import PagedKvCache

    # pages.rs:295-301: 2 layers * 2 * 16 pages * 4 heads * 4 slots * 8 dim * 4 B
    assert PagedKvCache.total_bytes(2, 4, 8, 4, 16, elem_bytes=4) == 32768
    p = vxo.Pages(2, 4, 8, 4, 8)  # pages.rs:272-284
    assert p.num_free() == 8
    got = p.alloc(3)
    assert got.tolist() == [0, 1, 2], "LIFO free list pops page 0 first"
    assert p.num_free() == 5
    p.free(got)
    assert p.num_free() == 8
    q = vxo.Pages(2, 4, 8, 4, 2)  # pages.rs:286-293: all-or-nothing
    assert q.alloc(2) is not None
    assert q.alloc(1) is None and q.num_free() == 0


# ------------------------------------------------------------------ numerics
def test_philox_known_answers():
    # Random123 Philox4x32-10 known-answer vectors (Salmon et al., SC'11)
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert vxo.philox(ctr, key).tolist() == want


def test_philox_matches_rocrand_fixture():
    import json
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "philox_rocrand.json")
    data = json.load(open(path))
    for case in data["cases"]:
        assert vxo.philox(case["ctr"], case["key"]).tolist() == case["out"]


def test_uniforms_layout():
    u = vxo.spec_uniforms(2, 0, 0, 3, 4)
    assert u.shape == (3, 5, 4) and (u >= 0).all() and (u < 1).all()
    r = vxo.philox([1, 0, 2, 0], [2, 0])
    assert np.allclose(u[1, 2], (r >> 8).astype(np.float64) / 2**24)


def test_deterministic_exp_accuracy():
    xs = np.concatenate([np.linspace(-87, 0, 40001), np.linspace(0, 88, 4001)]).astype(np.float32)
    worst = 0
    for x in xs[::3]:
        a = np.float32(vxo.expf(float(x)))
        b = np.float32(math.exp(float(x)))
        worst = max(worst, abs(int(a.view(np.int32)) - int(b.view(np.int32))))
    assert worst <= 2, f"{worst} ulp"
    assert vxo.expf(-88.0) == 0.0 and vxo.expf(0.0) == 1.0 and math.isinf(vxo.expf(90.0))


def test_round_to_dtypes():
    x = np.array([1.0, 1 + 2**-9, 1 + 3 * 2**-9, 65520.0, -2.5e-3, 6e-8], np.float32)
    bf = vxo.round_to(x, vxo.BF16)  # 8 significant bits, ties to even
    assert bf[:4].tolist() == [1.0, 1.0, 1 + 2**-7, 65536.0]
    assert abs(bf[4] - x[4]) <= 2**-9 * abs(x[4])
    f16 = vxo.round_to(x, vxo.F16)  # numpy's float16 conversion is IEEE RNE
    with np.errstate(over="ignore"):
        assert np.array_equal(f16, x.astype(np.float16).astype(np.float32))
    assert math.isinf(f16[3]) and f16[1] == 1 + 2**-9


# ---------------------------------------------------------------------- qmm
def test_qmm_matches_dense_matmul():
    # metal_qmm_4bit_parity.rs:107-133
    m, n, k, g = 3, 64, 128, 64
    x = rand_vec(m * k, 1).reshape(m, k)
    qw, sc, bi = quantize_mlx_4bit(rand_vec(n * k, 2), n, k, g)
    y = vxo.qmm_4bit(x, qw, sc, bi, None, g)
    ref = x.astype(np.float64) @ dequant(qw, sc, bi, g).T
    assert_close("cpu vs dense", y, ref, 1e-3, 1e-3)


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_qmm_group_sizes_and_bias(gs):
    m, n, k = 2, 40, 256
    x = rand_vec(m * k, 41).reshape(m, k)
    qw, sc, bi = quantize_mlx_4bit(rand_vec(n * k, 42), n, k, gs)
    bias = rand_vec(n, 43)
    y = vxo.qmm_4bit(x, qw, sc, bi, bias, gs)
    ref = x.astype(np.float64) @ dequant(qw, sc, bi, gs).T + bias
    assert_close("bias", y, ref, 1e-4, 1e-4)


def test_qmm_special_cases():
    rng = np.random.default_rng(0)
    m, n, k = 4, 8, 256
    x = rng.standard_normal((m, k)).astype(np.float32)
    sc = rng.uniform(0.002, 0.02, size=(n, k // 64)).astype(np.float32)
    bi = rng.normal(0, 0.01, size=(n, k // 64)).astype(np.float32)
    zero = np.zeros((n, k // 8), np.uint32)
    y = vxo.qmm_4bit(x, zero, sc, bi)
    xs = x.reshape(m, k // 64, 64).astype(np.float64).sum(axis=2)
    assert np.allclose(y, xs @ bi.T.astype(np.float64), atol=1e-5)  # q == 0: y = sum_g b_g sum x
    qw = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    full = vxo.qmm_4bit(x, qw, sc, bi)
    for i in range(m):  # rows are independent: M=1 equals the row of M>1 bit-for-bit
        assert np.array_equal(vxo.qmm_4bit(x[i:i + 1], qw, sc, bi), full[i:i + 1])
    # threads only split the output features: results are bit-identical
    assert np.array_equal(vxo.qmm_4bit(x, qw, sc, bi, threads=4), full)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        vxo.qmm_4bit(x[:, :12], qw[:, :1], sc, bi)


# ---------------------------------------------------------------- attention
def dense_attention(q, k_pool, v_pool, bt, cu, kvo, scale, tree_mask=None, window=0):
    """float64 attention over gathered K/V with an explicit visibility matrix
    (the reference's non-fused path qwen3.rs:518-541 + build_causal_mask :868-884)."""
    total, hq, d = q.shape
    _, hk, ps, _ = k_pool.shape
    g = hq // hk
    out = np.zeros((total, hq, d))
    for s in range(len(kvo)):
        lo, hi = cu[s], cu[s + 1]
        r = hi - lo
        off = kvo[s]
        nkv = off + r
        pos = np.arange(nkv)
        pages = bt[s][pos // ps]
        K = k_pool[pages, :, pos % ps, :].astype(np.float64)  # [nkv, hk, d]
        V = v_pool[pages, :, pos % ps, :].astype(np.float64)
        for t in range(r):
            if tree_mask is None:
                vis = pos <= off + t
            else:
                vis = (pos < off) | ((pos >= off) & (((tree_mask[lo + t] >> np.clip(pos - off, 0, 63).astype(np.uint64)) & 1) == 1))
            if window:
                vis &= pos >= off + t + 1 - window
            for h in range(hq):
                sc = K[:, h // g, :] @ q[lo + t, h].astype(np.float64) * scale
                sc = np.where(vis, sc, -np.inf)
                p = np.exp(sc - sc.max())
                out[lo + t, h] = (p / p.sum()) @ V[:, h // g, :]
    return out


def _attn_inputs(seed, n_rows, offs, hq=4, hk=2, d=32, ps=4, extra=3):
    rng = np.random.default_rng(seed)
    nb = [(o + r + ps - 1) // ps for o, r in zip(offs, n_rows)]
    P = sum(nb) + extra
    perm = rng.permutation(P)
    bt = np.zeros((len(offs), max(nb)), np.uint32)
    c = 0
    for s, n in enumerate(nb):
        bt[s, :n] = perm[c:c + n]
        c += n
    cu = np.concatenate([[0], np.cumsum(n_rows)]).astype(np.uint32)
    q = rng.standard_normal((cu[-1], hq, d)).astype(np.float32)
    kp = rng.standard_normal((P, hk, ps, d)).astype(np.float32)
    vp = rng.standard_normal((P, hk, ps, d)).astype(np.float32)
    return q, kp, vp, bt, cu, np.array(offs, np.uint32)


def test_attention_matches_dense_causal():
    q, kp, vp, bt, cu, kvo = _attn_inputs(0, [5, 1, 7], [9, 0, 22])
    got = vxo.paged_attention(q, kp, vp, bt, cu, kvo, 0.3)
    assert np.allclose(got, dense_attention(q, kp, vp, bt, cu, kvo, 0.3), atol=2e-5)


def test_attention_matches_dense_tree_and_window():
    par = [-1, 0, 0, 1, 1, 2, 3]
    masks, depth = vxo.tree_masks(np.array(par, np.int32))
    assert depth.tolist() == [0, 1, 1, 2, 2, 2, 3]
    assert masks[6] == (1 << 6) | (1 << 3) | (1 << 1) | 1
    q, kp, vp, bt, cu, kvo = _attn_inputs(1, [7, 7], [5, 13])
    tm = np.tile(masks, 2)
    got = vxo.paged_attention(q, kp, vp, bt, cu, kvo, 0.25, tree_mask=tm)
    assert np.allclose(got, dense_attention(q, kp, vp, bt, cu, kvo, 0.25, tree_mask=tm), atol=2e-5)
    got = vxo.paged_attention(q, kp, vp, bt, cu, kvo, 0.25, sliding_window=6)
    assert np.allclose(got, dense_attention(q, kp, vp, bt, cu, kvo, 0.25, window=6), atol=2e-5)


def test_attention_invariants():
    q, kp, vp, bt, cu, kvo = _attn_inputs(2, [4, 4], [6, 3])
    base = vxo.paged_attention(q, kp, vp, bt, cu, kvo, 0.2)
    # chain tree == causal, bit-for-bit
    chain = vxo.tree_masks(np.array([-1, 0, 1, 2], np.int32))[0]
    assert np.array_equal(vxo.paged_attention(q, kp, vp, bt, cu, kvo, 0.2, tree_mask=np.tile(chain, 2)), base)
    # relabelling physical pages (pool permutation + table remap) changes nothing
    P = kp.shape[0]
    perm = np.random.default_rng(3).permutation(P)
    inv = np.argsort(perm)
    got = vxo.paged_attention(q, kp[perm], vp[perm], inv[bt].astype(np.uint32), cu, kvo, 0.2)
    assert np.array_equal(got, base)
    # a single visible key returns its V row (metal_decode_parity.rs:239-256)
    one = vxo.paged_attention(q[:1], kp, vp, bt[:1], np.array([0, 1], np.uint32), np.array([0], np.uint32), 0.2)
    page = bt[0, 0]
    assert np.allclose(one[0], np.repeat(vp[page, :, 0, :], 2, axis=0), atol=1e-6)


# ---------------------------------------------------------------------- rope
def test_rope_tables_closed_form():
    # qwen3.rs:281-293: inv = 1f32 / (theta.powf(i/d) as f32); freqs = t * inv in f32
    c, s = vxo.rope_tables(4096, 128, 1e6)
    inv = np.float32(1.0) / (1e6 ** (np.arange(0, 128, 2) / 128)).astype(np.float32)
    arg = np.arange(4096, dtype=np.float32)[:, None] * inv[None, :]
    assert np.allclose(c, np.cos(arg.astype(np.float64)), atol=1.2e-7, rtol=0)
    assert np.allclose(s, np.sin(arg.astype(np.float64)), atol=1.2e-7, rtol=0)
    assert (c[0] == 1).all() and (s[0] == 0).all()


def test_rope_apply_is_complex_rotation():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 2, 16)).astype(np.float32)
    c, s = vxo.rope_tables(32, 16, 1e4)
    pos = np.array([0, 5, 31], np.uint32)
    y = vxo.rope_apply(x, c, s, pos)
    z = (x[..., :8] + 1j * x[..., 8:]) * np.exp(1j * np.arctan2(s[pos], c[pos]))[:, None, :]
    assert np.allclose(y, np.concatenate([z.real, z.imag], axis=-1), atol=1e-5)
    assert np.array_equal(y[0], x[0])  # offset 0 is the identity


def test_kv_scatter_exact():
    pool = np.random.default_rng(0).standard_normal((4, 2, 4, 8)).astype(np.float32)
    val = np.random.default_rng(1).standard_normal((2, 2, 8)).astype(np.float32)
    out = vxo.kv_scatter(pool, val, np.array([3, 0], np.uint32), np.array([1, 2], np.uint32))
    ref = pool.copy()
    ref[3, :, 1] = val[0]
    ref[0, :, 2] = val[1]
    assert np.array_equal(out, ref)


# ---------------------------------------------------------------- acceptance
def test_argmax_semantics():
    assert vxo.argmax(np.array([1, 3, 3, 2], np.float32)) == 1  # first index wins ties
    assert vxo.argmax(np.array([np.nan, 1, np.nan, 0.5], np.float32)) == 1  # NaN never wins
    assert vxo.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert vxo.argmax(np.array([np.nan, np.nan], np.float32)) == 0


def test_accept_greedy_cases():
    V = 10
    lg = np.zeros((2, 4, V), np.float32)
    am = [[3, 7, 1, 9], [2, 2, 5, 0]]
    for b in range(2):
        for i in range(4):
            lg[b, i, am[b][i]] = 1
    acc, tok = vxo.accept_greedy(lg, np.array([[3, 7, 4], [2, 2, 5]], np.uint32))
    assert acc.tolist() == [2, 3]
    assert tok[0, :3].tolist() == [3, 7, 1] and tok[1].tolist() == [2, 2, 5, 0]


def test_stochastic_identical_distributions_accept_all():
    rng = np.random.default_rng(0)
    B, k, V = 8, 4, 3000
    tl = rng.normal(0, 2, size=(B, k + 1, V)).astype(np.float32)
    dl = tl[:, :k].copy()
    uni = vxo.spec_uniforms(5, 0, 0, B, k)
    cand = vxo.sample_draft(dl, uni, 1.25)
    acc, tok = vxo.accept_stochastic(tl, dl, cand, uni, 1.25)
    assert (acc == k).all()
    assert np.array_equal(tok[:, :k], cand)


def test_stochastic_output_distribution_is_target():
    """Speculative sampling emits tokens distributed as p (Leviathan et al.
    2023, Thm 1).  Small vocab, many independent sequences, chi-square."""
    V, B = 6, 40000
    lt = np.array([1.0, 0.2, -0.5, 2.0, 0.0, -1.0], np.float32)
    ld = np.array([0.0, 1.5, 0.5, 0.5, -2.0, 0.3], np.float32)
    T = 1.0
    tl = np.broadcast_to(lt, (B, 2, V)).copy()
    dl = np.broadcast_to(ld, (B, 1, V)).copy()
    rng = np.random.default_rng(1)
    uni = rng.random((B, 2, 4)).astype(np.float32)
    cand = vxo.sample_draft(dl, uni, 1.0 / T)
    acc, tok = vxo.accept_stochastic(tl, dl, cand, uni, 1.0 / T)
    first = tok[:, 0]
    p = np.exp(lt - lt.max())
    p /= p.sum()
    counts = np.bincount(first, minlength=V)
    chi2 = (((counts - B * p) ** 2) / (B * p)).sum()
    assert chi2 < 25.0, (chi2, counts, B * p)  # 5 dof, p-value ~1e-4
    q = np.exp(ld - ld.max())
    q /= q.sum()
    rate = np.minimum(1, p / q) @ q
    assert abs(acc.mean() - rate) < 0.02


def test_tree_accept_walk():
    par = np.array([-1, 0, 0, 1, 2, 2], np.int32)
    V = 8
    lg = np.zeros((1, 6, V), np.float32)
    for node, best in enumerate([5, 1, 6, 0, 4, 2]):
        lg[0, node, best] = 1
    nodes = np.array([[9, 3, 5, 0, 7, 6]], np.uint32)  # root -> node 2 (5) -> node 5 (6) -> stop
    acc, path, tok = vxo.accept_tree(lg, par, nodes)
    assert acc[0] == 2 and path[0, :3].tolist() == [0, 2, 5] and tok[0, :3].tolist() == [5, 6, 2]
    # a chain tree reduces to the greedy chain
    chain = np.array([-1, 0, 1, 2], np.int32)
    lg = np.random.default_rng(0).standard_normal((3, 4, 50)).astype(np.float32)
    am = lg.argmax(axis=2)
    cand = am[:, :3].astype(np.uint32)
    cand[1, 1] += 1
    a1, t1 = vxo.accept_greedy(lg, cand)
    a2, p2, t2 = vxo.accept_tree(lg, chain, np.concatenate([np.zeros((3, 1), np.uint32), cand], axis=1))
    assert np.array_equal(a1, a2)
    for b in range(3):
        assert np.array_equal(t1[b, : a1[b] + 1], t2[b, : a2[b] + 1])
