"""GPU parity of the gfx950 kernels against the CPU oracle.

Cases and tolerances follow the reference's own Metal parity tests
(tests/metal_qmm_4bit_parity.rs, metal_decode_parity.rs,
metal_batched_kernels_parity.rs) on the same LCG inputs, plus the benchmark
configs' shapes (config 1 int4 verify GEMMs, config 2 acceptance, config 3 tree
masks).  Integer outputs (tokens, accept decisions, scatter bytes) must match
bit-exactly.
"""
import numpy as np
import pytest
import torch

import vxo
from refgen import assert_allclose_elementwise, assert_close, quantize_mlx_4bit, rand_vec

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
OD = {"f32": vxo.F32, "f16": vxo.F16, "bf16": vxo.BF16}


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def host(t):
    return t.float().cpu().numpy()


# ---------------------------------------------------------------- qmm_4bit
QMM_REF_CASES = [
    # (dtype, m, n, k, seed_x, seed_w, seed_bias, atol, rtol)  metal_qmm_4bit_parity.rs
    ("bf16", 4, 256, 1024, 11, 12, None, 5e-2, 5e-2),
    ("f16", 2, 128, 512, 21, 22, None, 1e-2, 1e-2),
    ("f32", 1, 64, 128, 31, 32, None, 1e-4, 1e-4),
    ("bf16", 2, 128, 512, 41, 42, 43, 5e-2, 5e-2),
    ("bf16", 8, 3072, 1024, 51, 52, None, 0.5, 0.05),
]


@pytest.mark.parametrize("case", QMM_REF_CASES, ids=lambda c: f"{c[0]}-m{c[1]}n{c[2]}k{c[3]}")
def test_qmm_reference_cases(cuda, case):
    dt, m, n, k, sx, sw, sb, atol, rtol = case
    x = rand_vec(m * k, sx).reshape(m, k)
    w = rand_vec(n * k, sw)
    qw, sc, bi = quantize_mlx_4bit(w, n, k, 64)
    bias = rand_vec(n, sb) if sb is not None else None
    cpu = vxo.qmm_4bit(x, qw, sc, bi, bias, 64)
    y = __import__("velox_amd.ops", fromlist=["x"]).qmm_4bit(
        dev(x, TD[dt]), u32(qw), dev(sc, TD[dt]), dev(bi, TD[dt]),
        None if bias is None else dev(bias, TD[dt]), 64)
    assert_close(f"qmm {dt}", host(y), cpu, atol, rtol)


QMV_CASES = [  # metal_qmv_mlx_parity.rs:124-155 (M = 1, the draft's matvec), tolerances :99-104
    ("f32", 4096, 4096, 0x1234, 1e-3, 1e-4),
    ("f16", 4096, 4096, 0x5678, 5e-2, 5e-3),
    ("bf16", 4096, 4096, 0xABCD, 5e-1, 1e-2),
    ("f32", 3072, 3072, 0xFEED, 1e-3, 1e-4),
    ("f16", 14336, 4096, 0xBEEF, 5e-2, 5e-3),
    ("f32", 8, 512, 0x1357, 1e-3, 1e-4),
]


@pytest.mark.parametrize("case", QMV_CASES, ids=lambda c: f"{c[0]}-n{c[1]}k{c[2]}")
def test_qmm_m1_reference_cases(cuda, case):
    """One-row qmm_4bit against the oracle on the reference's qmv cases
    (x and w from rand_vec(seed), rand_vec(seed + 1); the oracle takes the
    unrounded f32 values, as the reference's CPU side does)."""
    from velox_amd import ops

    dt, n, k, seed, atol, rtol = case
    x = rand_vec(k, seed).reshape(1, k)
    qw, sc, bi = quantize_mlx_4bit(rand_vec(n * k, seed + 1), n, k, 64)
    cpu = vxo.qmm_4bit(x, qw, sc, bi, None, 64, threads=8)
    y = ops.qmm_4bit(dev(x, TD[dt]), u32(qw), dev(sc, TD[dt]), dev(bi, TD[dt]), None, 64)
    assert_close(f"qmv {dt} {n}x{k}", host(y), cpu, atol, rtol)


def synth_linear(n, k, seed):
    from velox_amd import synth

    return synth.qlinear(seed, f"cfg1.{n}x{k}", n, k, 64)


CFG1_SHAPES = [(4608, 2560), (6144, 2560), (2560, 4096), (9728, 2560), (2560, 9728), (19456, 2560),
               (151936, 2560)]


def run_qmm(path, x, lin, n, out, residual=None, epilogue=None, round_dtype=None):
    """One f16 GEMM through the row-major MLX path (vx_qmm_4bit_ex) or the
    packed path the engine uses (vx_qmm_pack_4bit + vx_qmm_4bit_packed)."""
    from velox_amd import _lib, ops

    epi = _lib.EPI_STORE if epilogue is None else epilogue
    rdt = _lib.BF16 if round_dtype is None else round_dtype
    W, S, B = u32(lin["qweight"]), dev(lin["scales"]), dev(lin["biases"])
    if path == "row_major":
        return ops.qmm_4bit_ex(x, W, S, B, out, residual=residual, epilogue=epi, round_dtype=rdt)
    packed = ops.qmm_pack_4bit(W, S, B)
    return ops.qmm_4bit_packed(x, packed, n, out, residual=residual, epilogue=epi, round_dtype=rdt)


@pytest.mark.parametrize("path", ["mlx", "packed"])
@pytest.mark.parametrize("m", [5, 80])
@pytest.mark.parametrize("shape", CFG1_SHAPES, ids=lambda s: f"n{s[0]}k{s[1]}")
def test_qmm_config1_f16(cuda, m, shape, path):
    """Config 1: f16 activations ~N(0,1), seed 1; logits-style tolerance
    1e-2 + 1e-2|ref|.  `mlx`: the qmm_4bit drop-in on MLX tensors; `packed`:
    the engine's packed-weight kernel (f16 output rounding)."""
    from velox_amd import _lib, ops

    n, k = shape
    if path == "packed" and n % 32:
        pytest.skip("packed weights need N % 32 == 0")
    lin = synth_linear(n, k, 1)
    rng = np.random.Generator(np.random.Philox(key=[1, n * 7 + k]))
    x = rng.standard_normal((m, k)).astype(np.float16)
    if path == "mlx":
        y = ops.qmm_4bit(dev(x), u32(lin["qweight"]), dev(lin["scales"]), dev(lin["biases"]), None, 64)
        torch.cuda.synchronize()
        y2 = ops.qmm_4bit(dev(x), u32(lin["qweight"]), dev(lin["scales"]), dev(lin["biases"]), None, 64)
    else:
        y = torch.empty((m, n), dtype=torch.float16, device="cuda")
        y2 = torch.empty_like(y)
        run_qmm("packed", dev(x), lin, n, y, round_dtype=_lib.F16)
        torch.cuda.synchronize()
        run_qmm("packed", dev(x), lin, n, y2, round_dtype=_lib.F16)
    assert torch.equal(y, y2), "split-K reduction must be deterministic"
    cols = np.arange(n) if n <= 20000 else np.sort(np.random.default_rng(0).choice(n, 4096, replace=False))
    cpu = vxo.qmm_4bit(x.astype(np.float32), lin["qweight"][cols], lin["scales"][cols].astype(np.float32),
                       lin["biases"][cols].astype(np.float32), None, 64, threads=8)
    got = host(y)[:, cols]
    assert_allclose_elementwise(f"cfg1 m{m} {n}x{k}", got, vxo.round_to(cpu, vxo.F16), 1e-2, 1e-2)


QWEN3_8B_SHAPES = [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288), (151936, 4096)]


@pytest.mark.parametrize("m", [7, 32, 224, 600])
@pytest.mark.parametrize("shape", QWEN3_8B_SHAPES, ids=lambda s: f"n{s[0]}k{s[1]}")
def test_qmm_qwen3_8b_shapes(cuda, m, shape):
    """Config 4's GEMMs (Qwen3-8B: qkv, o, gate|up, down, LM head) on the
    packed path at the k = 6 verify row counts (7 per sequence, 224 for 32
    sequences), the 32-row draft and a 600-row prefill chunk; columns sampled
    for the oracle."""
    from velox_amd import _lib

    n, k = shape
    lin = synth_linear(n, k, 2)
    rng = np.random.Generator(np.random.Philox(key=[2, n * 7 + k + m]))
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    run_qmm("packed", dev(x), lin, n, y, round_dtype=_lib.F16)
    cols = np.sort(np.random.default_rng(m).choice(n, 1024, replace=False))
    cpu = vxo.qmm_4bit(x.astype(np.float32), lin["qweight"][cols], lin["scales"][cols].astype(np.float32),
                       lin["biases"][cols].astype(np.float32), None, 64, threads=8)
    assert_allclose_elementwise(f"8b m{m} {n}x{k}", host(y)[:, cols], vxo.round_to(cpu, vxo.F16), 1e-2, 1e-2)


@pytest.mark.parametrize("m", [1, 5, 16, 80, 97])
def test_qmm_bf16_fast_path_shapes(cuda, m):
    """bf16 activations (the reference's bf16 contract) through the MFMA path."""
    from velox_amd import ops

    n, k = 2560, 2560
    lin = synth_linear(n, k, 5)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    xb = vxo.round_to(x, vxo.BF16)
    sc = vxo.round_to(lin["scales"].astype(np.float32), vxo.BF16)
    bi = vxo.round_to(lin["biases"].astype(np.float32), vxo.BF16)
    y = ops.qmm_4bit(dev(xb, torch.bfloat16), u32(lin["qweight"]), dev(sc, torch.bfloat16),
                     dev(bi, torch.bfloat16), None, 64)
    cpu = vxo.qmm_4bit(xb, lin["qweight"], sc, bi, None, 64, threads=8)
    assert_allclose_elementwise(f"bf16 m{m}", host(y), cpu, 2e-2, 1e-2)


@pytest.mark.parametrize("path,m", [("row_major", 80), ("packed", 1), ("packed", 16), ("packed", 33),
                                    ("packed", 80), ("packed", 97)])
def test_qmm_epilogues(cuda, path, m):
    """Residual and SwiGLU epilogues of the fused verify forward (f16 X, bf16
    rounding), through the row-major and the packed paths; packed row counts
    cover 1-3 row tiles of 32 and several row blocks."""
    from velox_amd import _lib

    k, f = 2560, 1024
    gate = synth_linear(f, k, 7)
    up = synth_linear(f, k, 8)
    x = vxo.round_to(np.random.default_rng(3).standard_normal((m, k)).astype(np.float32), vxo.BF16)
    # interleave 16-row blocks gate|up as the engine does
    qw = np.concatenate([np.stack([gate["qweight"][i:i + 16], up["qweight"][i:i + 16]]).reshape(32, -1)
                         for i in range(0, f, 16)])
    sc = np.concatenate([np.stack([gate["scales"][i:i + 16], up["scales"][i:i + 16]]).reshape(32, -1)
                         for i in range(0, f, 16)])
    bi = np.concatenate([np.stack([gate["biases"][i:i + 16], up["biases"][i:i + 16]]).reshape(32, -1)
                         for i in range(0, f, 16)])
    out = torch.zeros((m, f), dtype=torch.float16, device="cuda")
    run_qmm(path, dev(x, torch.float16), {"qweight": qw, "scales": sc, "biases": bi}, 2 * f, out,
            epilogue=_lib.EPI_SWIGLU)
    g = vxo.round_to(vxo.qmm_4bit(x, gate["qweight"], gate["scales"].astype(np.float32),
                                  gate["biases"].astype(np.float32), None, 64, 8), vxo.BF16)
    u = vxo.round_to(vxo.qmm_4bit(x, up["qweight"], up["scales"].astype(np.float32),
                                  up["biases"].astype(np.float32), None, 64, 8), vxo.BF16)
    silu = vxo.round_to(g / (1 + np.exp(-g.astype(np.float64))).astype(np.float32), vxo.BF16)
    ref = vxo.round_to(silu * u, vxo.BF16)
    # g and u each carry the GEMM parity bound (1e-2 absolute) plus one bf16
    # ulp (their rounding to bf16 can flip); the product propagates it as
    # |silu(g)| e_u + |u| |silu'(g)| e_g (|silu'| <= 1.1), plus bf16 output
    # rounding.
    def ulp(v):
        return 2.0 ** (np.floor(np.log2(np.abs(v) + 1e-30)) - 7)

    e_g, e_u = 1e-2 + ulp(g), 1e-2 + ulp(u)
    bound = np.abs(silu) * e_u + 1.1 * np.abs(u) * e_g + 1e-2 * np.abs(ref) + 1e-3
    d = np.abs(host(out) - ref)
    assert (d <= bound).all(), f"swiglu: {int((d > bound).sum())} elements beyond the propagated bound"
    # residual: y = round(R + round(acc))
    o = synth_linear(1024, k, 9)
    r = vxo.round_to(np.random.default_rng(4).standard_normal((m, 1024)).astype(np.float32) * 100, vxo.BF16)
    rt = dev(r, torch.bfloat16)
    run_qmm(path, dev(x, torch.float16), o, 1024, rt, residual=rt, epilogue=_lib.EPI_RESIDUAL)
    acc = vxo.round_to(vxo.qmm_4bit(x, o["qweight"], o["scales"].astype(np.float32),
                                    o["biases"].astype(np.float32), None, 64, 8), vxo.BF16)
    ref = vxo.round_to(r + acc, vxo.BF16)
    # the GEMM bound (1e-2) plus one bf16 ulp of the rounded GEMM output and of the sum
    bound = 1e-2 + ulp(acc) + ulp(ref) + 1e-2 * np.abs(ref)
    d = np.abs(host(rt) - ref)
    assert (d <= bound).all(), f"residual: {int((d > bound).sum())} elements beyond the propagated bound"


def unpack_blocks(packed, n, k):
    """Decode the packed layout back to MLX tensors, independently of the GEMM
    kernels: per (32-row tile, 128-wide k step) a 2304-byte block; bytes
    [0, 2048) hold lane L's words j = 0..3 then 4..7 (16 bytes at 16 L and
    1024 + 16 L), lane L = (row L%32, k half L/32), word j = MLX word
    16 st + 2j + L/32 with the nibbles of k0..k7 at positions 0,4,1,5,2,6,3,7;
    bytes [2048, 2304) hold (s0, b0, s1, b1) per row."""
    T, S = n // 32, k // 128
    blk = packed.reshape(T, S, 2304)
    w = blk[:, :, :2048].copy().view(np.uint32).reshape(T, S, 2, 2, 32, 4)  # tile, step, part, kh, row, word
    pos = [0, 4, 1, 5, 2, 6, 3, 7]  # nibble position of k
    natural = np.zeros_like(w)
    for kk, p in enumerate(pos):
        natural |= ((w >> np.uint32(4 * p)) & np.uint32(0xF)) << np.uint32(4 * kk)
    # MLX word within the step = 8 part + 2 word + kh
    qw = natural.transpose(0, 4, 1, 2, 5, 3).reshape(n, k // 8)
    sb = blk[:, :, 2048:].copy().view(np.uint16).reshape(T, S, 32, 2, 2)  # tile, step, row, group, (s, b)
    sb = sb.transpose(0, 2, 1, 3, 4).reshape(n, k // 64, 2)
    return qw, sb[..., 0], sb[..., 1]


@pytest.mark.parametrize("shape", [(64, 256), (4608, 2560), (2560, 9728)], ids=lambda s: f"n{s[0]}k{s[1]}")
def test_qmm_pack_layout_round_trip(cuda, shape):
    """The packed blocks hold exactly the MLX words and f16 affine params."""
    from velox_amd import ops

    n, k = shape
    lin = synth_linear(n, k, 11)
    packed = ops.qmm_pack_4bit(u32(lin["qweight"]), dev(lin["scales"]), dev(lin["biases"]))
    qw, sc, bi = unpack_blocks(packed.cpu().numpy(), n, k)
    assert np.array_equal(qw, lin["qweight"].view(np.uint32))
    assert np.array_equal(sc, lin["scales"].view(np.uint16))
    assert np.array_equal(bi, lin["biases"].view(np.uint16))


def test_qmm_bias_rounds_once(cuda):
    """qmm_4bit with a bias rounds once (metal_kernels.rs:473-474:
    acc += bias; Y = (T)acc): the f16 result equals round_f16(acc + bias)
    bit for bit, where acc is the same GEMM's f32 accumulator (read through
    the extended entry point with f32 rounding and output)."""
    from velox_amd import _lib, ops

    m, n, k = 3, 256, 512
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.normal(0, 1, size=(m, k)).astype(np.float16)).cuda()
    lin = synth_linear(n, k, 13)
    qw = torch.from_numpy(lin["qweight"].view(np.int32)).cuda()
    sc = torch.from_numpy(lin["scales"]).cuda()
    bs = torch.from_numpy(lin["biases"]).cuda()
    bias = torch.from_numpy(rng.normal(0, 1, size=n).astype(np.float16)).cuda()
    y = ops.qmm_4bit(x, qw, sc, bs, bias=bias)
    acc = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.qmm_4bit_ex(x, qw, sc, bs, acc, round_dtype=_lib.F32)
    torch.cuda.synchronize()
    want = (acc.cpu().numpy() + bias.float().cpu().numpy()).astype(np.float16)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_prefill_rejects_inconsistent_seq_ids(cuda):
    """seq_id_per_q must name, for every row, the sequence whose cu_seqlens
    range holds it (the reference kernel reads it, MSL :307-395)."""
    from velox_amd import ops
    from velox_amd._lib import VeloxError

    q = torch.zeros(6, 4, 64, dtype=torch.float16, device="cuda")
    pool = torch.zeros(4, 2, 16, 64, dtype=torch.float16, device="cuda")
    bt = u32(np.array([[0, 1], [2, 3]]))
    cu = u32(np.array([0, 4, 6]))
    kvo = u32(np.array([0, 3]))
    ops.paged_prefill_attention(q, pool, pool, bt, cu, u32(np.array([0, 0, 0, 0, 1, 1])), kvo, 0.125)
    with pytest.raises(VeloxError, match="disagrees with cu_seqlens"):
        ops.paged_prefill_attention(q, pool, pool, bt, cu, u32(np.array([0, 0, 0, 1, 1, 1])), kvo, 0.125)
    with pytest.raises(VeloxError, match="disagrees with cu_seqlens"):
        ops.paged_prefill_attention(q, pool, pool, bt, cu, u32(np.array([0, 0, 0, 0, 1, 2])), kvo, 0.125)
    with pytest.raises(VeloxError, match="run from 0 to total_q"):
        ops.paged_prefill_attention(q, pool, pool, bt, u32(np.array([0, 4, 5])), u32(np.zeros(6)), kvo, 0.125)


def test_qmm_validation_errors(cuda):
    from velox_amd import ops
    from velox_amd._lib import VeloxError

    x = torch.zeros((2, 12), dtype=torch.float16, device="cuda")
    with pytest.raises(VeloxError, match="multiple of 8"):
        ops.qmm_4bit(x, torch.zeros((4, 1), dtype=torch.int32, device="cuda"),
                     torch.zeros((4, 1), dtype=torch.float16, device="cuda"),
                     torch.zeros((4, 1), dtype=torch.float16, device="cuda"), None, 64)


# ---------------------------------------------------------------- attention
DECODE_CASES = [  # metal_decode_parity.rs:150-256
    ("f32", 1, 4, 2, 32, 4, 4, 2, [5], [0, 1], 42),
    ("f16", 2, 8, 2, 64, 8, 16, 3, [10, 21], [3, 5, 0, 0, 1, 2], 7),
    ("bf16", 4, 16, 8, 128, 16, 16, 5, [16, 32, 48, 64],
     [0, 1, 0, 0, 0, 2, 3, 0, 0, 0, 4, 5, 6, 0, 0, 7, 8, 9, 10, 0], 13),
    ("bf16", 8, 16, 8, 128, 64, 16, 16, [240] * 8, [((s * 16 + b) % 64) for s in range(8) for b in range(16)], 99),
    ("bf16", 2, 16, 8, 128, 4, 16, 1, [1, 1], [0, 1], 3),
]
DECODE_TOL = {"f32": (1e-4, 1e-4), "f16": (5e-3, 5e-3), "bf16": (3e-2, 3e-2)}


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: f"{c[0]}-n{c[1]}-d{c[4]}")
def test_decode_attention_reference_cases(cuda, case):
    from velox_amd import ops

    dt, n, hq, hk, d, p, ps, mb, kv_lens, bt, seed = case
    scale = 1.0 / np.sqrt(d)
    q = vxo.round_to(rand_vec(n * hq * d, seed), OD[dt]).reshape(n, hq, d)
    k = vxo.round_to(rand_vec(p * hk * ps * d, seed + 1), OD[dt]).reshape(p, hk, ps, d)
    v = vxo.round_to(rand_vec(p * hk * ps * d, seed + 2), OD[dt]).reshape(p, hk, ps, d)
    bt = np.array(bt, np.uint32).reshape(n, mb)
    out = ops.paged_decode_attention(dev(q, TD[dt]), dev(k, TD[dt]), dev(v, TD[dt]), u32(bt),
                                     u32(np.array(kv_lens, np.uint32)), scale)
    cu = np.arange(n + 1, dtype=np.uint32)
    kvo = np.array(kv_lens, np.uint32) - 1
    cpu = vxo.paged_attention(q, k, v, bt, cu, kvo, scale)
    atol, rtol = DECODE_TOL[dt]
    assert_close(f"decode {dt}", host(out), cpu, atol, rtol)


def test_sliding_window_decode_reference_case(cuda):
    """metal_swa_parity.rs:48-170: one bf16 decode row, kv_len 96, window 32
    (visible positions 64..95): matches the oracle and differs from the
    global result (the window is not silently ignored)."""
    from velox_amd import ops

    hq, hk, d, ps, mb, p, kv_len, window = 8, 4, 64, 16, 8, 8, 96, 32
    scale = 1.0 / np.sqrt(d)
    q = vxo.round_to(rand_vec(hq * d, 11), vxo.BF16).reshape(1, hq, d)
    k = vxo.round_to(rand_vec(p * hk * ps * d, 12), vxo.BF16).reshape(p, hk, ps, d)
    v = vxo.round_to(rand_vec(p * hk * ps * d, 13), vxo.BF16).reshape(p, hk, ps, d)
    bt = np.arange(mb, dtype=np.uint32).reshape(1, mb)
    args = (dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), u32(bt),
            u32(np.array([kv_len], np.uint32)), scale)
    swa = host(ops.paged_decode_attention(*args, sliding_window=window))
    glob = host(ops.paged_decode_attention(*args))
    cpu = vxo.paged_attention(q, k, v, bt, np.array([0, 1], np.uint32), np.array([kv_len - 1], np.uint32), scale,
                              sliding_window=window)
    assert_close("decode swa", swa, cpu, 3e-2, 3e-2)
    assert np.abs(glob - swa).max() > 1e-2, "the window did not change the output"


def test_sliding_window_prefill_reference_case(cuda):
    """metal_swa_parity.rs:173-258: four bf16 queries at kv_offset 80 with
    window 16 each see only the last 16 positions of their causal history."""
    from velox_amd import ops

    hq, hk, d, ps, mb, p, window = 8, 4, 64, 16, 8, 8, 16
    scale = 1.0 / np.sqrt(d)
    q = vxo.round_to(rand_vec(4 * hq * d, 41), vxo.BF16).reshape(4, hq, d)
    k = vxo.round_to(rand_vec(p * hk * ps * d, 42), vxo.BF16).reshape(p, hk, ps, d)
    v = vxo.round_to(rand_vec(p * hk * ps * d, 43), vxo.BF16).reshape(p, hk, ps, d)
    bt = np.arange(mb, dtype=np.uint32).reshape(1, mb)
    cu, sid, kvo = np.array([0, 4], np.uint32), np.zeros(4, np.uint32), np.array([80], np.uint32)
    args = (dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), u32(bt), u32(cu), u32(sid),
            u32(kvo), scale)
    swa = host(ops.paged_prefill_attention(*args, sliding_window=window))
    glob = host(ops.paged_prefill_attention(*args))
    cpu = vxo.paged_attention(q, k, v, bt, cu, kvo, scale, sliding_window=window)
    assert_close("prefill swa", swa, cpu, 3e-2, 3e-2)
    assert np.abs(glob - swa).max() > 1e-2, "the window did not change the output"


def _prefill_case(new_lens, kv_offsets, bt, p, seed, dt="bf16", hq=16, hk=8, d=128, ps=16, tree=None):
    from velox_amd import ops

    cu = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.uint32)
    total = int(cu[-1])
    sid = np.repeat(np.arange(len(new_lens)), new_lens).astype(np.uint32)
    scale = 1.0 / np.sqrt(d)
    q = vxo.round_to(rand_vec(total * hq * d, seed), OD[dt]).reshape(total, hq, d)
    k = vxo.round_to(rand_vec(p * hk * ps * d, seed + 1), OD[dt]).reshape(p, hk, ps, d)
    v = vxo.round_to(rand_vec(p * hk * ps * d, seed + 2), OD[dt]).reshape(p, hk, ps, d)
    bt = np.asarray(bt, np.uint32).reshape(len(new_lens), -1)
    kvo = np.asarray(kv_offsets, np.uint32)
    tm = None
    if tree is not None:
        masks, _ = vxo.tree_masks(np.asarray(tree, np.int32))
        tm = np.tile(masks, len(new_lens))
    out = ops.paged_prefill_attention(dev(q, TD[dt]), dev(k, TD[dt]), dev(v, TD[dt]), u32(bt), u32(cu), u32(sid),
                                      u32(kvo), scale,
                                      tree_mask=None if tm is None else torch.from_numpy(tm.view(np.int64)).cuda())
    cpu = vxo.paged_attention(q, k, v, bt, cu, kvo, scale, tree_mask=tm)
    return host(out), cpu


def test_prefill_attention_one_seq(cuda):
    got, ref = _prefill_case([12], [0], [0, 0, 0, 0], 8, 21)  # metal_batched_kernels_parity.rs:246-295
    assert_close("prefill one seq", got, ref, 3e-2, 3e-2)


def test_prefill_attention_mixed_batch(cuda):
    got, ref = _prefill_case([8, 4, 1], [0, 20, 10], [0, 0, 0, 0, 2, 3, 0, 0, 4, 0, 0, 0], 16, 31)
    assert_close("prefill mixed batch", got, ref, 3e-2, 3e-2)


@pytest.mark.parametrize("ctx", [47, 300, 1100])
def test_verify_attention_chain_shuffled_pages(cuda, ctx):
    """Metric shape: 16 sequences x 5 verify rows, GQA 32/8, d=128, f16 KV,
    shuffled block tables; block-table permutation must not matter."""
    rng = np.random.default_rng(ctx)
    B, R, ps = 16, 5, 16
    nb = (ctx + R + ps - 1) // ps
    P = B * nb + 3
    perm = rng.permutation(P)[: B * nb].reshape(B, nb)
    offs = rng.integers(max(1, ctx - 40), ctx + 1, size=B)
    got, ref = _prefill_case([R] * B, offs, perm, P, 5, dt="f16", hq=32, hk=8)
    assert_allclose_elementwise("verify chain", got, ref, 1e-2, 1e-2)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_verify_attention_head_dims(cuda, d, dt):
    """Every head dim of the MFMA path (each stages V row-major with its own
    chunk permutation and reads it back transposed), shuffled pages, two key
    blocks per wave and a ragged last block."""
    rng = np.random.default_rng(d)
    B, R, ps, ctx = 3, 5, 16, 520
    nb = (ctx + R + ps - 1) // ps
    P = B * nb + 2
    perm = rng.permutation(P)[: B * nb].reshape(B, nb)
    got, ref = _prefill_case([R] * B, [ctx - 7, ctx - 90, ctx], perm, P, 17 + d, dt=dt, hq=8, hk=2, d=d)
    tol = 1e-2 if dt == "f16" else 3e-2
    assert_allclose_elementwise(f"verify d={d} {dt}", got, ref, tol, tol)


def tree_4_2_2():
    """16 draft nodes (4 + 8 + 4) under the root: node 0 = root, depth-1 nodes
    1-4, each with 2 children (5-12), and nodes 5 and 6 each with 2 children
    (13-16)."""
    par = [-1, 0, 0, 0, 0]
    for p in range(1, 5):
        par += [p, p]
    for p in (5, 6):
        par += [p, p]
    return par


def test_verify_attention_tree(cuda):
    par = tree_4_2_2()
    R, B, ps, ctx = len(par), 4, 16, 200
    nb = (ctx + R + ps - 1) // ps
    rng = np.random.default_rng(3)
    perm = rng.permutation(B * nb).reshape(B, nb)
    got, ref = _prefill_case([R] * B, [ctx] * B, perm, B * nb, 9, dt="f16", hq=32, hk=8, tree=par)
    assert_allclose_elementwise("tree attention", got, ref, 1e-2, 1e-2)


def test_tree_attention_config3_geometry(cuda):
    """Config 3 at its own geometry: 16 sequences at context 2048, each
    verifying the 4-2-2 tree plus its root (17 rows, 68 query vectors per KV
    head: the 32-vector query tiles and the KV-split merge both run), GQA
    32/8, head_dim 128, f16 KV on a shuffled block table."""
    par = tree_4_2_2()
    R, B, ps, ctx = len(par), 16, 16, 2048
    nb = (ctx + R + ps - 1) // ps
    rng = np.random.default_rng(33)
    P = B * nb + 5
    perm = rng.permutation(P)[: B * nb].reshape(B, nb)
    got, ref = _prefill_case([R] * B, [ctx] * B, perm, P, 303, dt="f16", hq=32, hk=8, tree=par)
    assert_allclose_elementwise("config-3 tree attention", got, ref, 1e-2, 1e-2)


def test_chain_attention_config4_geometry(cuda):
    """Config 4's verify attention: 32 sequences, k = 6 (7 rows each),
    contexts up to 4096 tokens, and the first 512 tokens (32 pages) shared by
    every group of 8 sequences through their block tables, the rest of each
    table on shuffled private pages."""
    B, R, ps, k_shared = 32, 7, 16, 32
    rng = np.random.default_rng(44)
    ctx = rng.integers(600, 4096 - R, size=B)
    ctx[0] = 4096 - R
    nb = (ctx + R + ps - 1) // ps
    groups = B // 8
    private = int((nb - k_shared).sum())
    P = groups * k_shared + private + 3
    perm = rng.permutation(P)
    shared = perm[: groups * k_shared].reshape(groups, k_shared)
    own = perm[groups * k_shared:]
    mb = int(nb.max())
    bt = np.zeros((B, mb), np.uint32)
    o = 0
    for b in range(B):
        bt[b, :k_shared] = shared[b // 8]
        n_own = int(nb[b]) - k_shared
        bt[b, k_shared: k_shared + n_own] = own[o: o + n_own]
        o += n_own
    got, ref = _prefill_case([R] * B, ctx, bt, P, 404, dt="f16", hq=32, hk=8)
    assert_allclose_elementwise("config-4 chain attention", got, ref, 1e-2, 1e-2)


def test_chain_tree_equals_causal(cuda):
    chain = [-1, 0, 1, 2, 3]
    a, _ = _prefill_case([5, 5], [30, 61], [1, 2, 3, 4, 5, 6, 7, 8, 9, 10], 11, 17, dt="f16", tree=chain)
    b, _ = _prefill_case([5, 5], [30, 61], [1, 2, 3, 4, 5, 6, 7, 8, 9, 10], 11, 17, dt="f16")
    assert np.array_equal(a, b)


# Sequences of 33..128 query vectors (rows x query heads per KV head) take the
# shared-KV kernel: one workgroup per (sequence, KV head, split) stages each
# key block once for all of them.
@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("splits", ["1", "3"])
def test_shared_kv_attention_head_dims(cuda, monkeypatch, d, dt, splits):
    """Causal rows, ragged per sequence (17, 9 and 12 rows x 4 query heads:
    68, 36 and 48 vectors), contexts that end mid-block, shuffled pages; one
    workgroup per item or three KV splits merged by the combine kernel."""
    monkeypatch.setenv("VX_ATTN_SHARED_SPLITS", splits)
    rng = np.random.default_rng(100 + d)
    rows, ps = [17, 9, 12], 16
    offs = [501, 430, 515]
    nb = (max(o + r for o, r in zip(offs, rows)) + ps - 1) // ps
    P = 3 * nb + 2
    perm = rng.permutation(P)[: 3 * nb].reshape(3, nb)
    got, ref = _prefill_case(rows, offs, perm, P, 61 + d, dt=dt, hq=8, hk=2, d=d)
    tol = 1e-2 if dt == "f16" else 3e-2
    assert_allclose_elementwise(f"shared-kv d={d} {dt} splits={splits}", got, ref, tol, tol)


@pytest.mark.parametrize("splits", ["1", "2"])
def test_shared_kv_attention_tree_bf16(cuda, monkeypatch, splits):
    """The 4-2-2 tree (68 vectors per KV head) in bf16 at d = 64, short
    contexts (the tree slots dominate the key range)."""
    monkeypatch.setenv("VX_ATTN_SHARED_SPLITS", splits)
    par = tree_4_2_2()
    R, B, ps = len(par), 3, 16
    offs = [0, 5, 70]
    nb = (max(offs) + R + ps - 1) // ps
    rng = np.random.default_rng(12)
    perm = rng.permutation(B * nb).reshape(B, nb)
    got, ref = _prefill_case([R] * B, offs, perm, B * nb, 19, dt="bf16", hq=8, hk=2, d=64, tree=par)
    assert_allclose_elementwise("shared-kv tree bf16", got, ref, 3e-2, 3e-2)


def test_shared_kv_attention_empty_sequence(cuda, monkeypatch):
    """A sequence with no rows between two that take the shared-KV kernel:
    its workgroups leave before any barrier and the merge skips it."""
    monkeypatch.setenv("VX_ATTN_SHARED_SPLITS", "3")
    rows, ps = [17, 0, 9], 16
    offs = [300, 50, 333]
    nb = (max(o + r for o, r in zip(offs, rows)) + ps - 1) // ps
    rng = np.random.default_rng(7)
    P = 3 * nb + 1
    perm = rng.permutation(P)[: 3 * nb].reshape(3, nb)
    got, ref = _prefill_case(rows, offs, perm, P, 29, dt="f16", hq=8, hk=2, d=128)
    assert_allclose_elementwise("shared-kv empty sequence", got, ref, 1e-2, 1e-2)


def test_shared_kv_attention_page_size_fallback(cuda):
    """A page size that is not a power of two (24) sends 68-vector sequences
    to the query-tile kernel instead; the 4-2-2 tree still matches the
    oracle."""
    par = tree_4_2_2()
    R, B, ps = len(par), 3, 24
    offs = [40, 101, 7]
    nb = (max(offs) + R + ps - 1) // ps
    rng = np.random.default_rng(24)
    perm = rng.permutation(B * nb + 1)[: B * nb].reshape(B, nb)
    got, ref = _prefill_case([R] * B, offs, perm, B * nb + 1, 23, dt="f16", hq=32, hk=8, ps=ps, tree=par)
    assert_allclose_elementwise("page size 24 tree", got, ref, 1e-2, 1e-2)


def test_shared_kv_attention_sliding_window(cuda):
    """Window 16 over 12 rows x 4 query heads (48 vectors, the shared-KV
    kernel) at kv_offset 80: matches the oracle and differs from the global
    result."""
    from velox_amd import ops

    hq, hk, d, ps, mb, p, window, R = 8, 2, 64, 16, 8, 8, 16, 12
    scale = 1.0 / np.sqrt(d)
    q = vxo.round_to(rand_vec(R * hq * d, 51), vxo.BF16).reshape(R, hq, d)
    k = vxo.round_to(rand_vec(p * hk * ps * d, 52), vxo.BF16).reshape(p, hk, ps, d)
    v = vxo.round_to(rand_vec(p * hk * ps * d, 53), vxo.BF16).reshape(p, hk, ps, d)
    bt = np.arange(mb, dtype=np.uint32).reshape(1, mb)
    cu, sid, kvo = np.array([0, R], np.uint32), np.zeros(R, np.uint32), np.array([80], np.uint32)
    args = (dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16), u32(bt), u32(cu), u32(sid),
            u32(kvo), scale)
    swa = host(ops.paged_prefill_attention(*args, sliding_window=window))
    glob = host(ops.paged_prefill_attention(*args))
    cpu = vxo.paged_attention(q, k, v, bt, cu, kvo, scale, sliding_window=window)
    assert_close("shared-kv swa", swa, cpu, 3e-2, 3e-2)
    assert np.abs(glob - swa).max() > 1e-2, "the window did not change the output"


def test_shared_kv_attention_matches_tiled(cuda, monkeypatch):
    """Config 3's geometry through both kernels (shared-KV and the 32-vector
    tiles, VX_ATTN_SHARED=0): the same attention up to f32 summation order."""
    par = tree_4_2_2()
    R, B, ps, ctx = len(par), 16, 16, 2048
    nb = (ctx + R + ps - 1) // ps
    rng = np.random.default_rng(34)
    P = B * nb + 5
    perm = rng.permutation(P)[: B * nb].reshape(B, nb)
    shared, ref = _prefill_case([R] * B, [ctx] * B, perm, P, 304, dt="f16", hq=32, hk=8, tree=par)
    monkeypatch.setenv("VX_ATTN_SHARED", "0")
    tiled, _ = _prefill_case([R] * B, [ctx] * B, perm, P, 304, dt="f16", hq=32, hk=8, tree=par)
    assert_allclose_elementwise("shared vs oracle", shared, ref, 1e-2, 1e-2)
    assert_allclose_elementwise("tiled vs oracle", tiled, ref, 1e-2, 1e-2)
    assert np.abs(shared.astype(np.float32) - tiled.astype(np.float32)).max() < 2e-3


# ---------------------------------------------------------------- rope / scatter
def test_rope_bf16_reference_case(cuda):
    from velox_amd import ops

    n, h, d, half, lmax = 4, 16, 128, 64, 1024  # metal_batched_kernels_parity.rs:78-111
    x = vxo.round_to(rand_vec(n * h * d, 1), vxo.BF16).reshape(n, h, d)
    c = vxo.round_to(rand_vec(lmax * half, 2), vxo.BF16).reshape(lmax, half)
    s = vxo.round_to(rand_vec(lmax * half, 3), vxo.BF16).reshape(lmax, half)
    off = np.array([0, 5, 100, 511], np.uint32)
    xt = dev(x, torch.bfloat16)
    ops.batched_rope_decode(xt, dev(c, torch.bfloat16), dev(s, torch.bfloat16), u32(off))
    cpu = vxo.rope_apply(x, c, s, off, vxo.BF16)
    assert_close("rope bf16", host(xt), cpu, 5e-2, 5e-2)
    assert np.array_equal(host(xt), cpu), "same arithmetic, same rounding: bit-identical"


def test_rope_f32_reference_case(cuda):
    from velox_amd import ops

    n, h, d, half, lmax = 2, 4, 64, 32, 256
    x = rand_vec(n * h * d, 5).reshape(n, h, d)
    c = rand_vec(lmax * half, 6).reshape(lmax, half)
    s = rand_vec(lmax * half, 7).reshape(lmax, half)
    off = np.array([3, 200], np.uint32)
    xt = dev(x)
    ops.batched_rope_decode(xt, dev(c), dev(s), u32(off))
    assert_close("rope f32", host(xt), vxo.rope_apply(x, c, s, off), 1e-5, 1e-5)


def test_batched_scatter_byte_exact(cuda):
    from velox_amd import ops

    p, h, s, d, n = 8, 8, 16, 128, 4  # metal_batched_kernels_parity.rs:144-189
    pool = vxo.round_to(rand_vec(p * h * s * d, 11), vxo.BF16).reshape(p, h, s, d)
    val = vxo.round_to(rand_vec(n * h * d, 13), vxo.BF16).reshape(n, h, d)
    pid = np.array([0, 3, 5, 7], np.uint32)
    sl = np.array([0, 7, 15, 5], np.uint32)
    pt = dev(pool, torch.bfloat16)
    ops.batched_scatter(pt, dev(val, torch.bfloat16), u32(pid), u32(sl))
    assert np.array_equal(host(pt), vxo.kv_scatter(pool, val, pid, sl))


# ---------------------------------------------------------------- acceptance
def _planted_logits(rng, b, r, v, dtype):
    lg = rng.normal(0, 3, size=(b, r, v)).astype(np.float32)
    # plant exact ties at the max (first index must win) in some rows
    for i in range(0, b * r, 3):
        row = lg.reshape(-1, v)[i]
        j1, j2 = sorted(rng.choice(v, 2, replace=False))
        row[j1] = row[j2] = row.max() + 1.0
    lg.reshape(-1, v)[5, :] = -np.inf  # all -inf row -> index 0
    return vxo.round_to(lg, OD[dtype])


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_accept_greedy_exact(cuda, dtype):
    from velox_amd import ops

    rng = np.random.default_rng(11)
    B, k, V = 16, 4, 151936
    lg = _planted_logits(rng, B, k + 1, V, dtype)
    am = lg.reshape(-1, V).argmax(axis=1).reshape(B, k + 1)
    cand = am[:, :k].astype(np.uint32).copy()
    for b in range(B):  # reject at a random position for half of the sequences
        if b % 2:
            cand[b, rng.integers(0, k)] += 1
    acc, tok = ops.accept_greedy(dev(lg, TD[dtype]), u32(cand))
    ref_acc, ref_tok = vxo.accept_greedy(lg, cand)
    assert np.array_equal(acc.cpu().numpy(), ref_acc)
    for b in range(B):
        a = ref_acc[b]
        assert np.array_equal(tok.cpu().numpy().view(np.uint32)[b, : a + 1], ref_tok[b, : a + 1])
    am_gpu = ops.argmax_rows(dev(lg.reshape(-1, V), TD[dtype])).cpu().numpy().view(np.uint32)
    assert np.array_equal(am_gpu, np.array([vxo.argmax(r) for r in lg.reshape(-1, V)], np.uint32))


@pytest.mark.parametrize("k", [4, 8])
def test_accept_stochastic_config2_bit_exact(cuda, k):
    """Config 2: B=16, V=151936, target ~N(0,3), draft = target + N(0,1), T=0.8,
    Philox(seed 2) uniforms.  Candidates drawn from q, then accept/resample:
    every token and accepted length must equal the host definition."""
    from velox_amd import ops

    B, V, T = 16, 151936, 0.8
    rng = np.random.Generator(np.random.Philox(key=[2, k]))
    tl = rng.normal(0, 3, size=(B, k + 1, V)).astype(np.float32)
    dl = (tl[:, :k] + rng.normal(0, 1, size=(B, k, V))).astype(np.float32)
    uni = vxo.spec_uniforms(2, 0, 0, B, k)
    inv_t = np.float32(1.0) / np.float32(T)
    cand = vxo.sample_draft(dl, uni, inv_t)
    u_draft = np.ascontiguousarray(uni[:, :k, 0]).reshape(-1)
    cand_gpu = ops.sample_rows(dev(dl.reshape(B * k, V)), dev(u_draft), T).cpu().numpy().view(np.uint32)
    assert np.array_equal(cand_gpu, cand.reshape(-1)), "draft draws must be bit-identical"
    acc, tok = ops.accept_stochastic(dev(tl), dev(dl), u32(cand), dev(uni), T)
    ref_acc, ref_tok = vxo.accept_stochastic(tl, dl, cand, uni, inv_t)
    assert np.array_equal(acc.cpu().numpy(), ref_acc)
    tk = tok.cpu().numpy().view(np.uint32)
    for b in range(B):
        a = ref_acc[b]
        assert np.array_equal(tk[b, : a + 1], ref_tok[b, : a + 1]), f"seq {b}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("V", [300, 8192, 8193, 20000])
def test_stochastic_draws_edge_cases(cuda, V, dtype):
    """Vocabularies off the 256 / 8192 grid, uniforms at 0 and just below 1,
    and peaked rows whose probabilities underflow to 0 outside a few tokens
    (the walk's fallbacks to the last positive index): draft draws, accepted
    lengths and tokens bit-identical to the host definition."""
    from velox_amd import ops

    B, k, T = 6, 3, 0.8
    rng = np.random.Generator(np.random.Philox(key=[9, V]))
    tl = rng.normal(0, 3, size=(B, k + 1, V)).astype(np.float32)
    tl[0] = -60.0
    tl[0, :, rng.integers(0, V, 3)] = 60.0  # three live tokens per row, the rest exp(-150) -> 0
    tl[1, :, V - 1] = 40.0                  # mass at the very last index
    dl = (tl[:, :k] + rng.normal(0, 1, size=(B, k, V))).astype(np.float32)
    dl[0] = tl[0, :k]
    if dtype == "bf16":
        tl, dl = vxo.round_to(tl, vxo.BF16), vxo.round_to(dl, vxo.BF16)
    uni = vxo.spec_uniforms(9, 0, 0, B, k).copy()
    top = np.float32(np.nextafter(np.float32(1), np.float32(0)))
    uni[2, :, :] = 0.0
    uni[3, :, :] = top
    uni[4, :, 1] = top  # reject every candidate: residual draws
    inv_t = np.float32(1.0) / np.float32(T)
    cand = vxo.sample_draft(dl, uni, inv_t)
    u_draft = np.ascontiguousarray(uni[:, :k, 0]).reshape(-1)
    cand_gpu = ops.sample_rows(dev(dl.reshape(B * k, V), TD[dtype]), dev(u_draft), T).cpu().numpy().view(np.uint32)
    assert np.array_equal(cand_gpu, cand.reshape(-1)), "draft draws must be bit-identical"
    acc, tok = ops.accept_stochastic(dev(tl, TD[dtype]), dev(dl, TD[dtype]), u32(cand), dev(uni), T)
    ref_acc, ref_tok = vxo.accept_stochastic(tl, dl, cand, uni, inv_t)
    assert np.array_equal(acc.cpu().numpy(), ref_acc)
    tk = tok.cpu().numpy().view(np.uint32)
    for b in range(B):
        a = ref_acc[b]
        assert np.array_equal(tk[b, : a + 1], ref_tok[b, : a + 1]), f"seq {b}"


def test_accept_tree_exact(cuda):
    from velox_amd import ops

    par = tree_4_2_2()
    R, B, V = len(par), 8, 151936
    rng = np.random.default_rng(5)
    lg = vxo.round_to(rng.normal(0, 3, size=(B, R, V)).astype(np.float32), vxo.BF16)
    am = lg.reshape(-1, V).argmax(axis=1).reshape(B, R)
    nt = rng.integers(0, V, size=(B, R)).astype(np.uint32)
    for b in range(B):  # plant accepted paths of various depths
        cur = 0
        for _ in range(b % 4):
            kids = [j for j in range(R) if par[j] == cur]
            if not kids:
                break
            j = kids[rng.integers(0, len(kids))]
            nt[b, j] = am[b, cur]
            cur = j
    acc, path, tok = ops.accept_tree(dev(lg, torch.bfloat16), par, u32(nt))
    ra, rp, rt = vxo.accept_tree(lg, np.array(par, np.int32), nt)
    assert np.array_equal(acc.cpu().numpy(), ra)
    for b in range(B):
        a = ra[b]
        assert np.array_equal(path.cpu().numpy()[b, : a + 1], rp[b, : a + 1])
        assert np.array_equal(tok.cpu().numpy().view(np.uint32)[b, : a + 1], rt[b, : a + 1])


def _pool_copy(dst_ptr, src_ptr, nbytes):
    import ctypes as C

    rt = C.CDLL("libamdhip64.so.7")
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    assert rt.hipMemcpy(dst_ptr, src_ptr, nbytes, 3) == 0  # device to device


def test_kv_compact_path(cuda):
    """Tree-path compaction: positions kv_offset + d take the rows of node
    path[d] (read before any move) in every layer, K/V and head; other rows
    are untouched.  Shuffled pages, a path crossing a page boundary, a
    sequence with nothing accepted."""
    from velox_amd import engine, ops

    L, HK, D, ps, P = 2, 2, 64, 16, 12
    pg = engine.PagedKvCache(L, HK, D, ps, P)
    rng = np.random.default_rng(4)
    pool_elems = P * HK * ps * D
    pools = [rng.standard_normal(pool_elems).astype(np.float16) for _ in range(2 * L)]
    for i, arr in enumerate(pools):
        t = torch.from_numpy(arr).cuda()
        _pool_copy(pg.layer_pool_ptr(i // 2, i % 2), t.data_ptr(), t.numel() * 2)
    torch.cuda.synchronize()
    bt = np.array([[7, 2], [0, 11], [5, 9]], np.uint32)
    kvo = np.array([3, 10, 12], np.uint32)
    r = 7
    paths = np.zeros((3, r), np.int32)
    paths[0, :4] = [0, 1, 3, 6]
    paths[2, :3] = [0, 2, 5]
    acc = np.array([3, 0, 2], np.int32)
    ops.kv_compact_path(pg, u32(bt), u32(kvo), torch.from_numpy(acc).cuda(), torch.from_numpy(paths).cuda())
    torch.cuda.synchronize()
    for i, arr in enumerate(pools):
        want = arr.reshape(P, HK, ps, D).copy()
        src = arr.reshape(P, HK, ps, D)
        for b in range(3):
            for d in range(1, acc[b] + 1):
                sp, dp = int(kvo[b]) + int(paths[b, d]), int(kvo[b]) + d
                want[bt[b, dp // ps], :, dp % ps] = src[bt[b, sp // ps], :, sp % ps]
        got = torch.empty(pool_elems, dtype=torch.float16, device="cuda")
        _pool_copy(got.data_ptr(), pg.layer_pool_ptr(i // 2, i % 2), pool_elems * 2)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().reshape(P, HK, ps, D), want), f"pool {i} differs"


def test_empty_batches_through_the_drop_ins(cuda):
    """Zero rows through the reference-shaped operators return empty results
    (torch hands zero-element tensors over with null data pointers)."""
    from velox_amd import ops

    lin = synth_linear(256, 256, 3)
    y = ops.qmm_4bit(torch.empty((0, 256), dtype=torch.float16, device="cuda"), u32(lin["qweight"]),
                     dev(lin["scales"]), dev(lin["biases"]), None, 64)
    assert tuple(y.shape) == (0, 256)
    kp = torch.zeros((4, 2, 16, 64), dtype=torch.float16, device="cuda")
    u = lambda *s: torch.zeros(s, dtype=torch.int32, device="cuda")  # noqa: E731
    out = ops.paged_prefill_attention(torch.empty((0, 4, 64), dtype=torch.float16, device="cuda"), kp, kp.clone(),
                                      u(0, 2), u(1), u(0), u(0), 0.125)
    assert tuple(out.shape) == (0, 4, 64)
    out = ops.paged_decode_attention(torch.empty((0, 4, 64), dtype=torch.float16, device="cuda"), kp, kp.clone(),
                                     u(0, 2), u(0), 0.125)
    assert tuple(out.shape) == (0, 4, 64)
    tab = torch.zeros((16, 32), dtype=torch.bfloat16, device="cuda")
    ops.batched_rope_decode(torch.empty((0, 4, 64), dtype=torch.bfloat16, device="cuda"), tab, tab.clone(), u(0))
    before = kp.clone()
    ops.batched_scatter(kp, torch.empty((0, 2, 64), dtype=torch.float16, device="cuda"), u(0), u(0))
    assert torch.equal(kp, before)
    assert tuple(ops.argmax_rows(torch.empty((0, 10), dtype=torch.bfloat16, device="cuda")).shape) == (0,)
    acc, tok = ops.accept_greedy(torch.empty((0, 5, 10), dtype=torch.bfloat16, device="cuda"), u(0, 4))
    assert tuple(acc.shape) == (0,) and tuple(tok.shape) == (0, 5)
    torch.cuda.synchronize()
