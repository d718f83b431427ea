"""Input generators and comparison helpers of the reference's Rust tests,
restated so the parity tests read like them.

rand_vec: the LCG of tests/metal_qmm_4bit_parity.rs:14-24 (same in
tests/metal_decode_parity.rs:17-26 and tests/metal_batched_kernels_parity.rs:16-24).
quantize_mlx_4bit: tests/metal_qmm_4bit_parity.rs:28-60.
assert_close: max-|diff| index vs atol + rtol*|ref| (metal_qmm_4bit_parity.rs:83-101).
"""
import numpy as np

_A = 6364136223846793005
_C = 1442695040888963407
_M = (1 << 64) - 1


_BLOCK = 4096


def _lcg_states(n: int, seed: int) -> np.ndarray:
    """States s_1..s_n of s_i = s_{i-1} * A + C (mod 2^64), s_0 = seed * A + C.
    The first block is stepped one by one; later blocks jump B steps at once
    (s_{i+B} = A^B s_i + C_B, with numpy's wrapping uint64 arithmetic)."""
    out = np.empty(n, np.uint64)
    if n == 0:
        return out
    b = min(n, _BLOCK)
    s = (seed * _A + _C) & _M
    for i in range(b):
        s = (s * _A + _C) & _M
        out[i] = s
    ab, cb = 1, 0
    for _ in range(b):
        ab, cb = (ab * _A) & _M, (cb * _A + _C) & _M
    ab, cb = np.uint64(ab), np.uint64(cb)
    for j in range(b, n, b):
        m = min(b, n - j)
        out[j:j + m] = out[j - b:j - b + m] * ab + cb
    return out


def rand_vec(n: int, seed: int) -> np.ndarray:
    out = ((_lcg_states(n, seed) >> np.uint64(33)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    # (x as u32 as f32) / (u32::MAX as f32) - 0.5, all in f32
    return (out.astype(np.float32) / np.float32(4294967295.0)) - np.float32(0.5)


def quantize_mlx_4bit(w: np.ndarray, n: int, k: int, gs: int):
    w = w.reshape(n, k).astype(np.float32)
    kg = k // gs
    grp = w.reshape(n, kg, gs)
    wmin = grp.min(axis=2)
    wmax = grp.max(axis=2)
    scale = np.maximum((wmax - wmin) / np.float32(15.0), np.float32(1e-12)).astype(np.float32)
    bias = wmin.astype(np.float32)
    q = (grp - bias[:, :, None]) / scale[:, :, None]
    q = np.sign(q) * np.floor(np.abs(q) + np.float32(0.5))  # f32::round: half away from zero
    q = np.clip(q, 0, 15).astype(np.uint32).reshape(n, k)
    packed = np.zeros((n, k // 8), np.uint32)
    for b in range(8):
        packed |= q[:, b::8] << np.uint32(4 * b)
    return packed, scale, bias


def dequant(qweight, scales, biases, gs=64):
    n, kp = qweight.shape
    k = kp * 8
    codes = np.zeros((n, k), np.float64)
    for b in range(8):
        codes[:, b::8] = (qweight >> np.uint32(4 * b)) & 0xF
    s = np.repeat(np.asarray(scales, np.float64), gs, axis=1)
    bb = np.repeat(np.asarray(biases, np.float64), gs, axis=1)
    return codes * s + bb


def assert_close(label, got, ref, atol, rtol):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    assert got.shape == ref.shape, f"{label}: length mismatch"
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    d = np.abs(got - ref)
    i = int(np.argmax(d))
    tol = atol + rtol * abs(ref[i])
    assert d[i] <= tol, f"{label}: max_err={d[i]} (idx={i}: got={got[i]} ref={ref[i]}) > tol={tol}"


def assert_allclose_elementwise(label, got, ref, atol, rtol):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{label}: {int(bad.sum())} elements out of tolerance; first at "
                           f"{int(np.argmax(bad))}: got={got[np.argmax(bad)]} ref={ref[np.argmax(bad)]}")
