"""vx_qmm_4bit_noalloc: the allocation-free variant of vx_qmm_4bit gives the
same results, bit for bit, on two calls in a row (the second smaller, so it
reads a scratch array still holding the first call's partials), in f16 and
bf16, with and without a bias, and rejects a shape whose split-K partials do
not fit its static scratch."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(m, n, k, dt, seed, with_bias):
    from velox_amd import synth

    rng = np.random.default_rng(seed)
    lin = synth.qlinear(seed, f"noalloc.{n}x{k}", n, k, 64)
    td = torch.float16 if dt == "f16" else torch.bfloat16
    x = torch.from_numpy(rng.normal(0, 1, size=(m, k)).astype(np.float32)).to(td).cuda()
    qw = torch.from_numpy(lin["qweight"].view(np.int32)).cuda()
    sc = torch.from_numpy(lin["scales"]).to(td).cuda()
    bs = torch.from_numpy(lin["biases"]).to(td).cuda()
    bias = torch.from_numpy(rng.normal(0, 1, size=n).astype(np.float32)).to(td).cuda() if with_bias else None
    return x, qw, sc, bs, bias


def _call(fn, x, qw, sc, bs, bias, m, n, k):
    from velox_amd import _lib

    y = torch.full((m, n), float("nan"), dtype=x.dtype, device="cuda")
    dt = _lib.F16 if x.dtype == torch.float16 else _lib.BF16
    rc = fn(x.data_ptr(), qw.data_ptr(), sc.data_ptr(), bs.data_ptr(), None if bias is None else bias.data_ptr(),
            y.data_ptr(), m, n, k, 64, dt, torch.cuda.current_stream().cuda_stream)
    return rc, y


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_noalloc_matches_qmm_4bit_on_consecutive_calls(cuda, dt):
    from velox_amd import _lib

    L = _lib.lib
    # verify-row shapes whose plans split K (partials in the scratch), then
    # a smaller one on the same scratch
    for i, (m, n, k, with_bias) in enumerate([(80, 2560, 9728, False), (5, 2560, 4096, True)]):
        x, qw, sc, bs, bias = _inputs(m, n, k, dt, 40 + i, with_bias)
        rc_ref, ref = _call(L.vx_qmm_4bit, x, qw, sc, bs, bias, m, n, k)
        rc, got = _call(L.vx_qmm_4bit_noalloc, x, qw, sc, bs, bias, m, n, k)
        torch.cuda.synchronize()
        assert rc_ref == 0 and rc == 0, L.vx_last_error().decode()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i} ({m}x{n}x{k}) differs"
        print(f"[noalloc] {dt} call {i}: {m}x{n}x{k} identical", flush=True)


def test_noalloc_rejects_shapes_beyond_its_scratch(cuda):
    from velox_amd import _lib

    L = _lib.lib
    # 80 verify rows of a wide projection: the plan splits K four ways over
    # 128 column blocks, 4 x 80 x 16384 x 4 B = 21 MB of partials
    m, n, k = 80, 16384, 16384
    x = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    qw = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    sc = torch.zeros((n, k // 64), dtype=torch.float16, device="cuda")
    y = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    rc = L.vx_qmm_4bit_noalloc(x.data_ptr(), qw.data_ptr(), sc.data_ptr(), sc.data_ptr(), None, y.data_ptr(), m, n,
                               k, 64, _lib.F16, torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and "static scratch" in L.vx_last_error().decode()
