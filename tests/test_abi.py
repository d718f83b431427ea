"""The C ABI library loads without a GPU, exports every entry point declared in
include/velox_hip.h, and rejects invalid arguments with the reference's
messages before touching a device (no compute calls here)."""
import ctypes as C
import os

import pytest

from velox_amd import _lib


def test_every_declared_symbol_is_exported():
    syms = _lib.header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(_lib.lib, s)]
    assert not missing, missing
    assert _lib.lib.vx_version().decode().startswith("velox_amd")


def test_one_hip_runtime_whatever_the_import_order():
    """Importing velox_amd before torch must not load a second HIP runtime."""
    import subprocess
    import sys

    code = ("import velox_amd, torch; m = open('/proc/self/maps').read(); "
            "print(len({l.split()[-1] for l in m.splitlines() if 'amdhip64' in l}))")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True,
                         cwd=os.path.dirname(_lib.HERE))
    assert out.stdout.strip() == "1", out.stdout + out.stderr


def _err(rc):
    assert rc != 0
    return _lib.lib.vx_last_error().decode()


def test_qmm_validation_matches_reference():
    L = _lib.lib
    # metal_kernels.rs:2084-2097
    assert "multiple of 8" in _err(L.vx_qmm_4bit(1, 1, 1, 1, None, 1, 2, 4, 12, 64, _lib.F16, None))
    assert "group_size" in _err(L.vx_qmm_4bit(1, 1, 1, 1, None, 1, 2, 4, 128, 48, _lib.F16, None))
    assert "group_size" in _err(L.vx_qmm_4bit(1, 1, 1, 1, None, 1, 2, 4, 128, 0, _lib.F16, None))
    assert "dtype" in _err(L.vx_qmm_4bit(1, 1, 1, 1, None, 1, 2, 4, 128, 64, 7, None))


def test_attention_validation_matches_reference():
    L = _lib.lib
    # metal_kernels.rs:1702-1711
    args = [1] * 9
    assert "divisible" in _err(L.vx_paged_attention(*args, 4, 1, 1, 4, 6, 4, 128, 16, 0.1, 0, _lib.F16, None))
    assert "D_MAX" in _err(L.vx_paged_attention(*args, 4, 1, 1, 4, 8, 4, 512, 16, 0.1, 0, _lib.F16, None))
    assert "multiple of 32" in _err(L.vx_paged_attention(*args, 4, 1, 1, 4, 8, 4, 80, 16, 0.1, 0, _lib.F16, None))


def test_acceptance_validation():
    L = _lib.lib
    assert "draft_k" in _err(L.vx_accept_greedy(1, 1, 1, 1, 2, 0, 10, _lib.BF16, None))
    bad = (C.c_int32 * 3)(0, 0, 1)
    assert "root" in _err(L.vx_accept_tree(1, C.cast(bad, C.c_void_p), 1, 1, 1, 1, 1, 3, 10, _lib.BF16, None))
    fwd = (C.c_int32 * 3)(-1, 2, 1)
    assert "precede" in _err(L.vx_accept_tree(1, C.cast(fwd, C.c_void_p), 1, 1, 1, 1, 1, 3, 10, _lib.BF16, None))
    assert "temperature" in _err(L.vx_accept_stochastic(1, 1, 1, 1, 1, 1, 2, 4, 10, 0.0, _lib.F32, None, 0, None))


def test_pages_validation():
    out = C.c_void_p()
    # pages.rs:94-96
    assert "page" in _err(_lib.lib.vx_pages_create(2, 4, 8, 4, 0, _lib.F16, C.byref(out)))
    assert "dtype" in _err(_lib.lib.vx_pages_create(2, 4, 8, 4, 4, _lib.F32, C.byref(out)))


def test_no_fallback_when_library_missing(tmp_path, monkeypatch):
    import importlib.util
    import shutil

    pkg = tmp_path / "velox_amd"
    shutil.copytree(_lib.HERE, pkg, ignore=shutil.ignore_patterns("*.so", "_build", "__pycache__", "csrc"))
    spec = importlib.util.spec_from_file_location("velox_amd_nolib._lib", pkg / "_lib.py")
    mod = importlib.util.module_from_spec(spec)
    with pytest.raises(ImportError, match="no CPU fallback"):
        spec.loader.exec_module(mod)


def test_empty_inputs_are_no_ops():
    """Zero rows are valid input to every kernel entry point (the reference
    returns empty tensors): the call succeeds without touching the pointers,
    which PyTorch leaves null for zero-element tensors.  Shape validation
    still runs first."""
    L, F16, BF16 = _lib.lib, _lib.F16, _lib.BF16
    Z = None
    assert L.vx_qmm_4bit(Z, Z, Z, Z, Z, Z, 0, 4096, 256, 64, F16, Z) == 0
    assert L.vx_qmm_4bit(Z, Z, Z, Z, Z, Z, 5, 0, 256, 64, F16, Z) == 0
    assert "multiple of 8" in _err(L.vx_qmm_4bit(Z, Z, Z, Z, Z, Z, 0, 4096, 12, 64, F16, Z))
    assert L.vx_qmm_4bit_ex(Z, Z, Z, Z, Z, Z, 0, 128, 256, 64, 0, BF16, F16, _lib.EPI_STORE, Z, 0, Z) == 0
    assert L.vx_qmm_4bit_packed(Z, Z, Z, Z, 0, 128, 256, 0, BF16, F16, _lib.EPI_STORE, Z, 0, Z) == 0
    assert L.vx_paged_attention(Z, Z, Z, Z, Z, Z, Z, Z, Z, 0, 0, 1, 1, 4, 2, 64, 16, 0.125, 0, F16, Z) == 0
    assert "divisible" in _err(L.vx_paged_attention(Z, Z, Z, Z, Z, Z, Z, Z, Z, 0, 0, 1, 1, 4, 3, 64, 16, 0.125,
                                                    0, F16, Z))
    assert L.vx_paged_decode_attention(Z, Z, Z, Z, Z, Z, 0, 1, 1, 4, 2, 64, 16, 0.125, 0, F16, Z) == 0
    assert L.vx_rope_inplace(Z, Z, Z, Z, 0, 4, 64, 16, BF16, Z) == 0
    assert L.vx_kv_scatter(Z, Z, Z, Z, 0, 1, 2, 16, 64, F16, Z) == 0
    assert L.vx_argmax_rows(Z, Z, 0, 10, BF16, Z) == 0
    assert L.vx_accept_greedy(Z, Z, Z, Z, 0, 4, 10, BF16, Z) == 0
    assert L.vx_accept_stochastic(Z, Z, Z, Z, Z, Z, 0, 4, 10, 0.8, BF16, Z, 0, Z) == 0
    assert L.vx_sample_rows(Z, Z, 1, Z, 0, 10, 0.8, BF16, Z, 0, Z) == 0
