"""ctypes binding of libvelox_hip.so (the C ABI declared in include/velox_hip.h).

The library must have been built (velox_amd/build.py, or __graft_entry__.build());
importing this module fails loudly otherwise — there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvelox_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "velox_hip.h")

F32, F16, BF16 = 0, 1, 2
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with `python velox_amd/build.py` "
                      "(velox_amd has no CPU fallback)")



def _share_torch_hip_runtime() -> None:
    """Bind the library to the HIP runtime PyTorch ships, when PyTorch is
    installed.  libtorch_hip needs `libamdhip64.so` from its own lib folder,
    this library `libamdhip64.so.7`; loaded in the other order the process
    would hold two HIP (and HSA) runtimes, and the second one to initialise
    finds no device.  Preloading torch's copy (soname libamdhip64.so.7) makes
    both names resolve to it."""
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    rt = os.path.join(list(spec.submodule_search_locations)[0], "lib", "libamdhip64.so")
    if os.path.exists(rt):
        C.CDLL(rt, mode=C.RTLD_GLOBAL)


_share_torch_hip_runtime()
lib = C.CDLL(LIB_PATH)

vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int
f32 = C.c_float
u32p = C.POINTER(C.c_uint32)


class QwenConfig(C.Structure):
    _fields_ = [("vocab", i64), ("hidden", i64), ("inter", i64), ("layers", i64), ("n_heads", i64),
                ("n_kv_heads", i64), ("head_dim", i64), ("max_pos", i64), ("group_size", i64),
                ("rope_theta", C.c_double), ("rms_eps", C.c_double)]


class QLinearHost(C.Structure):
    _fields_ = [("qweight", vp), ("scales", vp), ("biases", vp)]


class LayerHost(C.Structure):
    _fields_ = [("ln1", vp), ("ln2", vp), ("q_norm", vp), ("k_norm", vp), ("q", QLinearHost),
                ("k", QLinearHost), ("v", QLinearHost), ("o", QLinearHost), ("gate", QLinearHost),
                ("up", QLinearHost), ("down", QLinearHost)]


class WeightsHost(C.Structure):
    _fields_ = [("embed", vp), ("layers", vp), ("norm", vp), ("lm_head", QLinearHost)]


class SeqSlice(C.Structure):
    _fields_ = [("new_tokens", i64), ("kv_offset", i64), ("block_table", vp), ("n_blocks", i64)]


class RoundOutcome(C.Structure):
    _fields_ = [("accepted", C.c_int32), ("n_committed", C.c_int32), ("stop", C.c_int32)]


class StepProfile(C.Structure):
    _fields_ = [("draft_ms", C.c_double), ("verify_ms", C.c_double), ("accept_ms", C.c_double),
                ("verify_kernel_ms", C.c_double * 3), ("verify_kernel_bytes", C.c_double * 3),
                ("verify_kernel_launches", C.c_int64 * 3), ("draft_kernel_ms", C.c_double * 3),
                ("draft_kernel_bytes", C.c_double * 3), ("draft_kernel_launches", C.c_int64 * 3)]


class RoundTrace(C.Structure):
    _fields_ = [("n", i64), ("draft_k", i64), ("vocab", i64), ("temperature", f32), ("has_draft_logits", C.c_int32),
                ("serial", C.c_uint64)]


class SchedConfig(C.Structure):
    _fields_ = [("max_running_requests", i64), ("max_batch_tokens", i64), ("prefix_cache_capacity", i64),
                ("draft_k", i64)]


class SchedStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "steps", "tokens_generated", "requests_completed", "requests_aborted", "last_batch_size", "last_step_us",
        "prefix_cache_hits", "prefix_cache_misses", "prefix_tokens_skipped", "rounds", "draft_tokens_proposed",
        "draft_tokens_accepted", "prefill_tokens")]


i64p = C.POINTER(i64)
ADD_STATE_FN = C.CFUNCTYPE(i32, vp, u32p, i64, i64, u32p, u32p, i64, C.c_uint32, f32, i64p)
PREFILL_CHUNK_FN = C.CFUNCTYPE(i32, vp, i64p, i64p, i64)
STEP_FN = C.CFUNCTYPE(i32, vp, i64p, i64, i64, C.POINTER(RoundOutcome), u32p)
STATE_PAGES_FN = C.CFUNCTYPE(i64, vp, i64, i32, u32p, i64)
FREE_STATE_FN = C.CFUNCTYPE(None, vp, i64)
REF_FN = C.CFUNCTYPE(None, vp, i32, u32p, i64)


class SchedBackend(C.Structure):
    _fields_ = [("ctx", vp), ("page_size", i64), ("add_state", ADD_STATE_FN), ("prefill_chunk", PREFILL_CHUNK_FN),
                ("step", STEP_FN), ("state_pages", STATE_PAGES_FN), ("free_state", FREE_STATE_FN),
                ("incref", REF_FN), ("decref", REF_FN)]


_SIGS = {
    "vx_last_error": (C.c_char_p, []),
    "vx_version": (C.c_char_p, []),
    "vx_qmm_4bit": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i32, vp]),
    "vx_qmm_4bit_noalloc": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i32, vp]),
    "vx_qmm_4bit_ex": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i32, i32, i32, i32, vp,
                             C.c_size_t, vp]),
    "vx_qmm_workspace_size": (C.c_size_t, [i64, i64, i64]),
    "vx_qmm_packed_size": (C.c_size_t, [i64, i64]),
    "vx_qmm_pack_4bit": (i32, [vp, vp, vp, vp, i64, i64, vp]),
    "vx_qmm_4bit_packed": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, i32, i32, i32, vp, C.c_size_t, vp]),
    "vx_paged_attention": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64,
                                 i64, i64, f32, C.c_uint32, i32, vp]),
    "vx_paged_decode_attention": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64,
                                        f32, C.c_uint32, i32, vp]),
    "vx_rope_inplace": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i32, vp]),
    "vx_kv_scatter": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, vp]),
    "vx_argmax_rows": (i32, [vp, vp, i64, i64, i32, vp]),
    "vx_accept_greedy": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, vp]),
    "vx_accept_stochastic": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, f32, i32, vp, C.c_size_t,
                                   vp]),
    "vx_sample_rows": (i32, [vp, vp, i64, vp, i64, i64, f32, i32, vp, C.c_size_t, vp]),
    "vx_accept_tree": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i32, vp]),
    "vx_pages_create": (i32, [i64, i64, i64, i64, i64, i32, C.POINTER(vp)]),
    "vx_pages_destroy": (None, [vp]),
    "vx_pages_alloc": (i32, [vp, i64, u32p]),
    "vx_pages_incref": (None, [vp, u32p, i64]),
    "vx_pages_free": (None, [vp, u32p, i64]),
    "vx_pages_num_free": (i64, [vp]),
    "vx_pages_refcount": (C.c_uint32, [vp, C.c_uint32]),
    "vx_pages_pool": (vp, [vp, i64, i32]),
    "vx_kv_compact_path": (i32, [vp, vp, i64, vp, vp, vp, i64, i64, vp]),
    "vx_model_create": (i32, [C.POINTER(QwenConfig), C.POINTER(WeightsHost), i64, C.POINTER(vp)]),
    "vx_model_destroy": (None, [vp]),
    "vx_forward": (i32, [vp, vp, u32p, C.POINTER(SeqSlice), i64, i32, C.POINTER(C.c_int32), vp, vp]),
    "vx_spec_create": (i32, [vp, vp, vp, vp, f32, C.c_uint64, i32, C.POINTER(vp)]),
    "vx_spec_destroy": (None, [vp]),
    "vx_spec_prefill": (i32, [vp, C.POINTER(u32p), C.POINTER(i64), i64, C.POINTER(i64)]),
    "vx_spec_step": (i32, [vp, C.POINTER(i64), i64, i64, i64, C.POINTER(RoundOutcome), u32p, vp]),
    "vx_spec_state_kv_len": (i64, [vp, i64]),
    "vx_spec_state_num_tokens": (i64, [vp, i64]),
    "vx_spec_state_tokens": (i32, [vp, i64, u32p, i64]),
    "vx_spec_last_trace": (i32, [vp, u32p, C.POINTER(f32)]),
    "vx_spec_set_tracing": (i32, [vp, i32]),
    "vx_spec_last_trace_info": (i32, [vp, C.POINTER(RoundTrace), C.POINTER(i64), u32p, u32p]),
    "vx_spec_last_trace_draft": (i32, [vp, C.POINTER(f32), C.POINTER(f32)]),
    "vx_spec_free": (None, [vp, i64]),
    "vx_spec_set_profiling": (i32, [vp, i32]),
    "vx_spec_last_profile": (i32, [vp, C.POINTER(StepProfile)]),
    "vx_spec_add_state": (i32, [vp, u32p, i64, i64, u32p, u32p, i64, C.c_uint32, f32, C.POINTER(i64)]),
    "vx_spec_prefill_chunk": (i32, [vp, C.POINTER(i64), C.POINTER(i64), i64, vp]),
    "vx_spec_state_pages": (i64, [vp, i64, i32, u32p, i64]),
    "vx_sched_create": (i32, [vp, C.POINTER(SchedConfig), u32p, i64, vp, C.POINTER(vp)]),
    "vx_sched_create_with_backend": (i32, [C.POINTER(SchedBackend), C.POINTER(SchedConfig), u32p, i64,
                                           C.POINTER(vp)]),
    "vx_sched_destroy": (None, [vp]),
    "vx_sched_submit": (i32, [vp, u32p, i64, i64, f32, i64, C.POINTER(i64)]),
    "vx_sched_step": (i32, [vp, C.POINTER(i64)]),
    "vx_sched_poll": (i32, [vp, i64, u32p, i64, C.POINTER(i64), C.POINTER(i32), C.POINTER(i32)]),
    "vx_sched_abort": (i32, [vp, i64]),
    "vx_sched_release": (i32, [vp, i64]),
    "vx_sched_get_stats": (i32, [vp, C.POINTER(SchedStats)]),
    "vx_sched_num_waiting": (i64, [vp]),
    "vx_sched_num_running": (i64, [vp]),
    "vx_sched_cache_pages": (i64, [vp]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


class VeloxError(RuntimeError):
    pass


def check(rc: int) -> None:
    if rc != 0:
        raise VeloxError(lib.vx_last_error().decode())


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(vx_[a-z0-9_]+)\s*\(", text)) - {"vx_dtype"})
