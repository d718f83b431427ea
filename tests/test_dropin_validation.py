"""The drop-ins reject what the reference's host wrappers reject, before any
device work: Q/K/V dtype agreement, U32 index tensors and contiguity
(metal_kernels.rs:1274-1291 decode, :1726-1745 prefill, :1436-1447 RoPE,
:1565-1575 scatter), and malformed token trees at the C ABI (a cycle or a
parent that does not precede its node would send the ancestor walk of
vx_forward out of bounds).  CPU tensors suffice: every case raises first."""
import ctypes as C

import pytest
import torch

from velox_amd import _lib, ops
from velox_amd._lib import VeloxError


def attn_inputs(total_q=5, n=1, hq=4, hk=2, d=64, p=3, ps=16, dt=torch.float16):
    q = torch.zeros(total_q, hq, d, dtype=dt)
    k = torch.zeros(p, hk, ps, d, dtype=dt)
    v = torch.zeros(p, hk, ps, d, dtype=dt)
    bt = torch.zeros(n, 2, dtype=torch.int32)
    cu = torch.tensor([0, total_q], dtype=torch.int32)
    sid = torch.zeros(total_q, dtype=torch.int32)
    kvo = torch.zeros(n, dtype=torch.int32)
    return q, k, v, bt, cu, sid, kvo


def test_prefill_rejects_wide_index_tensors_and_mixed_dtypes():
    q, k, v, bt, cu, sid, kvo = attn_inputs()
    with pytest.raises(VeloxError, match="index tensors must be U32"):
        ops.paged_prefill_attention(q, k, v, bt.long(), cu, sid, kvo, 0.1)
    with pytest.raises(VeloxError, match="index tensors must be U32"):
        ops.paged_prefill_attention(q, k, v, bt, cu.float(), sid, kvo, 0.1)
    with pytest.raises(VeloxError, match="Q/K/V dtype mismatch"):
        ops.paged_prefill_attention(q.float(), k, v, bt, cu, sid, kvo, 0.1)
    with pytest.raises(VeloxError, match="must be contiguous"):
        ops.paged_prefill_attention(q, k, v, bt, cu, torch.zeros(10, dtype=torch.int32)[::2], kvo, 0.1)
    with pytest.raises(VeloxError, match="tree_mask"):
        ops.paged_prefill_attention(q, k, v, bt, cu, sid, kvo, 0.1, tree_mask=torch.zeros(5, dtype=torch.int32))


def test_decode_rejects_what_the_reference_rejects():
    q, k, v, bt, _, _, _ = attn_inputs(total_q=1)
    lens = torch.ones(1, dtype=torch.int32)
    with pytest.raises(VeloxError, match="Q/K/V dtype mismatch"):
        ops.paged_decode_attention(q.float(), k, v, bt, lens, 0.1)
    with pytest.raises(VeloxError, match="block_table and kv_lens must be U32"):
        ops.paged_decode_attention(q, k, v, bt.long(), lens, 0.1)
    with pytest.raises(VeloxError, match="block_table and kv_lens must be U32"):
        ops.paged_decode_attention(q, k, v, bt, lens.long(), 0.1)
    with pytest.raises(VeloxError, match="k_pool must be contiguous"):
        ops.paged_decode_attention(q, k.transpose(0, 1).contiguous().transpose(0, 1), v, bt, lens, 0.1)


def test_rope_and_scatter_index_dtypes():
    x = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    cs = torch.zeros(16, 32, dtype=torch.bfloat16)
    with pytest.raises(VeloxError, match="offsets must be U32"):
        ops.batched_rope_decode(x, cs, cs, torch.zeros(2, dtype=torch.float32))
    with pytest.raises(VeloxError, match="offsets must be U32"):
        ops.batched_rope_decode(x, cs, cs, torch.zeros(2, dtype=torch.int64))
    pool = torch.zeros(3, 4, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(VeloxError, match="page_ids and slots must be U32"):
        ops.batched_scatter(pool, x, torch.zeros(2, dtype=torch.int64), torch.zeros(2, dtype=torch.int32))


def test_acceptance_drop_ins_check_shapes_and_dtypes():
    lg = torch.zeros(2, 5, 10, dtype=torch.bfloat16)
    with pytest.raises(VeloxError, match="candidates must be U32"):
        ops.accept_greedy(lg, torch.zeros(2, 4, dtype=torch.int64))
    with pytest.raises(VeloxError, match=r"candidates must be \[B, k\]"):
        ops.accept_greedy(lg, torch.zeros(2, 3, dtype=torch.int32))
    with pytest.raises(VeloxError, match="uniforms must be f32"):
        ops.accept_stochastic(lg, lg[:, :4].contiguous(), torch.zeros(2, 4, dtype=torch.int32),
                              torch.zeros(2, 5, 4, dtype=torch.float64), 0.8)
    with pytest.raises(VeloxError, match="parents for"):
        ops.accept_tree(lg, [-1, 0, 0], torch.zeros(2, 5, dtype=torch.int32))


def _seq(nt):
    return _lib.SeqSlice(nt, 0, None, 0)


@pytest.mark.parametrize("parents,msg", [
    ([0, 0, 1], "root"),            # no root
    ([-1, 2, 1], "precede"),        # 1 -> 2 -> 1: a cycle
    ([-1, 0, 5], "precede"),        # parent past the tree
    ([-1, 0, 2], "precede"),        # a self-loop
])
def test_forward_validates_the_tree_before_using_it(parents, msg):
    arr = (C.c_int32 * len(parents))(*parents)
    seqs = (_lib.SeqSlice * 1)(_seq(len(parents)))
    ids = (C.c_uint32 * len(parents))()
    rc = _lib.lib.vx_forward(None, None, ids, seqs, 1, 1, arr, None, None)
    assert rc != 0 and msg in _lib.lib.vx_last_error().decode()


def test_forward_rejects_trees_beyond_64_nodes():
    par = [-1] + list(range(64))
    arr = (C.c_int32 * 65)(*par)
    seqs = (_lib.SeqSlice * 1)(_seq(65))
    rc = _lib.lib.vx_forward(None, None, (C.c_uint32 * 65)(), seqs, 1, 1, arr, None, None)
    assert rc != 0 and "1..64 nodes" in _lib.lib.vx_last_error().decode()


def test_python_forward_checks_the_tree_length():
    from velox_amd import engine

    m = engine.PagedQwen3.__new__(engine.PagedQwen3)
    m.cfg = {"vocab": 8}
    with pytest.raises(VeloxError, match="needs new_tokens"):
        m._run(None, [1, 2, 3], [(3, 0, [0])], True, [-1, 0], None)
