"""Operator-level mirror of the reference's Metal kernels (src/paged/metal_kernels.rs),
running the gfx950 kernels through the C ABI.

Same names, argument meaning and failure conditions as the reference:
tensors are torch tensors on the GPU (torch provides device memory and the
current stream only), outputs are freshly allocated like the reference's
`Tensor::zeros` outputs, and shape/dtype/contiguity violations raise
VeloxError with the reference's messages.
"""
from __future__ import annotations

import torch

from ._lib import BF16, EPI_STORE, F16, F32, VeloxError, check, lib

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


def _dt(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DT:
        raise VeloxError(f"{what}: unsupported dtype {t.dtype}")
    return _DT[t.dtype]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise VeloxError(msg)


def _contig(name: str, **ts) -> None:
    for label, t in ts.items():
        if t is not None and not t.is_contiguous():
            raise VeloxError(f"{name}: {label} must be contiguous")


def _p(t):
    return None if t is None else t.data_ptr()


# The reference's index tensors are U32; torch carries the same 32-bit words
# as int32 (its uint32 has few kernels), so both are accepted.
_U32 = (torch.int32, torch.uint32)


def _u32(msg: str, *ts) -> None:
    for t in ts:
        if t is not None and t.dtype not in _U32:
            raise VeloxError(msg)


def qmm_4bit(x, qweight, scales, biases, bias=None, group_size=64):
    """qmm_4bit (metal_kernels.rs:2069-2076): Y[M,N] = X . deq(W)^T (+ bias)."""
    _need(x.dim() == 2 and qweight.dim() == 2, "qmm_4bit: x and qweight must be 2-D")
    m, k = x.shape
    n, kp = qweight.shape
    _need(k % 8 == 0, f"qmm_4bit: K={k} must be a multiple of 8")
    _need(kp == k // 8, f"qmm_4bit: qweight dim1 {kp} != K/8 {k // 8} (K={k})")
    _need(group_size != 0 and group_size % 8 == 0 and k % group_size == 0,
          f"qmm_4bit: group_size={group_size} must be a multiple of 8 and divide K={k}")
    kg = k // group_size
    _need(tuple(scales.shape) == (n, kg) and tuple(biases.shape) == (n, kg),
          f"qmm_4bit: scales {list(scales.shape)} / biases {list(biases.shape)} mismatch expected [{n},{kg}]")
    _need(scales.dtype == x.dtype and biases.dtype == x.dtype, "qmm_4bit: scales/biases dtype must match X")
    _need(qweight.dtype in (torch.int32, torch.uint32), "qmm_4bit: qweight must be U32")
    if bias is not None:
        _need(bias.dim() == 1 and bias.shape[0] == n and bias.dtype == x.dtype,
              f"qmm_4bit: bias must be [N={n}] of same dtype as X")
    _contig("qmm_4bit", x=x, qweight=qweight, scales=scales, biases=biases, bias=bias)
    y = torch.zeros((m, n), dtype=x.dtype, device=x.device)
    check(lib.vx_qmm_4bit(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                          _p(bias), y.data_ptr(), m, n, k, group_size, _dt(x, "qmm_4bit"), _stream()))
    return y


def qmm_4bit_ex(x, qweight, scales, biases, out, residual=None, x_shift=0, round_dtype=BF16,
                epilogue=EPI_STORE, workspace=None):
    """Fused-epilogue int4 GEMM used by the verify forward (f16 X, f16 affine params)."""
    m, k = x.shape
    n = qweight.shape[0]
    ws = _p(workspace)
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib.vx_qmm_4bit_ex(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                             out.data_ptr(), _p(residual), m, n, k, 64, x_shift, round_dtype,
                             _DT[out.dtype], epilogue, ws, wsb, _stream()))
    return out


def qmm_pack_4bit(qweight, scales, biases):
    """Packed copy of MLX int4 g64 weights (f16 scales/biases) for qmm_4bit_packed."""
    n, kp = qweight.shape
    k = kp * 8
    _need(n % 32 == 0 and k % 128 == 0, f"qmm_pack_4bit: N={n} must be a multiple of 32 and K={k} of 128")
    _need(tuple(scales.shape) == (n, k // 64) and tuple(biases.shape) == (n, k // 64),
          "qmm_pack_4bit: scales/biases must be [N, K/64]")
    _contig("qmm_pack_4bit", qweight=qweight, scales=scales, biases=biases)
    out = torch.empty(int(lib.vx_qmm_packed_size(n, k)), dtype=torch.uint8, device=qweight.device)
    check(lib.vx_qmm_pack_4bit(qweight.data_ptr(), scales.data_ptr(), biases.data_ptr(), out.data_ptr(), n, k,
                               _stream()))
    return out


def qmm_4bit_packed(x, packed, n, out, residual=None, x_shift=0, round_dtype=BF16, epilogue=EPI_STORE,
                    workspace=None):
    """qmm_4bit_ex over packed weights (see qmm_pack_4bit)."""
    m, k = x.shape
    ws = _p(workspace)
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib.vx_qmm_4bit_packed(x.data_ptr(), packed.data_ptr(), out.data_ptr(), _p(residual), m, n, k, x_shift,
                                 round_dtype, _DT[out.dtype], epilogue, ws, wsb, _stream()))
    return out


def paged_prefill_attention(q, k_pool, v_pool, block_table, cu_seqlens, seq_id_per_q, kv_offsets, scale,
                            sliding_window=0, tree_mask=None):
    """paged_prefill_attention (metal_kernels.rs:1680-1690), plus an optional per-row
    tree mask (uint64 [total_q]) for tree verification."""
    total_q, h_q, d = q.shape
    p, h_kv, ps, kd = k_pool.shape
    _need(d == kd, "prefill: head_dim mismatch Q vs K pool")
    _need(h_q % h_kv == 0, "prefill: H_q must be divisible by H_kv")
    _need(d <= 256, f"prefill: head_dim {d} > D_MAX 256")
    _need(d % 32 == 0, f"prefill: head_dim {d} must be a multiple of 32")
    n_blk, max_blocks = block_table.shape
    _need(cu_seqlens.shape[0] == n_blk + 1 and seq_id_per_q.shape[0] == total_q and kv_offsets.shape[0] == n_blk,
          f"prefill: shape mismatch (block_table N={n_blk}, cu_seqlens={cu_seqlens.shape[0]}, "
          f"seq_id_per_q={seq_id_per_q.shape[0]}, kv_offsets={kv_offsets.shape[0]})")
    _need(k_pool.dtype == q.dtype and v_pool.dtype == q.dtype, "prefill: Q/K/V dtype mismatch")
    _contig("prefill", q=q, k_pool=k_pool, v_pool=v_pool, block_table=block_table, cu_seqlens=cu_seqlens,
            seq_id_per_q=seq_id_per_q, kv_offsets=kv_offsets, tree_mask=tree_mask)
    _u32("prefill: index tensors must be U32", block_table, cu_seqlens, seq_id_per_q, kv_offsets)
    if tree_mask is not None:
        _need(tree_mask.dtype in (torch.int64, torch.uint64) and tuple(tree_mask.shape) == (total_q,),
              "prefill: tree_mask must be a 64-bit [total_q] tensor")
    out = torch.zeros_like(q)
    check(lib.vx_paged_attention(q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), block_table.data_ptr(),
                                 cu_seqlens.data_ptr(), seq_id_per_q.data_ptr(), kv_offsets.data_ptr(),
                                 _p(tree_mask), out.data_ptr(), total_q, n_blk, max_blocks, p, h_q, h_kv, d,
                                 ps, scale, sliding_window, _dt(q, "prefill"), _stream()))
    return out


def paged_decode_attention(q, k_pool, v_pool, block_table, kv_lens, scale, sliding_window=0):
    """paged_decode_attention (metal_kernels.rs:1227-1235)."""
    n, h_q, d = q.shape
    p, h_kv, ps, kd = k_pool.shape
    _need(k_pool.shape == v_pool.shape and d == kd,
          "paged_decode_attention: K/V pool shapes must match Q head_dim")
    _need(h_q % h_kv == 0, f"paged_decode_attention: H_q={h_q} must be divisible by H_kv={h_kv}")
    _need(d <= 256, f"paged_decode_attention: head_dim {d} > D_MAX 256")
    _need(d % 32 == 0, f"paged_decode_attention: head_dim {d} not divisible by 32")
    n_bt, max_blocks = block_table.shape
    _need(n_bt == n, f"paged_decode_attention: block_table N={n_bt} mismatches Q N={n}")
    _need(kv_lens.shape[0] == n, f"paged_decode_attention: kv_lens N={kv_lens.shape[0]} mismatches Q N={n}")
    _need(k_pool.dtype == q.dtype and v_pool.dtype == q.dtype, "paged_decode_attention: Q/K/V dtype mismatch")
    _u32("paged_decode_attention: block_table and kv_lens must be U32", block_table, kv_lens)
    _contig("paged_decode_attention", q=q, k_pool=k_pool, v_pool=v_pool, block_table=block_table, kv_lens=kv_lens)
    out = torch.zeros_like(q)
    check(lib.vx_paged_decode_attention(q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                                        block_table.data_ptr(), kv_lens.data_ptr(), out.data_ptr(), n,
                                        max_blocks, p, h_q, h_kv, d, ps, scale, sliding_window,
                                        _dt(q, "paged_decode_attention"), _stream()))
    return out


def batched_rope_decode(x, cos, sin, offsets):
    """batched_rope_decode (metal_kernels.rs:1414-1419): in place on x [N, H, D]."""
    n, h, d = x.shape
    lmax, half = cos.shape
    _need(tuple(sin.shape) == (lmax, half) and half * 2 == d,
          f"batched_rope_decode: cos/sin shape [Lmax, {half}] mismatches D={d}")
    _need(offsets.shape[0] == n, f"batched_rope_decode: offsets N={offsets.shape[0]} mismatches X N={n}")
    _need(cos.dtype == x.dtype and sin.dtype == x.dtype, "batched_rope_decode: cos/sin dtype must match X")
    _u32("batched_rope_decode: offsets must be U32", offsets)
    _contig("batched_rope_decode", x=x, cos=cos, sin=sin, offsets=offsets)
    check(lib.vx_rope_inplace(x.data_ptr(), cos.data_ptr(), sin.data_ptr(), offsets.data_ptr(), n, h, d, lmax,
                              _dt(x, "batched_rope_decode"), _stream()))


def batched_scatter(pool, values, page_ids, slots):
    """batched_scatter (metal_kernels.rs:1543-1548): pool[page_ids[n], h, slots[n], :] = values[n]."""
    p, h, s, d = pool.shape
    n, vh, vd = values.shape
    _need(vh == h and vd == d, f"batched_scatter: values [{n},{vh},{vd}] mismatches pool [_,{h},_,{d}]")
    _need(page_ids.shape[0] == n and slots.shape[0] == n, "batched_scatter: page_ids/slots N mismatches values N")
    _need(pool.dtype == values.dtype, "batched_scatter: pool/values dtype mismatch")
    _u32("batched_scatter: page_ids and slots must be U32", page_ids, slots)
    _contig("batched_scatter", pool=pool, values=values, page_ids=page_ids, slots=slots)
    check(lib.vx_kv_scatter(pool.data_ptr(), values.data_ptr(), page_ids.data_ptr(), slots.data_ptr(), n, p, h,
                            s, d, _dt(pool, "batched_scatter"), _stream()))


# ------------------------------------------------------------------ acceptance
def argmax_rows(logits):
    _contig("argmax", logits=logits)
    rows, vocab = logits.shape
    out = torch.zeros(rows, dtype=torch.int32, device=logits.device)
    check(lib.vx_argmax_rows(logits.data_ptr(), out.data_ptr(), rows, vocab, _dt(logits, "argmax"), _stream()))
    return out


def accept_greedy(logits, candidates):
    """logits [B, k+1, V]; candidates [B, k] -> (accepted [B], tokens [B, k+1])."""
    b, r, v = logits.shape
    _need(tuple(candidates.shape) == (b, r - 1), "accept_greedy: candidates must be [B, k]")
    _u32("accept_greedy: candidates must be U32", candidates)
    _contig("accept_greedy", logits=logits, candidates=candidates)
    acc = torch.zeros(b, dtype=torch.int32, device=logits.device)
    tok = torch.zeros((b, r), dtype=torch.int32, device=logits.device)
    check(lib.vx_accept_greedy(logits.data_ptr(), candidates.data_ptr(), acc.data_ptr(), tok.data_ptr(), b,
                               r - 1, v, _dt(logits, "accept_greedy"), _stream()))
    return acc, tok


def accept_stochastic(target_logits, draft_logits, candidates, uniforms, temperature):
    b, r, v = target_logits.shape
    _need(tuple(draft_logits.shape) == (b, r - 1, v) and draft_logits.dtype == target_logits.dtype,
          "accept_stochastic: draft logits must be [B, k, V] in the target's dtype")
    _need(tuple(candidates.shape) == (b, r - 1), "accept_stochastic: candidates must be [B, k]")
    _need(uniforms.dtype == torch.float32 and tuple(uniforms.shape) == (b, r, 4),
          "accept_stochastic: uniforms must be f32 [B, k+1, 4]")
    _u32("accept_stochastic: candidates must be U32", candidates)
    _contig("accept_stochastic", target_logits=target_logits, draft_logits=draft_logits, candidates=candidates,
            uniforms=uniforms)
    acc = torch.zeros(b, dtype=torch.int32, device=target_logits.device)
    tok = torch.zeros((b, r), dtype=torch.int32, device=target_logits.device)
    check(lib.vx_accept_stochastic(target_logits.data_ptr(), draft_logits.data_ptr(), candidates.data_ptr(),
                                   uniforms.data_ptr(), acc.data_ptr(), tok.data_ptr(), b, r - 1, v,
                                   temperature, _dt(target_logits, "accept_stochastic"), None, 0, _stream()))
    return acc, tok


def sample_rows(logits, uniforms, temperature, uniform_stride=1):
    rows, v = logits.shape
    _need(uniforms.dtype == torch.float32 and uniforms.numel() >= (rows - 1) * uniform_stride + 1,
          "sample: uniforms must be f32 with one value per row")
    _contig("sample", logits=logits, uniforms=uniforms)
    out = torch.zeros(rows, dtype=torch.int32, device=logits.device)
    check(lib.vx_sample_rows(logits.data_ptr(), uniforms.data_ptr(), uniform_stride, out.data_ptr(), rows, v,
                             temperature, _dt(logits, "sample"), None, 0, _stream()))
    return out


def kv_compact_path(pages, block_tables, kv_offsets, accepted, path):
    """Move each sequence's accepted tree path to consecutive KV positions
    (vx_kv_compact_path): pages is an engine.PagedKvCache; block_tables
    uint32 [B, max_blocks], kv_offsets uint32 [B], accepted int32 [B] and
    path int32 [B, r] are device tensors (accepted / path as accept_tree
    returns them)."""
    b, mb = block_tables.shape
    _need(path.dim() == 2 and path.shape[0] == b and accepted.shape[0] == b and kv_offsets.shape[0] == b,
          "kv_compact_path: shape mismatch")
    _u32("kv_compact_path: index tensors must be 32-bit", block_tables, kv_offsets, accepted, path)
    _contig("kv_compact_path", block_tables=block_tables, kv_offsets=kv_offsets, accepted=accepted, path=path)
    check(lib.vx_kv_compact_path(pages._h, block_tables.data_ptr(), mb, kv_offsets.data_ptr(), accepted.data_ptr(),
                                 path.data_ptr(), b, path.shape[1], _stream()))


def accept_tree(logits, parents, node_tokens):
    """logits [B, R, V]; parents: host ints (parents[0] = -1); node_tokens [B, R]."""
    import ctypes as C

    b, r, v = logits.shape
    _need(len(parents) == r, f"accept_tree: {len(parents)} parents for {r} nodes")
    _need(tuple(node_tokens.shape) == (b, r), "accept_tree: node_tokens must be [B, R]")
    _u32("accept_tree: node_tokens must be U32", node_tokens)
    _contig("accept_tree", logits=logits, node_tokens=node_tokens)
    par = (C.c_int32 * r)(*[int(x) for x in parents])
    acc = torch.zeros(b, dtype=torch.int32, device=logits.device)
    path = torch.zeros((b, r), dtype=torch.int32, device=logits.device)
    tok = torch.zeros((b, r), dtype=torch.int32, device=logits.device)
    check(lib.vx_accept_tree(logits.data_ptr(), C.cast(par, C.c_void_p), node_tokens.data_ptr(), acc.data_ptr(),
                             path.data_ptr(), tok.data_ptr(), b, r, v, _dt(logits, "accept_tree"), _stream()))
    return acc, path, tok
