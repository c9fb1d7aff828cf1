"""Block-sparse attention on the GPU behind the reference's two sparse-branch entry points.

* :func:`block_sparse_attention` — the Triton module's API
  (``wan/modules/hsa/block_sparse_triton.py:371-382``): ``(q2k_index, q2k_num)`` for inference, or
  ``block_map`` for the differentiable path (``:353-368``).
* :func:`block_sparse_attention_reference` — the torch module's API
  (``wan/modules/hsa/block_sparse_torch.py:16-64``).
* :func:`map_to_index` — ``block_sparse_triton.py:44-57``.

Both attention entry points run ``wa_bsa_fwd`` (bf16 MFMA, fp32 accumulation); the backward runs
``wa_bsa_bwd``. Inputs are ``[B, H, N, D]`` padded to the block size, as in the reference.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _lib

__all__ = ["block_sparse_attention", "block_sparse_attention_reference", "map_to_index", "bsa_forward",
           "bsa_backward"]


def map_to_index(block_map: torch.Tensor):
    """Boolean ``[B, H, Nq, Nkv]`` mask -> ascending ``(index, num)``, index padded with -1."""
    dev = _lib.require_gpu(block_map)
    m = block_map.to(torch.bool).contiguous()
    index = torch.empty(m.shape, dtype=torch.int32, device=dev)
    num = torch.empty(m.shape[:-1], dtype=torch.int32, device=dev)
    rows = m.numel() // max(m.shape[-1], 1)
    _lib.call("wa_map_to_index", m.data_ptr(), rows, m.shape[-1], index.data_ptr(), num.data_ptr(),
              _lib.stream_ptr(dev))
    return index, num


_UNIT_CACHE: dict = {}


def unit_table(bsz: int, visits_per_slot, nq: int, split: int, device) -> tuple[torch.Tensor, int]:
    """Device ``[n, 2]`` int32 list of (row, split) units when every row's visit count is known on
    the host (top-k routing: ``num = min(k_h, Nkv)``), ordered head by head so that consecutive
    units — which the kernel places on the same XCD — share key blocks. A row with no visits gets
    its split-0 unit, which writes the empty row. Cached per shape."""
    key = (str(device), bsz, tuple(visits_per_slot), nq, split)
    hit = _UNIT_CACHE.get(key)
    if hit is None:
        units = []
        n_slots = len(visits_per_slot)
        for b in range(bsz):
            for hs, nv in enumerate(visits_per_slot):
                ns = -(-int(nv) // split) if nv > 0 else 1
                for qb in range(nq):
                    row = (b * n_slots + hs) * nq + qb
                    units.extend((row, sp) for sp in range(ns))
        t = torch.tensor(units if units else [(0, 0)], dtype=torch.int32, device=device).view(-1, 2)
        hit = (t, len(units))
        _UNIT_CACHE[key] = hit
    return hit


def bsa_forward(q, k, v, *, index, num, block_size, layout="bhld", block_sizes=None, heads=None,
                out=None, out_dtype=None, want_lse=False, epilogue=_lib.WA_EPI_PLAIN, x=None, gate_w=None,
                gate_b=None, gate_pre_bf16=False, gate_out_bf16=False, attn_round_bf16=False, lq=None,
                lkv=None, visits=None, split=None, arrivals=None, noalloc=False, scale=0.0):
    """Launch ``wa_bsa_fwd`` on bf16 q/k/v in ``layout`` ("bhld" = [B, H, L, D], "blhd" = [B, L, H, D]).

    ``index=None`` attends densely to every key block. ``visits`` (optional) gives each launched
    head's exact visit count ``min(num, width)`` when the host knows it (top-k routing): the launch
    then covers exactly the needed (row, split) units. ``arrivals`` (optional): an int32 tensor of
    at least ``B * n_heads * ceil(lq / block_size)`` zeros (left zero), which spares the launch
    clearing its own. ``noalloc``: launch ``wa_bsa_fwd_noalloc`` instead, whose workspace is the
    library's static device array (no workspace tensor; ``arrivals`` must be None). ``scale``:
    the logit scale (0: ``D ** -0.5``). An empty ``heads`` list launches nothing. Returns
    ``(out, lse)``.
    """
    dev = _lib.require_gpu(q, k, v)
    strides = _lib.bhld if layout == "bhld" else _lib.blhd
    if layout == "bhld":
        bsz, nheads, ltok, d = q.shape
        lkv_tok = k.shape[2]
    else:
        bsz, ltok, nheads, d = q.shape
        lkv_tok = k.shape[1]
    lq = ltok if lq is None else lq
    lkv = lkv_tok if lkv is None else lkv
    if out is None:
        shape = (bsz, nheads, ltok, d) if layout == "bhld" else (bsz, ltok, nheads, d)
        out = torch.empty(shape, dtype=out_dtype or q.dtype, device=dev)
    lse = torch.empty((bsz, nheads, lq), dtype=torch.float32, device=dev) if want_lse else None
    qp, q_sb, q_st, q_sh = strides(q)
    kp, k_sb, k_st, k_sh = strides(k)
    vp, v_sb, v_st, v_sh = strides(v)
    op, o_sb, o_st, o_sh = strides(out)
    if x is not None:
        xp, x_sb, x_st, x_sh = strides(x)
        x_dt = _lib.dtype_code(x)
    else:
        xp, x_sb, x_st, x_sh, x_dt = None, 0, 0, 0, 0
    nkv = -(-lkv // block_size)
    nq = -(-lq // block_size)
    width = index.shape[-1] if index is not None else nkv
    n_slots = heads.numel() if heads is not None else nheads
    if n_slots == 0:
        return out, lse
    split = int(split or _lib.bsa_default_split(block_size))
    units, n_units, max_visits = None, 0, width
    if visits is not None:
        vis = [max(0, min(int(n), width)) for n in visits]
        if len(vis) != n_slots:
            raise ValueError(f"visits lists {len(vis)} heads, launch has {n_slots}")
        units, n_units = unit_table(bsz, vis, nq, split, dev)
        max_visits = max(max(vis), 1)
    rows = bsz * n_slots * nq
    if arrivals is not None and (arrivals.dtype != torch.int32 or arrivals.numel() < rows
                                 or not arrivals.is_contiguous() or arrivals.device != dev):
        raise ValueError(f"arrivals must be a contiguous int32 tensor of >= {rows} elements on {dev}")
    if noalloc:
        if arrivals is not None:
            raise ValueError("noalloc launches keep their arrival counters in the static scratch array")
        ws = None
    else:
        ws_bytes = _lib.lib().wa_bsa_fwd_workspace_bytes(rows, max_visits, split, block_size, d)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    args = _lib.BsaFwdArgs(
        qp, q_sb, q_st, q_sh, kp, k_sb, k_st, k_sh, vp, v_sb, v_st, v_sh,
        op, o_sb, o_st, o_sh, _lib.dtype_code(out), _lib.ptr(lse),
        _lib.ptr(index), _lib.ptr(num), width, _lib.ptr(block_sizes),
        *_lib.heads_arg(heads),
        bsz, nheads, lq, lkv, d, block_size, float(scale), epilogue,
        xp, x_sb, x_st, x_sh, x_dt, _lib.ptr(gate_w), _lib.ptr(gate_b),
        int(gate_pre_bf16), int(gate_out_bf16), int(attn_round_bf16),
        _lib.ptr(ws), _lib.ptr(units), n_units, max_visits, split, _lib.ptr(arrivals))
    _lib.call("wa_bsa_fwd_noalloc" if noalloc else "wa_bsa_fwd", args, _lib.stream_ptr(dev))
    return out, lse


# Head dims the kernels take; any other head dim up to 128 runs zero-padded to the next one at
# its own scale (zero channels add nothing to q . k, and the output's padding is cut off).
KERNEL_HEAD_DIMS = (64, 128)


def padded_head_dim(d: int, dims=KERNEL_HEAD_DIMS) -> int:
    """The kernel head dim a head dim of ``d`` runs at: the smallest of ``dims`` not below it."""
    for kd in dims:
        if d <= kd:
            return kd
    raise ValueError(f"head_dim must be at most {dims[-1]} for the gfx950 kernels, got {d}")


def _pad_qkv(q, k, v):
    """``(q, k, v, d, scale)`` with the head dim zero-padded to a kernel head dim (differentiable);
    ``scale`` is 0 (the kernel default) when no padding was needed."""
    d = q.shape[-1]
    dp = padded_head_dim(d)
    if dp == d:
        return q, k, v, d, 0.0
    pad = (0, dp - d)
    return (torch.nn.functional.pad(q, pad), torch.nn.functional.pad(k, pad), torch.nn.functional.pad(v, pad), d,
            d ** -0.5)


def _check_padded(q, k, index, num, block_size):
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError("expected [B, H, N, D] tensors")
    if q.shape[2] % block_size or k.shape[2] % block_size:
        raise ValueError(f"token counts must be multiples of the block size {block_size}")
    nq = q.shape[2] // block_size
    if index.shape[:3] != (q.shape[0], q.shape[1], nq) or num.shape != (q.shape[0], q.shape[1], nq):
        raise ValueError("q2k_index / q2k_num do not match the query blocks")


def _prep(t):
    return _lib.kernel_ready(t, torch.bfloat16)


class _BlockSparseAttention(torch.autograd.Function):
    """Differentiable block-sparse attention (reference ``block_sparse_triton.py:353-368``)."""

    @staticmethod
    def forward(ctx, q, k, v, index, num, block_sizes, block_size, scale=0.0):
        qb, kb, vb = _prep(q), _prep(k), _prep(v)
        # fp32 output: the backward's delta = rowsum(o * do) uses it unrounded
        out, lse = bsa_forward(qb, kb, vb, index=index, num=num, block_size=block_size,
                               block_sizes=block_sizes, out_dtype=torch.float32, want_lse=True, scale=scale)
        ctx.save_for_backward(qb, kb, vb, out, lse, index, num, block_sizes)
        ctx.block_size = block_size
        ctx.scale = scale
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        return out.to(q.dtype)

    @staticmethod
    def backward(ctx, grad_out):
        qb, kb, vb, out, lse, index, num, block_sizes = ctx.saved_tensors
        dq, dk, dv = bsa_backward(qb, kb, vb, out, lse, grad_out, index=index, num=num,
                                  block_size=ctx.block_size, block_sizes=block_sizes, scale=ctx.scale)
        qd, kd, vd = ctx.dtypes
        return dq.to(qd), dk.to(kd), dv.to(vd), None, None, None, None, None


def bsa_backward(q, k, v, out, lse, grad_out, *, index, num, block_size, block_sizes=None, layout="bhld",
                 heads=None, lq=None, lkv=None, dq=None, dk=None, dv=None, scale=0.0):
    """Gradients of :func:`bsa_forward` (``wa_bsa_bwd``)."""
    from . import _bwd
    return _bwd.bsa_backward(q, k, v, out, lse, grad_out, index=index, num=num, block_size=block_size,
                             block_sizes=block_sizes, layout=layout, heads=heads, lq=lq, lkv=lkv,
                             dq=dq, dk=dk, dv=dv, scale=scale)


def block_sparse_attention(q, k, v, *, block_sizes, q2k_index=None, q2k_num=None, block_map=None):
    """Block-sparse attention over ``[B, H, N, D]`` tensors padded to the block size.

    Pass ``block_map`` for a differentiable call, or ``(q2k_index, q2k_num)`` for inference.
    Returns ``[B, H, N, D]`` in ``q.dtype``.
    """
    _lib.require_gpu(q, k, v)
    block_size = k.shape[2] // block_sizes.numel()
    if block_map is not None:
        index, num = map_to_index(block_map)
        _check_padded(q, k, index, num, block_size)
        qx, kx, vx, d, scale = _pad_qkv(q, k, v)
        out = _BlockSparseAttention.apply(qx, kx, vx, index, num, block_sizes.to(torch.int32).contiguous(),
                                          block_size, scale)
        return out[..., :d].contiguous() if scale else out
    if q2k_index is None or q2k_num is None:
        raise ValueError("provide either block_map or both q2k_index and q2k_num")
    return block_sparse_attention_reference(q, k, v, q2k_index, q2k_num, block_sizes, block_size)


def block_sparse_attention_reference(q, k, v, q2k_index, q2k_num, block_sizes, block_size: int):
    """Attention over selected blocks for ``[B, H, N, D]`` inputs padded to ``block_size``.

    Same contract as ``block_sparse_torch.py:16-64`` (first ``num`` slots, ids clamped, partial
    block masked, empty rows 0, result in ``q.dtype``), computed by the HIP kernel (bf16 operands,
    fp32 accumulation). Differentiable in q, k, v.
    """
    _lib.require_gpu(q, k, v)
    index = q2k_index.to(torch.int32).contiguous()
    num = q2k_num.to(torch.int32).contiguous()
    _check_padded(q, k, index, num, block_size)
    sizes = block_sizes.to(device=q.device, dtype=torch.int32).contiguous()
    qx, kx, vx, d, scale = _pad_qkv(q, k, v)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        out = _BlockSparseAttention.apply(qx, kx, vx, index, num, sizes, block_size, scale)
    else:
        out_dtype = torch.float32 if q.dtype == torch.float32 else torch.bfloat16
        out, _ = bsa_forward(_prep(qx), _prep(kx), _prep(vx), index=index, num=num, block_size=block_size,
                             block_sizes=sizes, out_dtype=out_dtype, scale=scale)
        out = out.to(q.dtype)
    return out[..., :d].contiguous() if scale else out
