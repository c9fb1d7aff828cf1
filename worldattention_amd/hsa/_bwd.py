"""Host wrapper of ``wa_bsa_bwd``: gradients of the block-sparse attention.

Replaces the Triton backward of ``wan/modules/hsa/block_sparse_triton.py:142-368`` (and the autograd
of ``block_sparse_torch.py:16-64``) for any query / key lengths.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["bsa_backward"]


def bsa_backward(q, k, v, out, lse, grad_out, *, index, num, block_size, block_sizes=None, layout="bhld",
                 heads=None, lq=None, lkv=None, dq=None, dk=None, dv=None, accumulate=False, scale=0.0):
    """``(dq, dk, dv)`` of :func:`bsa_forward` in ``layout`` (fp32; given ``dk`` / ``dv`` may be bf16).

    ``out`` is the forward's attention output (fp32 preferred, it sets ``delta``), ``lse`` its
    natural-log log-sum-exp ``[B, H, Lq]``; ``scale`` the forward's logit scale (0: ``D ** -0.5``).
    Given ``dq`` / ``dk`` / ``dv`` buffers are written, or
    added to with ``accumulate`` (fp32 only); only the heads in ``heads`` (device int32) are touched.
    """
    dev = _lib.require_gpu(q, k, v, out, grad_out)
    strides = _lib.bhld if layout == "bhld" else _lib.blhd
    if layout == "bhld":
        bsz, nheads, ltok, d = q.shape
        lkv_tok = k.shape[2]
    else:
        bsz, ltok, nheads, d = q.shape
        lkv_tok = k.shape[1]
    lq = ltok if lq is None else lq
    lkv = lkv_tok if lkv is None else lkv
    if dq is None:
        dq = torch.zeros(q.shape, dtype=torch.float32, device=dev)
    if dk is None:
        dk = torch.zeros(k.shape, dtype=torch.float32, device=dev)
    if dv is None:
        dv = torch.zeros(v.shape, dtype=torch.float32, device=dev)
    if dk.dtype != dv.dtype or dk.dtype not in (torch.float32, torch.bfloat16) or dq.dtype != torch.float32:
        raise ValueError("dq must be fp32 and dk / dv both fp32 or both bf16")
    if accumulate and dk.dtype != torch.float32:
        raise ValueError("bf16 dk / dv are written, not accumulated")
    grad_out = grad_out if grad_out.stride(-1) == 1 else grad_out.contiguous()
    n_slots = heads.numel() if heads is not None else nheads
    if n_slots == 0:
        return dq, dk, dv
    ws = torch.empty((_lib.lib().wa_bsa_bwd_workspace_bytes(bsz, n_slots, lq, lkv, d, block_size),),
                     dtype=torch.uint8, device=dev)
    width = index.shape[-1] if index is not None else 0
    args = _lib.BsaBwdArgs(
        *strides(q), *strides(k), *strides(v),
        *strides(out), _lib.dtype_code(out),
        *strides(grad_out), _lib.dtype_code(grad_out),
        lse.data_ptr(), _lib.ptr(index), _lib.ptr(num), width, _lib.ptr(block_sizes),
        *_lib.heads_arg(heads),
        bsz, nheads, lq, lkv, d, block_size, float(scale),
        *strides(dq), int(accumulate), *strides(dk), int(accumulate), *strides(dv), int(accumulate),
        ws.data_ptr(), _lib.dtype_code(dk))
    _lib.call("wa_bsa_bwd", args, _lib.stream_ptr(dev))
    return dq, dk, dv
