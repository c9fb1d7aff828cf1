"""Cache-write side of HSA decoding: append a chunk's keys and values to the KV cache.

The reference writes each generated chunk's roped keys and values into ``kv_cache["k"/"v"]``
with slice assignments, and compresses the written, segment-aligned token range into
``kv_cache["k_coarse"/"v_coarse"]`` (``wan/modules/causal_model.py:286-327`` ``write_coarse_cache``,
``:393-405`` the direct insert). Every later attention call then pools the whole key cache again
for routing (``wan/modules/hsa/routing.py:45-61`` over all ``kv_len`` tokens).

:func:`kv_append` does the same writes on the GPU, in place, and keeps one more tensor beside
the cache: ``kv_cache["k_block_sums"]``, the fp32 sums of every key block (``[B, H,
ceil(cap / block_size), D]``), recomputed for the blocks the chunk touches only. A routing call
over the first ``L`` cache tokens forms its block means from these sums exactly as pooling the
keys would (the means' rounding depends on ``L``, which is why sums and not means are kept), so
it pools only the queries: pass them as ``hsa_attention(..., k_block_sums=...)``.

The reference assigns into clones of the cache tensors and commits them after the step
(``clone_cache_tensors``); the clones cost two full cache copies per call and change nothing in
what attention sees, so the writes here go to the cache itself.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from .. import _lib
from .attention import _compress

__all__ = ["kv_append", "new_block_sums"]


def new_block_sums(k_cache: torch.Tensor, block_size: int) -> torch.Tensor:
    """Zeroed fp32 key block sums ``[B, H, ceil(cap / block_size), D]`` for a ``[B, cap, H, D]`` cache."""
    bsz, cap, heads, d = k_cache.shape
    return torch.zeros((bsz, heads, math.ceil(cap / block_size), d), dtype=torch.float32, device=k_cache.device)


def kv_append(kv_cache: dict, k_new: torch.Tensor, v_new: torch.Tensor, *, write_start: int,
              block_size: Optional[int] = None, hsa_module=None, heads: Optional[Sequence[int]] = None) -> dict:
    """Write ``k_new`` / ``v_new`` ``[B, n, H, D]`` into cache tokens ``[write_start, write_start + n)``.

    * ``kv_cache["k"]`` / ``kv_cache["v"]`` (``[B, cap, H, D]``, bf16 or fp32): the slice
      assignment of ``causal_model.py:398-400``.
    * ``kv_cache["k_block_sums"]`` (created on first use when ``block_size`` is given): the sums
      of every key block holding a new token are recomputed over cache tokens
      ``[0, write_start + n)``, for ``heads`` (default all; routing reads the sparse heads only).
    * ``kv_cache["k_coarse"]`` / ``["v_coarse"]``, when present and ``hsa_module`` (an
      :class:`~worldattention_amd.hsa.HSAAttention`) is given: the chunk is compressed straight
      into the slots ``hsa_module.token_range_to_coarse(write_start, write_start + n)`` names
      (``write_coarse_cache``, ``causal_model.py:296-318``; the range must be segment-aligned,
      as there).

    Returns the reference's update record fields: ``write_start_index``, ``write_end_index``,
    ``new_k``, ``new_v``, ``new_k_coarse``, ``new_v_coarse`` (views of the written slots, or None).
    """
    kc, vc = kv_cache["k"], kv_cache["v"]
    dev = _lib.require_gpu(kc, vc, k_new, v_new)
    if kc.shape != vc.shape or kc.dtype != vc.dtype or kc.dim() != 4:
        raise ValueError(f"cache k / v must be matching [B, cap, H, D] tensors, got {tuple(kc.shape)} and "
                         f"{tuple(vc.shape)}")
    bsz, cap, heads_n, d = kc.shape
    if k_new.shape != v_new.shape or k_new.dim() != 4 or k_new.shape[0] != bsz or tuple(k_new.shape[2:]) != (heads_n, d):
        raise ValueError(f"new k / v must be [B={bsz}, n, H={heads_n}, D={d}], got {tuple(k_new.shape)} and "
                         f"{tuple(v_new.shape)}")
    n = k_new.shape[1]
    start = int(write_start)
    if start < 0 or start + n > cap:
        raise ValueError(f"tokens [{start}, {start + n}) do not fit a cache of {cap}")
    if kc.stride(-1) != 1 or vc.stride(-1) != 1:
        raise ValueError("cache channel dimension must be contiguous")
    k_src = k_new.to(kc.dtype) if k_new.dtype != kc.dtype else k_new
    v_src = v_new.to(kc.dtype) if v_new.dtype != kc.dtype else v_new
    k_src = k_src if k_src.stride(-1) == 1 else k_src.contiguous()
    v_src = v_src if v_src.stride(-1) == 1 else v_src.contiguous()

    sums = kv_cache.get("k_block_sums")
    if sums is None and block_size is not None:
        sums = new_block_sums(kc, block_size)
        kv_cache["k_block_sums"] = sums
    bs = 0
    if sums is not None:
        if block_size is None:
            raise ValueError("kv_cache holds k_block_sums: pass the block_size they were made with")
        bs = int(block_size)
        if (sums.dtype != torch.float32 or not sums.is_contiguous()
                or tuple(sums.shape) != (bsz, heads_n, math.ceil(cap / bs), d)):
            raise ValueError(f"k_block_sums must be contiguous fp32 [{bsz}, {heads_n}, {math.ceil(cap / bs)}, {d}], "
                             f"got {sums.dtype} {tuple(sums.shape)}")
    heads_t = _lib.head_list(heads, dev) if heads is not None else None
    coarse = hsa_module is not None and "k_coarse" in kv_cache and "v_coarse" in kv_cache and n > 0
    if coarse:  # validated before anything is written
        c0, c1 = hsa_module.token_range_to_coarse(start, start + n)

    ck, cv, nk, nv = _lib.blhd(kc), _lib.blhd(vc), _lib.blhd(k_src), _lib.blhd(v_src)
    args = _lib.KvAppendArgs(ck[0], ck[1], ck[2], ck[3], cv[0], cv[1], cv[2], cv[3],
                             nk[0], nk[1], nk[2], nk[3], nv[0], nv[1], nv[2], nv[3], _lib.dtype_code(kc),
                             bsz, cap, heads_n, d, start, n, _lib.ptr(sums), bs, _lib.ptr(heads_t),
                             0 if heads_t is None else heads_t.numel())
    _lib.call("wa_kv_append", args, _lib.stream_ptr(dev))

    new_kc = new_vc = None
    if coarse:
        new_kc = kv_cache["k_coarse"][:, c0:c1]
        new_vc = kv_cache["v_coarse"][:, c0:c1]
        seg, bsm = hsa_module.proj_segment_len, hsa_module.block_size
        with torch.no_grad():
            _compress(k_src, hsa_module.k_proj_mat, segment_len=seg, block_size=bsm, layout="blhd", out=new_kc)
            _compress(v_src, hsa_module.v_proj_mat, segment_len=seg, block_size=bsm, layout="blhd", out=new_vc)
    return {
        "action": "direct_insert",
        "write_start_index": start,
        "write_end_index": start + n,
        "new_k": kc[:, start:start + n],
        "new_v": vc[:, start:start + n],
        "new_k_coarse": new_kc,
        "new_v_coarse": new_vc,
    }
