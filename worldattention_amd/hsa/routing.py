"""Head-adaptive block routing on the GPU, with the reference's call signatures.

Mirrors ``wan/modules/hsa/routing.py`` (``BlockRouting`` :25-42, ``block_mean_pool`` :45-61,
``block_attention_map`` :64-68, ``build_block_routing`` :71-118, helpers :121-142). The compute
runs in ``libworldattention_amd`` (``wa_block_mean_pool``, ``wa_route``); sorting is stable, so
equal weights keep ascending block order. Adds the north-star per-head top-k rule
(:func:`build_topk_routing`).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from .. import _lib

__all__ = [
    "BlockRouting",
    "build_block_routing",
    "build_topk_routing",
    "block_attention_map",
    "block_mean_pool",
    "block_counts",
    "pad_to_len",
    "variable_block_sizes",
]


class BlockRouting:
    """Which key blocks each query block attends to (same fields as the reference).

    index: ``[B, H, Nq, Nkv]`` int32 key-block ids, descending block-attention weight (stable).
    num: ``[B, H, Nq]`` int32 selected count per row (the first ``num`` entries of ``index``).
    mask: ``[B, H, Nq, Nkv]`` bool selection mask, or None.
    thresholds: ``[H]`` per-head coverage threshold (zeros for top-k routing).
    """

    __slots__ = ("index", "num", "mask", "thresholds")

    def __init__(self, index, num, mask, thresholds):
        self.index = index
        self.num = num
        self.mask = mask
        self.thresholds = thresholds


def block_counts(q_len: int, kv_len: int, block_size: int) -> tuple[int, int, int, int]:
    """Padded lengths and block counts (``routing.py:138-142``)."""
    q_pad = math.ceil(q_len / block_size) * block_size
    kv_pad = math.ceil(kv_len / block_size) * block_size
    return q_pad, kv_pad, q_pad // block_size, kv_pad // block_size


def pad_to_len(x: torch.Tensor, target_len: int) -> torch.Tensor:
    """Zero-pad ``[B, L, H, D]`` along the token axis (``routing.py:129-135``).

    The HIP kernels never need padded copies (they bound-check the trailing block); this helper
    is kept for API compatibility.
    """
    pad_len = target_len - x.shape[1]
    if pad_len <= 0:
        return x
    pad = torch.zeros((x.shape[0], pad_len, x.shape[2], x.shape[3]), device=x.device, dtype=x.dtype)
    return torch.cat([x, pad], dim=1)


def variable_block_sizes(kv_len: int, kv_len_padded: int, block_size: int, device) -> torch.Tensor:
    """Real token count of each key block (``routing.py:121-126``)."""
    kv_blocks = kv_len_padded // block_size
    sizes = torch.full((kv_blocks,), block_size, dtype=torch.int32, device=device)
    sizes[-1] = kv_len - (kv_blocks - 1) * block_size
    return sizes


def pool_blhd(x: torch.Tensor, logical_len: int, num_blocks: int, block_size: int,
              heads: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
              emulate: bool = True) -> torch.Tensor:
    """Block means of a ``[B, L, H, D]`` tensor into fp32 ``[B, H, N, D]`` (no transposes)."""
    dev = _lib.require_gpu(x)
    x = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
    if x.stride(-1) != 1:
        x = x.contiguous()
    b, _, h, d = x.shape
    if out is None:
        out = torch.empty((b, h, num_blocks, d), dtype=torch.float32, device=dev)
    p, sb, st, sh = _lib.blhd(x)
    args = _lib.PoolArgs(p, sb, st, sh, _lib.dtype_code(x), b, logical_len, h, d, block_size, num_blocks,
                         *_lib.heads_arg(heads), out.data_ptr(), int(emulate))
    _lib.call("wa_block_mean_pool", args, _lib.stream_ptr(dev))
    return out


def pool_blhd_many(jobs, block_size: int, heads: Optional[torch.Tensor] = None, emulate: bool = True):
    """:func:`pool_blhd` of several ``(x, logical_len, num_blocks)`` jobs in as few launches as
    possible (one for tensors of one dtype and alignment); returns their outputs in order."""
    if not jobs:
        return []
    dev = _lib.require_gpu(*(x for x, _, _ in jobs))
    outs, keep = [], []
    arr = (_lib.PoolArgs * len(jobs))()
    for i, (x, logical_len, num_blocks) in enumerate(jobs):
        x = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
        if x.stride(-1) != 1:
            x = x.contiguous()
        b, _, h, d = x.shape
        out = torch.empty((b, h, num_blocks, d), dtype=torch.float32, device=dev)
        p, sb, st, sh = _lib.blhd(x)
        arr[i] = _lib.PoolArgs(p, sb, st, sh, _lib.dtype_code(x), b, logical_len, h, d, block_size, num_blocks,
                               *_lib.heads_arg(heads), out.data_ptr(), int(emulate))
        outs.append(out)
        keep.append(x)
    _lib.call("wa_block_mean_pool_n", arr, len(jobs), _lib.stream_ptr(dev))
    return outs


def block_mean_pool(x: torch.Tensor, logical_len: int, num_blocks: int, block_size: int) -> torch.Tensor:
    """Mean-pool ``[B, H, num_blocks*block_size, D]`` into ``[B, H, num_blocks, D]``.

    Same contract and result dtype as ``routing.py:45-61``: a trailing partial block averages its
    real tokens only; with no partial block the result keeps ``x.dtype``, otherwise it is fp32.
    """
    dev = _lib.require_gpu(x)
    bsz, heads, tokens, d = x.shape
    if tokens != num_blocks * block_size:
        raise ValueError(f"expected {num_blocks * block_size} tokens, got {tokens}")
    src = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
    if src.stride(-1) != 1:
        src = src.contiguous()
    out = torch.empty((bsz, heads, num_blocks, d), dtype=torch.float32, device=dev)
    p, sb, st, sh = _lib.bhld(src)
    args = _lib.PoolArgs(p, sb, st, sh, _lib.dtype_code(src), bsz, logical_len, heads, d, block_size,
                         num_blocks, None, 0, out.data_ptr(), 1)
    _lib.call("wa_block_mean_pool", args, _lib.stream_ptr(dev))
    if logical_len % block_size == 0:
        return out.to(x.dtype)
    return out


def pool_for_routing(q, k, q_len: int, kv_len: int, block_size: int, heads=None, *, k_block_sums=None,
                     k_pooled=None):
    """Pooled queries and keys of one routing call, and the key arguments of :func:`_route`.

    The keys are pooled here unless the caller holds them: ``k_pooled`` (fp32 ``[B, H, >= Nkv, D]``
    block means of exactly these ``kv_len`` keys, e.g. :func:`pool_blhd`'s output) or
    ``k_block_sums`` (fp32 ``[B, H, >= Nkv, D]`` block sums, as :func:`worldattention_amd.hsa.kvcache.kv_append`
    keeps them for a cache; routing forms from them the means of the first ``kv_len`` tokens).
    Either way only the queries are pooled.
    """
    _, _, nq, nkv = block_counts(q_len, kv_len, block_size)
    if k_block_sums is not None and k_pooled is not None:
        raise ValueError("pass k_block_sums or k_pooled, not both")
    held = k_block_sums if k_block_sums is not None else k_pooled
    if held is None:
        qp, kp = pool_blhd_many([(q, q_len, nq), (k, kv_len, nkv)], block_size, heads=heads)
        return qp, kp, {}
    b, _, h, d = k.shape
    if (held.dtype != torch.float32 or held.dim() != 4 or held.shape[0] != b or held.shape[1] != h
            or held.shape[3] != d or held.shape[2] < nkv or not held.is_contiguous()):
        raise ValueError(f"cached key blocks must be contiguous fp32 [{b}, {h}, >= {nkv}, {d}], got "
                         f"{held.dtype} {tuple(held.shape)}")
    _lib.require_gpu(held, q)
    (qp,) = pool_blhd_many([(q, q_len, nq)], block_size, heads=heads)
    key_args = dict(nkv=nkv, k_pooled_blocks=held.shape[2])
    if k_block_sums is not None:
        key_args.update(k_sum_len=kv_len, block_size=block_size, k_sum_bf16=k.dtype == torch.bfloat16)
    return qp, held, key_args


def _route(probs, qp, kp, *, mode, tau_min=0.0, tau_max=1.0, head_k=None, heads=None,
           return_mask=False, want_probs=False, clear=None, nkv=None, k_pooled_blocks=0, k_sum_len=0,
           block_size=0, k_sum_bf16=False, scale=0.0):
    """``clear`` (optional): a contiguous int32 device tensor the launch zeroes (the arrivals of
    the block-sparse launch that follows). ``nkv`` / ``k_pooled_blocks`` / ``k_sum_len`` /
    ``block_size`` / ``k_sum_bf16``: cached key blocks (:func:`pool_for_routing`). ``scale``: the
    map's logit scale (0: the pooled vectors' ``D ** -0.5``)."""
    src = probs if probs is not None else qp
    dev = _lib.require_gpu(src, kp)
    if probs is not None:
        probs = probs.float().contiguous()
        bsz, nheads, nq, nkv = probs.shape
        d = 0
    else:
        qp = qp.float().contiguous()
        kp = kp.float().contiguous()
        bsz, nheads, nq, d = qp.shape
        nkv = kp.shape[2] if nkv is None else nkv
    index = torch.empty((bsz, nheads, nq, nkv), dtype=torch.int32, device=dev)
    # the kernel writes num of unrouted heads (0) and every threshold: no fill needed
    num = torch.empty((bsz, nheads, nq), dtype=torch.int32, device=dev)
    thresholds = torch.empty((nheads,), dtype=torch.float32, device=dev)
    mask = torch.zeros((bsz, nheads, nq, nkv), dtype=torch.bool, device=dev) if return_mask else None
    probs_out = (torch.empty((bsz, nheads, nq, nkv), dtype=torch.float32, device=dev)
                 if want_probs and probs is None else None)
    ws = None
    if mode == _lib.WA_ROUTE_GINI:
        nbytes = _lib.lib().wa_route_workspace_bytes(bsz, nheads, nq, nkv)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    head_k_t = None
    if head_k is not None:
        head_k_t = _lib.head_list(head_k, dev)
    # the threshold is tau_min + G * (tau_max - tau_min) in fp32, with the span formed in double
    args = _lib.RouteArgs(_lib.ptr(probs), _lib.ptr(qp), _lib.ptr(kp), bsz, nheads, nq, nkv, d, mode,
                          float(tau_min), float(tau_max - tau_min), _lib.ptr(head_k_t), *_lib.heads_arg(heads),
                          index.data_ptr(), num.data_ptr(),
                          thresholds.data_ptr(), _lib.ptr(mask), _lib.ptr(probs_out), _lib.ptr(ws),
                          _lib.ptr(clear), 0 if clear is None else clear.numel(), int(k_sum_len),
                          int(block_size), int(bool(k_sum_bf16)), int(k_pooled_blocks), float(scale))
    _lib.call("wa_route", args, _lib.stream_ptr(dev))
    return BlockRouting(index=index, num=num, mask=mask, thresholds=thresholds), probs_out


def block_attention_map(q_pooled: torch.Tensor, k_pooled: torch.Tensor) -> torch.Tensor:
    """fp32 ``softmax(qp kp^T / sqrt(D))`` over pooled blocks (``routing.py:64-68``)."""
    _, probs = _route(None, q_pooled, k_pooled, mode=_lib.WA_ROUTE_TOPK, head_k=None, want_probs=True)
    return probs


def build_block_routing(block_attn: torch.Tensor, tau_min: float, tau_max: float, *,
                        return_mask: bool = False) -> BlockRouting:
    """Gini cumulative-mass routing (``routing.py:71-118``) on the GPU.

    ``G_h`` = mean over (batch, query block) of ``sum_m (N+1-2m) p_(m) / N``;
    ``tau_h = tau_min + G_h (tau_max - tau_min)``; a sorted slot is kept while the mass strictly
    before it is below ``tau_h``.
    """
    route, _ = _route(block_attn, None, None, mode=_lib.WA_ROUTE_GINI, tau_min=tau_min, tau_max=tau_max,
                      return_mask=return_mask)
    return route


def build_topk_routing(block_attn: torch.Tensor, topk, *, return_mask: bool = False) -> BlockRouting:
    """North-star per-head top-k routing: ``num = min(k_h, Nkv)``, ties to the lowest block id.

    ``topk`` is an int or one budget per head (0 leaves a head unrouted).
    """
    nheads = block_attn.shape[1]
    ks = [int(topk)] * nheads if isinstance(topk, int) else [int(k) for k in topk]
    if len(ks) != nheads:
        raise ValueError(f"expected {nheads} per-head budgets, got {len(ks)}")
    route, _ = _route(block_attn, None, None, mode=_lib.WA_ROUTE_TOPK, head_k=ks, return_mask=return_mask)
    return route
