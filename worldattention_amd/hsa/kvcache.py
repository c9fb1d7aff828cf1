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

import ctypes
import math
from typing import Optional, Sequence

import torch

from .. import _lib
from .attention import _compress

__all__ = ["kv_append", "new_block_sums", "refresh_block_sums", "qkv_epilogue", "kv_roll", "cache_step"]


def new_block_sums(k_cache: torch.Tensor, block_size: int) -> torch.Tensor:
    """Zeroed fp32 key block sums ``[B, H, ceil(cap / block_size), D]`` for a ``[B, cap, H, D]`` cache."""
    bsz, cap, heads, d = k_cache.shape
    return torch.zeros((bsz, heads, math.ceil(cap / block_size), d), dtype=torch.float32, device=k_cache.device)


def refresh_block_sums(kv_cache: dict, length: int) -> None:
    """Recompute ``kv_cache["k_block_sums"]`` (if kept) for the first ``length`` cache tokens, e.g.
    after something other than these functions rewrote the keys (an HKV page install)."""
    sums = kv_cache.get("k_block_sums")
    if sums is None or length <= 0:
        return
    bs = int(kv_cache["k_block_sums_block_size"])
    kc = kv_cache["k"]
    dev = _lib.require_gpu(kc, sums)
    bsz, cap, heads_n, d = kc.shape
    p, sb, st, sh = _lib.blhd(kc)
    nblk = -(-int(length) // bs)
    args = _lib.PoolArgs(p, sb, st, sh, _lib.dtype_code(kc), bsz, int(length), heads_n, d, bs, nblk, None, 0,
                         sums.data_ptr(), 1, 0, sums.shape[2], 1)
    _lib.call("wa_block_mean_pool", args, _lib.stream_ptr(dev))


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
        kv_cache["k_block_sums_block_size"] = int(block_size)
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
                             bsz, cap, heads_n, d, start, n, _lib.ptr(sums), bs, *_lib.heads_arg(heads_t))
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


def _grid_rows(grid_sizes, batch: int):
    """Per-sample ``(f, h, w)`` rows from a ``[B, 3]`` tensor / nested list (one per sample, as the
    reference's ``grid_sizes``) or one triple for the whole batch."""
    if isinstance(grid_sizes, torch.Tensor):
        rows = grid_sizes.reshape(-1, 3).tolist()
    elif len(grid_sizes) and isinstance(grid_sizes[0], (list, tuple)):
        rows = [list(r) for r in grid_sizes]
    else:
        return [tuple(int(x) for x in grid_sizes)] * batch
    if len(rows) != batch:
        raise ValueError(f"grid_sizes holds {len(rows)} grids for a batch of {batch}")
    return [tuple(int(x) for x in r) for r in rows]


def _table(freqs: torch.Tensor, dev) -> torch.Tensor:
    """The RoPE table as device fp64 (re, im) pairs ``[rows, D/2, 2]``."""
    t = torch.view_as_real(freqs) if freqs.is_complex() else freqs
    if t.dtype != torch.float64:
        raise ValueError(f"freqs must be the complex128 RoPE table, got {freqs.dtype}")
    return t.to(dev).contiguous()


def qkv_epilogue(q, k, v, kv_cache: dict, *, grid_sizes, freqs, start_frame: int, write_start: int,
                 src_offset: int = 0, write_len: Optional[int] = None, norm_q=None, norm_k=None, eps: float = 1e-6,
                 block_size: Optional[int] = None) -> torch.Tensor:
    """One launch for a layer's q / k / v projections ``[B, n, H, D]``: returns ``rope(norm_q(q))``
    and writes ``rope(norm_k(k))`` / ``v`` tokens ``[src_offset, src_offset + write_len)`` to cache
    tokens ``[write_start, ...)`` (``wa_qkv_epilogue``). ``norm_q`` / ``norm_k``: the RMSNorm
    weights ``[H * D]`` (or None: no norm); ``freqs``: the model's complex128 RoPE table. With
    ``block_size``, ``kv_cache["k_block_sums"]`` is kept as :func:`kv_append` keeps it."""
    kc, vc = kv_cache["k"], kv_cache["v"]
    dev = _lib.require_gpu(q, k, v, kc, vc)
    if not (q.shape == k.shape == v.shape) or q.dim() != 4:
        raise ValueError(f"q, k, v must be matching [B, n, H, D], got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    bsz, n, heads, d = q.shape
    if kc.shape[0] != bsz or tuple(kc.shape[2:]) != (heads, d) or vc.shape != kc.shape:
        raise ValueError(f"cache {tuple(kc.shape)} does not hold [B={bsz}, cap, H={heads}, D={d}] tokens")
    dtype = kc.dtype
    if dtype not in (torch.bfloat16, torch.float32) or vc.dtype != dtype:
        raise ValueError(f"cache dtype must be bf16 or fp32, got {kc.dtype} / {vc.dtype}")
    if (norm_q is None) != (norm_k is None):
        raise ValueError("give both RMSNorm weights or neither")
    ready = [_lib.kernel_ready(t, dtype) for t in (q, k, v)]
    q_out = torch.empty((bsz, n, heads, d), dtype=dtype, device=dev)
    table = _table(freqs, dev)
    rows = _grid_rows(grid_sizes, bsz)
    f, gh, gw = rows[0]
    # samples with grids of their own (the reference loops over grid_sizes per sample)
    per_sample = (ctypes.c_int64 * (3 * bsz))(*[x for r in rows for x in r]) if len(set(rows)) > 1 else None
    wlen = n - src_offset if write_len is None else int(write_len)
    sums = None
    if block_size is not None:
        sums = kv_cache.get("k_block_sums")
        if sums is None:
            sums = new_block_sums(kc, block_size)
            kv_cache["k_block_sums"] = sums
            kv_cache["k_block_sums_block_size"] = int(block_size)
    wq = wk = None
    w_dtype = 0
    if norm_q is not None:
        if norm_q.numel() != heads * d or norm_k.numel() != heads * d:
            raise ValueError(f"RMSNorm weights must hold H * D = {heads * d} values")
        wdt = norm_q.dtype if norm_q.dtype in (torch.bfloat16, torch.float32) else torch.float32
        wq = norm_q.detach().to(dev, wdt).contiguous()
        wk = norm_k.detach().to(dev, wdt).contiguous()
        w_dtype = _lib.dtype_code(wq)
    qq, kk, vv = (_lib.blhd(t) for t in ready)
    qo, ck, cv = _lib.blhd(q_out), _lib.blhd(kc), _lib.blhd(vc)
    args = _lib.QkvEpilogueArgs(*qq, *kk, *vv, _lib.dtype_code(kc), bsz, n, heads, d, *qo, *ck, *cv,
                                kc.shape[1], int(write_start), int(src_offset), wlen, table.data_ptr(),
                                table.shape[0], f, gh, gw, int(start_frame), _lib.ptr(wq), _lib.ptr(wk), w_dtype,
                                float(eps), _lib.ptr(sums), int(block_size or 0), per_sample)
    _lib.call("wa_qkv_epilogue", args, _lib.stream_ptr(dev))
    return q_out


def kv_roll(kv_cache: dict, *, sink_tokens: int, num_evicted: int, num_rolled: int,
            block_size: Optional[int] = None, hsa_module=None, heads: Optional[Sequence[int]] = None) -> None:
    """Move cache tokens ``[sink + evicted, sink + evicted + rolled)`` to ``[sink, sink + rolled)``
    in place (``wa_kv_roll``), with the coarse rows of those segments when the cache has a coarse
    tier and ``hsa_module`` is given (``causal_model.py:326-356``), and the key block sums."""
    kc, vc = kv_cache["k"], kv_cache["v"]
    dev = _lib.require_gpu(kc, vc)
    bsz, cap, heads_n, d = kc.shape
    sums = kv_cache.get("k_block_sums")
    if sums is not None and block_size is None:
        raise ValueError("kv_cache holds k_block_sums: pass the block_size they were made with")
    heads_t = _lib.head_list(heads, dev) if heads is not None else None
    coarse = hsa_module is not None and "k_coarse" in kv_cache and "v_coarse" in kv_cache
    c_dst = c_src = c_rows = 0
    kcc = vcc = None
    if coarse:
        _, c_dst = hsa_module.token_range_to_coarse(0, int(sink_tokens))
        c_src, c_end = hsa_module.token_range_to_coarse(int(sink_tokens + num_evicted),
                                                        int(sink_tokens + num_evicted + num_rolled))
        c_rows = max(0, c_end - c_src)
        kcc, vcc = kv_cache["k_coarse"], kv_cache["v_coarse"]
        if kcc.dtype != kc.dtype or vcc.dtype != kc.dtype:
            raise ValueError("the coarse tier must have the cache dtype")
    kp, vp = _lib.blhd(kc), _lib.blhd(vc)
    kcp = _lib.blhd(kcc) if coarse else (None, 0, 0, 0)
    vcp = _lib.blhd(vcc) if coarse else (None, 0, 0, 0)
    args = _lib.KvRollArgs(*kp, *vp, _lib.dtype_code(kc), bsz, cap, heads_n, d, int(sink_tokens), int(num_evicted),
                           int(num_rolled), _lib.ptr(sums), int(block_size or 0), *_lib.heads_arg(heads_t), *kcp, *vcp,
                           kcc.shape[1] if coarse else 0, c_dst, c_src, c_rows)
    _lib.call("wa_kv_roll", args, _lib.stream_ptr(dev))


def _index(kv_cache: dict, key: str) -> int:
    t = kv_cache[key]
    return int(t.item()) if isinstance(t, torch.Tensor) else int(t)


def cache_step(kv_cache: dict, q, k, v, *, grid_sizes, freqs, current_start: int, sink_size: int,
               local_attn_size: int, max_attention_size: int, norm_q=None, norm_k=None, eps: float = 1e-6,
               hsa_module=None, block_size: Optional[int] = None, sink_recache_after_switch: bool = False):
    """The cache side of one ``CausalWanSelfAttention.forward`` call with a KV cache
    (``causal_model.py:268-437`` and the commit ``:1016-1119``), in place on the GPU.

    ``q``, ``k``, ``v``: the layer's projections ``[B, n, H, D]`` before the RMSNorm (weights
    ``norm_q`` / ``norm_k``, or None) and RoPE. The roll (when the window is full) is
    :func:`kv_roll`, the norm + RoPE + insert one :func:`qkv_epilogue` launch, and a coarse tier
    (``kv_cache["k_coarse"/"v_coarse"]`` with ``hsa_module``) gets the written segments compressed
    into its slots. ``kv_cache["global_end_index"]`` / ``["local_end_index"]`` move as the
    reference's commit moves them (not for a recompute). With ``block_size`` the key block sums are
    kept for routing (``hsa_attention(..., k_block_sums=...)``).

    Returns ``(roped_q, attn_k, attn_v, attn_kc, attn_vc, info)``: the attention inputs of
    ``run_hsa_core_attn`` (views of the cache where the window is one contiguous range; the
    reference's ``torch.cat`` of sink and local range otherwise) and the update record, whose
    ``"k_block_sums"`` is the tensor to pass to ``hsa_attention`` (None unless the window is the
    cache's first tokens and sums are kept).
    """
    rows = _grid_rows(grid_sizes, q.shape[0])
    frame_seqlen = rows[0][1] * rows[0][2]  # sample 0's frame, as causal_model.py:269 takes it
    start_frame = current_start // frame_seqlen
    n = q.shape[1]
    current_end = current_start + n
    sink = sink_size * frame_seqlen
    cap = kv_cache["k"].shape[1]
    global_end = _index(kv_cache, "global_end_index")
    local_end = _index(kv_cache, "local_end_index")
    coarse = hsa_module is not None and "k_coarse" in kv_cache and "v_coarse" in kv_cache
    recompute = current_end <= global_end and current_start > 0
    roll = local_attn_size != -1 and current_end > global_end and n + local_end > cap
    evicted = rolled = 0
    if roll:
        evicted = n + local_end - cap
        rolled = local_end - evicted - sink
        new_local_end = local_end + current_end - global_end - evicted
    else:
        new_local_end = local_end + current_end - global_end
    local_start = new_local_end - n
    write_start = max(local_start, sink) if recompute else local_start
    if not roll and sink_recache_after_switch:
        write_start = local_start
    offset = max(0, write_start - local_start)
    write_len = max(0, new_local_end - write_start)
    if coarse and write_len > 0:  # refused before anything is written, as the reference's step refuses
        c0, c1 = hsa_module.token_range_to_coarse(write_start, new_local_end)
    if roll:
        kv_roll(kv_cache, sink_tokens=sink, num_evicted=evicted, num_rolled=rolled, block_size=block_size,
                hsa_module=hsa_module if coarse else None)
    roped_q = qkv_epilogue(q, k, v, kv_cache, grid_sizes=rows, freqs=freqs, start_frame=start_frame,
                           write_start=write_start, src_offset=offset, write_len=write_len, norm_q=norm_q,
                           norm_k=norm_k, eps=eps, block_size=block_size)
    kc, vc = kv_cache["k"], kv_cache["v"]
    new_kc = new_vc = None
    if coarse and write_len > 0:
        new_kc, new_vc = kv_cache["k_coarse"][:, c0:c1], kv_cache["v_coarse"][:, c0:c1]
        seg, bsm = hsa_module.proj_segment_len, hsa_module.block_size
        with torch.no_grad():
            _compress(kc[:, write_start:new_local_end], hsa_module.k_proj_mat, segment_len=seg, block_size=bsm,
                      layout="blhd", out=new_kc)
            _compress(vc[:, write_start:new_local_end], hsa_module.v_proj_mat, segment_len=seg, block_size=bsm,
                      layout="blhd", out=new_vc)

    def coarse_slice(a, b):
        if not coarse:
            return None, None
        s0, s1 = hsa_module.token_range_to_coarse(a, b)
        return kv_cache["k_coarse"][:, s0:s1], kv_cache["v_coarse"][:, s0:s1]

    if sink > 0:
        budget = max_attention_size - sink
        if budget > 0:
            lsw = max(sink, new_local_end - budget)
            if lsw == sink:  # sink and local range are one contiguous run: views, no copy
                attn_k, attn_v = kc[:, :new_local_end], vc[:, :new_local_end]
                attn_kc, attn_vc = coarse_slice(0, new_local_end)
            else:
                attn_k = torch.cat([kc[:, :sink], kc[:, lsw:new_local_end]], dim=1)
                attn_v = torch.cat([vc[:, :sink], vc[:, lsw:new_local_end]], dim=1)
                attn_kc = attn_vc = None
                if coarse:
                    ks, vs = coarse_slice(0, sink)
                    kl, vl = coarse_slice(lsw, new_local_end)
                    attn_kc, attn_vc = torch.cat([ks, kl], dim=1), torch.cat([vs, vl], dim=1)
        else:
            attn_k, attn_v = kc[:, :sink], vc[:, :sink]
            attn_kc, attn_vc = coarse_slice(0, sink)
    else:
        ws = max(0, new_local_end - max_attention_size)
        attn_k, attn_v = kc[:, ws:new_local_end], vc[:, ws:new_local_end]
        attn_kc, attn_vc = coarse_slice(ws, new_local_end)
    if not recompute:
        for key, val in (("global_end_index", current_end), ("local_end_index", new_local_end)):
            if isinstance(kv_cache[key], torch.Tensor):
                kv_cache[key].fill_(val)
            else:
                kv_cache[key] = val
    info = {"action": "roll_and_insert" if roll else "direct_insert", "sink_tokens": sink,
            "num_rolled_tokens": rolled, "num_evicted_tokens": evicted, "local_start_index": local_start,
            "local_end_index": new_local_end, "write_start_index": write_start, "write_end_index": new_local_end,
            "new_k": kc[:, write_start:new_local_end], "new_v": vc[:, write_start:new_local_end],
            "new_k_coarse": new_kc, "new_v_coarse": new_vc, "current_end": current_end, "is_recompute": recompute}
    # the cached key sums describe the window only when it is the cache's first tokens
    prefix = attn_k.data_ptr() == kc.data_ptr() and attn_k.shape[1] == new_local_end
    info["k_block_sums"] = kv_cache.get("k_block_sums") if prefix and block_size is not None else None
    return roped_q, attn_k, attn_v, attn_kc, attn_vc, info
