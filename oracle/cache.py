"""CPU oracle for the KV-cache write side of a causal attention step — test infrastructure only.

Restates, on CPU tensors, what one ``CausalWanSelfAttention.forward`` call with a KV cache does
before its attention call and what ``_apply_cache_updates`` commits afterwards:

* ``rms_norm``: ``WanRMSNorm.forward`` (``wan/modules/model.py:78-86``);
* ``causal_rope``: ``causal_rope_apply`` (``wan/modules/causal_model.py:34-62``) through
  :func:`oracle.hkv.rope_apply_3d`;
* ``cache_step``: the index arithmetic, roll, insert and coarse-tier writes of
  ``run_cache_prepare_kv`` (``causal_model.py:286-437``) on clones of the cache, the attention
  window of ``run_hsa_core_attn`` (``:486-530``), and the commit of ``_apply_cache_updates``
  (``:1016-1119``) including the index update.

pinned by: ``tests/test_oracle_cache.py`` — the norm against an fp64 brute force and a constant-row
known answer; the rotation against a per-element cos/sin loop; the cache contents against the
sliding-window invariant (sink frames followed by the most recent frames, in order) over a run of
chunks with eviction and a recompute step; coarse slots against direct compression of the window.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import hkv as OK
from . import hsa as OH


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps)`` over the last dim in fp32, in x's dtype, times ``weight``."""
    if weight is None:
        return x
    xf = x.float()
    normed = (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).type_as(x)
    return normed * weight


def _grids(grid, batch: int):
    """Per-sample ``(f, h, w)`` rows: a triple is shared by the batch, a ``[B, 3]`` list / tensor
    gives each sample its own (``grid_sizes`` of ``causal_model.py:43``)."""
    rows = grid.tolist() if isinstance(grid, torch.Tensor) else grid
    if len(rows) and isinstance(rows[0], (list, tuple)):
        if len(rows) != batch:
            raise ValueError(f"{len(rows)} grids for a batch of {batch}")
        return [tuple(int(v) for v in r) for r in rows]
    return [tuple(int(v) for v in rows)] * batch


def causal_rope(x: torch.Tensor, grid, freqs: torch.Tensor, start_frame: int) -> torch.Tensor:
    """3-D RoPE of ``[B, L, H, D]``; ``grid``: one ``(f, h, w)`` for the batch or one per sample;
    each sample's tokens past its ``f * h * w`` pass through (``causal_model.py:34-62``, which loops
    over the samples)."""
    out = []
    for i, (f, h, w) in enumerate(_grids(grid, x.shape[0])):
        seq = f * h * w
        xi = x[i:i + 1]
        rot = OK.rope_apply_3d(xi[:, :seq], freqs, f, h, w, start_frame=start_frame)
        out.append(torch.cat([rot, xi[:, seq:]], dim=1) if seq < x.shape[1] else rot)
    return torch.cat(out, dim=0)


def cache_step(kv_cache: dict, q, k, v, *, grid, freqs, current_start: int, sink_size: int,
               local_attn_size: int, max_attention_size: int, norm_q=None, norm_k=None, eps: float = 1e-6,
               proj=None, sink_recache_after_switch: bool = False):
    """One cached attention step. ``kv_cache``: ``{"k", "v", "global_end_index",
    "local_end_index"}`` (+ ``"k_coarse"``, ``"v_coarse"``); ``proj``: ``(k_proj_mat, v_proj_mat,
    segment_len, block_size)`` of the HSA module when the coarse tier is kept.

    Returns ``(roped_q, attn_k, attn_v, attn_kc, attn_vc, info)``; the cache dict is updated in
    place as the commit leaves it.
    """
    b, n_tok, heads, d = q.shape  # the norms run over a token's H * D channels, before the head view
    q = rms_norm(q.reshape(b, n_tok, heads * d), norm_q, eps).reshape(b, n_tok, heads, d)
    k = rms_norm(k.reshape(b, n_tok, heads * d), norm_k, eps).reshape(b, n_tok, heads, d)
    g0 = _grids(grid, b)[0]  # the frame length of sample 0, as causal_model.py:269 takes it
    frame_seqlen = g0[1] * g0[2]
    start_frame = current_start // frame_seqlen
    roped_q = causal_rope(q, grid, freqs, start_frame).type_as(v)
    roped_k = causal_rope(k, grid, freqs, start_frame).type_as(v)
    n = roped_q.shape[1]
    current_end = current_start + n
    sink = sink_size * frame_seqlen
    cap = kv_cache["k"].shape[1]
    global_end = int(kv_cache["global_end_index"].item())
    local_end = int(kv_cache["local_end_index"].item())
    coarse = proj is not None and "k_coarse" in kv_cache and "v_coarse" in kv_cache
    if coarse:
        k_proj, v_proj, seg, bsz = proj
        rank = k_proj.shape[0]

    def to_coarse(a: int, b: int):
        return OH.token_range_to_coarse(a, b, seg, rank)

    tk, tv = kv_cache["k"].clone(), kv_cache["v"].clone()
    tkc = kv_cache["k_coarse"].clone() if coarse else None
    tvc = kv_cache["v_coarse"].clone() if coarse else None
    recompute = current_end <= global_end and current_start > 0
    rolled = evicted = 0
    roll = local_attn_size != -1 and current_end > global_end and n + local_end > cap
    if roll:
        evicted = n + local_end - cap
        rolled = local_end - evicted - sink
        tk[:, sink:sink + rolled] = tk[:, sink + evicted:sink + evicted + rolled].clone()
        tv[:, sink:sink + rolled] = tv[:, sink + evicted:sink + evicted + rolled].clone()
        if coarse:
            _, c_sink = to_coarse(0, sink)
            c0, c1 = to_coarse(sink + evicted, sink + evicted + rolled)
            if c1 > c0:
                tkc[:, c_sink:c_sink + c1 - c0] = tkc[:, c0:c1].clone()
                tvc[:, c_sink:c_sink + c1 - c0] = tvc[:, c0:c1].clone()
        new_local_end = local_end + current_end - global_end - evicted
    else:
        new_local_end = local_end + current_end - global_end
    local_start = new_local_end - n
    write_start = max(local_start, sink) if recompute else local_start
    if not roll and sink_recache_after_switch:
        write_start = local_start
    offset = max(0, write_start - local_start)
    write_len = max(0, new_local_end - write_start)
    new_k = roped_k[:, offset:offset + write_len]
    new_v = v[:, offset:offset + write_len]
    if write_len > 0:
        tk[:, write_start:new_local_end] = new_k
        tv[:, write_start:new_local_end] = new_v
        if coarse:
            c0, c1 = to_coarse(write_start, new_local_end)
            kc_new, vc_new = OH.compress_kv(new_k.transpose(1, 2), new_v.transpose(1, 2), segment_len=seg,
                                            k_proj_mat=k_proj, v_proj_mat=v_proj, block_size=bsz)
            tkc[:, c0:c1] = kc_new.transpose(1, 2)
            tvc[:, c0:c1] = vc_new.transpose(1, 2)

    # the attention window (run_hsa_core_attn)
    def coarse_slice(a, b):
        if not coarse:
            return None, None
        c0, c1 = to_coarse(a, b)
        return tkc[:, c0:c1], tvc[:, c0:c1]

    if sink > 0:
        budget = max_attention_size - sink
        ks, vs = tk[:, :sink], tv[:, :sink]
        kcs, vcs = coarse_slice(0, sink)
        if budget > 0:
            lsw = max(sink, new_local_end - budget)
            attn_k = torch.cat([ks, tk[:, lsw:new_local_end]], dim=1)
            attn_v = torch.cat([vs, tv[:, lsw:new_local_end]], dim=1)
            kcl, vcl = coarse_slice(lsw, new_local_end)
            attn_kc = torch.cat([kcs, kcl], dim=1) if coarse else None
            attn_vc = torch.cat([vcs, vcl], dim=1) if coarse else None
        else:
            attn_k, attn_v, attn_kc, attn_vc = ks, vs, kcs, vcs
    else:
        ws = max(0, new_local_end - max_attention_size)
        attn_k, attn_v = tk[:, ws:new_local_end], tv[:, ws:new_local_end]
        attn_kc, attn_vc = coarse_slice(ws, new_local_end)

    # the commit: the clones become the cache; the indices move unless this was a recompute
    kv_cache["k"].copy_(tk)
    kv_cache["v"].copy_(tv)
    if coarse:
        kv_cache["k_coarse"].copy_(tkc)
        kv_cache["v_coarse"].copy_(tvc)
    if not recompute:
        kv_cache["global_end_index"].fill_(current_end)
        kv_cache["local_end_index"].fill_(new_local_end)
    info = {"action": "roll_and_insert" if roll else "direct_insert", "num_evicted_tokens": evicted,
            "num_rolled_tokens": rolled, "sink_tokens": sink, "local_start_index": local_start,
            "local_end_index": new_local_end, "write_start_index": write_start, "write_end_index": new_local_end,
            "current_end": current_end, "is_recompute": recompute}
    return roped_q, attn_k, attn_v, attn_kc, attn_vc, info


def segment_rank(segment_len: int, block_size: int) -> int:
    return math.ceil(segment_len / block_size)
