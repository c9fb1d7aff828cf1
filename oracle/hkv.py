"""CPU oracle for the Hierarchical KV cache (HKV) — test infrastructure only.

Restates ``pipeline/hkv/rope.py``, ``pipeline/hkv/retrieval.py`` and the page bookkeeping of
``pipeline/hkv/cache.py`` / ``pipeline/hkv/tiering.py`` on CPU tensors. Top-k selections use a
stable descending sort, i.e. the lowest candidate index wins a tie (the reference's
``torch.topk`` leaves tie order to the implementation; on tie-free scores both agree).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------------------------
# Temporal rotary bands (rope.py:22-82)
# ----------------------------------------------------------------------------------------------
def temporal_complex_dims(head_dim: int) -> int:
    """Complex pairs in the temporal band: ``half - 2*(half//3)``. Follows ``rope.py:22-25``.

    pinned by: the RoPE split of ``wan/modules/model.py:29-36`` (22 of 64 pairs at D=128).
    """
    half = head_dim // 2
    return half - 2 * (half // 3)


def temporal_band(freqs: torch.Tensor, head_dim: int) -> torch.Tensor:
    """First ``temporal_complex_dims`` columns of a ``[positions, D/2]`` table. ``rope.py:28-30``."""
    return freqs[:, : temporal_complex_dims(head_dim)]


def rope_freqs(max_positions: int, head_dim: int, theta: float = 10000.0) -> torch.Tensor:
    """Wan 3-D RoPE table ``[max_positions, D/2]`` complex128 (temporal | height | width bands).

    Follows ``wan/modules/model.py:29-36`` and ``wan/modules/causal_model.py:806-811``.
    """
    def params(dim):
        inv = 1.0 / torch.pow(theta, torch.arange(0, dim, 2).to(torch.float64).div(dim))
        ang = torch.outer(torch.arange(max_positions), inv)
        return torch.polar(torch.ones_like(ang), ang)
    d = head_dim
    return torch.cat([params(d - 4 * (d // 6)), params(2 * (d // 6)), params(2 * (d // 6))], dim=1)


def rope_apply_3d(x: torch.Tensor, freqs: torch.Tensor, frames: int, height: int, width: int,
                  start_frame: int = 0) -> torch.Tensor:
    """3-D RoPE of ``[B, F*H*W, heads, D]`` at frames ``start_frame..``. ``causal_model.py:34-62``."""
    b, length, heads, d = x.shape
    c = d // 2
    ft, fh, fw = freqs.split([c - 2 * (c // 3), c // 3, c // 3], dim=1)
    per_pos = torch.cat([
        ft[start_frame:start_frame + frames].view(frames, 1, 1, -1).expand(frames, height, width, -1),
        fh[:height].view(1, height, 1, -1).expand(frames, height, width, -1),
        fw[:width].view(1, 1, width, -1).expand(frames, height, width, -1),
    ], dim=-1).reshape(length, 1, -1)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(b, length, heads, -1, 2))
    return torch.view_as_real(xc * per_pos).flatten(3).to(x.dtype)


def _apply_factor(k: torch.Tensor, factor: torch.Tensor, num_temporal: int) -> torch.Tensor:
    shape = k.shape
    ck = torch.view_as_complex(k.to(torch.float32).contiguous().reshape(*shape[:-1], shape[-1] // 2, 2)).clone()
    ck[..., :num_temporal] = ck[..., :num_temporal] * factor.to(torch.complex64)
    return torch.view_as_real(ck).reshape(shape).to(k.dtype)


def _factor(freqs: torch.Tensor, new_ids: torch.Tensor, orig_ids: torch.Tensor) -> torch.Tensor:
    top = freqs.shape[0] - 1
    return freqs[new_ids.clamp(0, top)] * freqs[orig_ids.clamp(0, top)].conj()


def shift_temporal_rope(k, temporal_freqs, new_frame0: int, orig_frame0: int):
    """Rotate a page's temporal band from ``orig_frame0`` to ``new_frame0``. ``rope.py:50-67``.

    pinned by: shift == re-encode at the new frame against a full 3-band RoPE, shift-by-0,
    invertibility, clamping (reference ``tests/test_hkv_rope.py:65-120``).
    """
    nt = temporal_complex_dims(k.shape[-1])
    f = _factor(temporal_freqs, torch.as_tensor(int(new_frame0)), torch.as_tensor(int(orig_frame0)))
    return _apply_factor(k, f, nt)


def derope_temporal(k, temporal_freqs, frame_ids):
    """Remove each token's temporal rotation, ``[B, T, H, D]``. ``rope.py:70-82``.

    pinned by: de-rope == spatial-only encoding, position independence
    (reference ``tests/test_hkv_rope.py:91-114``).
    """
    nt = temporal_complex_dims(k.shape[-1])
    f = _factor(temporal_freqs, torch.zeros_like(frame_ids), frame_ids)
    f = f.view(*([1] * (k.dim() - 3)), frame_ids.shape[0], 1, nt)
    return _apply_factor(k, f, nt)


# ----------------------------------------------------------------------------------------------
# Retrieval (retrieval.py:32-126)
# ----------------------------------------------------------------------------------------------
def prompt_index(prompt_embeds: torch.Tensor) -> torch.Tensor:
    """Unit mean prompt vector. ``retrieval.py:32-38``. pinned by: unit norm, order invariance."""
    return F.normalize(prompt_embeds.float().mean(dim=1).mean(dim=0), dim=0)


def query_index(q_tokens: torch.Tensor) -> torch.Tensor:
    """Mean of pre-RoPE queries ``[B, T, H*D] -> [H*D]``. ``retrieval.py:41-47``."""
    return q_tokens.float().mean(dim=1).mean(dim=0)


def page_key_index(keys, page_spans, *, frame_seq_length, start_frame, temporal_freqs):
    """De-roped mean key per page, ``[P, H*D]`` fp32 (None without pages). ``retrieval.py:50-72``.

    pinned by: start-frame invariance (reference ``tests/test_hkv_retrieval.py:101-137``) and a
    per-page fp64 mean in tests/test_oracle_hkv.py.
    """
    if not page_spans:
        return None
    frame_ids = start_frame + torch.arange(keys.shape[1]) // frame_seq_length
    content = derope_temporal(keys, temporal_freqs, frame_ids).flatten(2).float()
    return torch.stack([content[:, s:e].mean(dim=1).mean(dim=0) for s, e in page_spans], dim=0)


def score_pages(query_vec, page_index, scale: Optional[float] = None):
    """``page_index @ q / sqrt(dim)``. ``retrieval.py:75-89``. pinned by: ``:58-63`` closed form."""
    if page_index.numel() == 0:
        return page_index.new_zeros((0,))
    scores = page_index @ query_vec.to(page_index.dtype).reshape(-1)
    if scale is None:
        scale = float(page_index.shape[-1]) ** 0.5
    if scale and scale > 0:
        scores = scores / scale
    return scores


def stable_topk(scores: torch.Tensor, k: int) -> List[int]:
    """Indices of the ``k`` largest scores, highest first, lowest index first among ties."""
    k = min(int(k), scores.shape[0])
    if k <= 0:
        return []
    _, order = torch.sort(scores, descending=True, stable=True)
    return [int(i) for i in order[:k].tolist()]


def select_top_chunks(query_vec, chunk_index, topk: int) -> List[int]:
    """Stage 1 cosine ranking. ``retrieval.py:92-102``. pinned by: ``:40-55``."""
    if chunk_index.numel() == 0 or topk <= 0:
        return []
    return stable_topk(chunk_index @ query_vec.to(chunk_index.dtype).reshape(-1), topk)


def select_topk_pages(query_vec, candidates, topk: int, scale=None):
    """Stage 2 global top-k over pooled candidates. ``retrieval.py:105-126``. pinned by: ``:66-98``."""
    if topk <= 0 or not candidates:
        return []
    index = torch.stack([c[2].reshape(-1).float() for c in candidates], dim=0)
    scores = score_pages(query_vec.float(), index, scale=scale)
    return [(int(candidates[i][0]), int(candidates[i][1]), float(scores[i])) for i in stable_topk(scores, topk)]


# ----------------------------------------------------------------------------------------------
# Page bookkeeping (cache.py:87-299)
# ----------------------------------------------------------------------------------------------
def page_spans(valid_tokens: int, page_tokens: int) -> List[Tuple[int, int]]:
    """Pages of ``page_tokens`` with a partial last page. ``cache.py:109-112``."""
    return [(s, min(s + page_tokens, valid_tokens)) for s in range(0, valid_tokens, page_tokens)]


def chronological(selected, chunk_start_frames, chunk_spans):
    """Sort ``(chunk, page)`` by (chunk start frame, page start). ``cache.py:172-178``."""
    return sorted(selected, key=lambda p: (chunk_start_frames[p[0]], chunk_spans[p[0]][p[1]][0]))


def install_plan(entries, capacity: int, current_start_frame: int, frame_seq_length: int,
                 chunk_start_frames):
    """Truncate to capacity and plan the re-rope frame moves. ``cache.py:203-213, 273-286``.

    ``entries`` are ``(chunk, start, end)`` token spans in install order. Returns the installed
    spans and, per span, ``(orig_frame, new_frame)``.
    """
    budget, installed = capacity, []
    for chunk, s, e in entries:
        if budget <= 0:
            break
        take = min(e - s, budget)
        installed.append((chunk, s, s + take))
        budget -= take
    total = sum(e - s for _, s, e in installed)
    base = current_start_frame - total // frame_seq_length
    moves, offset = [], 0
    for chunk, s, e in installed:
        moves.append((chunk_start_frames[chunk] + s // frame_seq_length, base + offset // frame_seq_length))
        offset += e - s
    return installed, moves
