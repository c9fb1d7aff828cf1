"""Two-stage HKV retrieval on the GPU, with the reference's signatures.

Mirrors ``pipeline/hkv/retrieval.py``: ``prompt_index`` (:32-38), ``query_index`` (:41-47),
``page_key_index`` (:50-72), ``score_pages`` (:75-89), ``select_top_chunks`` (:92-102) and
``select_topk_pages`` (:105-126). Means and de-rotation run in ``wa_hkv_page_summary`` (one pass
over the keys, de-roped values rounded to the key dtype before pooling, as the reference's
``derope_temporal`` returns the key dtype); scores and the top-k run in ``wa_hkv_score_topk``.
The reference ranks with ``torch.topk``, whose order among equal scores is unspecified; here the
lower index wins a tie, which agrees with it whenever scores are distinct.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch

from .. import _lib
from ._ops import factor_table, score_topk, segment_means
from .rope import temporal_complex_dims

__all__ = [
    "prompt_index",
    "query_index",
    "page_key_index",
    "score_pages",
    "select_top_chunks",
    "select_topk_pages",
    "select_pages",
]


def prompt_index(prompt_embeds: torch.Tensor) -> torch.Tensor:
    """Unit-norm mean of ``[B, tokens, dim]`` prompt embeddings -> ``[dim]`` fp32."""
    if prompt_embeds.dim() != 3:
        raise ValueError(f"prompt_embeds must be [B, tokens, dim], got {tuple(prompt_embeds.shape)}")
    dim = prompt_embeds.shape[-1]
    return segment_means(prompt_embeds, heads=1, head_dim=dim, normalize=True)[0]


def query_index(q_tokens: torch.Tensor) -> torch.Tensor:
    """Mean of pre-rotation queries ``[B, tokens, H * D]`` over batch and tokens -> ``[H * D]``."""
    if q_tokens.dim() != 3:
        raise ValueError(f"q_tokens must be [B, tokens, H*D], got {tuple(q_tokens.shape)}")
    return segment_means(q_tokens, heads=1, head_dim=q_tokens.shape[-1])[0]


def _regular_page_tokens(page_spans: Sequence[Tuple[int, int]], num_tokens: int) -> Optional[int]:
    """The page size when the spans are consecutive pages of one size (last one possibly short)."""
    size = int(page_spans[0][1]) - int(page_spans[0][0])
    if size <= 0:
        return None
    for i, (s, e) in enumerate(page_spans):
        if int(s) != i * size or int(e) != min((i + 1) * size, num_tokens):
            return None
    return size if int(page_spans[-1][1]) == num_tokens else None


def page_key_index(keys: torch.Tensor, page_spans: Sequence[Tuple[int, int]], *, frame_seq_length: int,
                   start_frame: int, temporal_freqs: torch.Tensor) -> Optional[torch.Tensor]:
    """De-rotated mean key per page: ``keys`` ``[B, tokens, H, D]`` (rotated, as cached) ->
    ``[num_pages, H * D]`` fp32, or None without pages. Token t sits at frame
    ``start_frame + t // frame_seq_length``."""
    if not page_spans:
        return None
    if keys.dim() != 4:
        raise ValueError(f"keys must be [B, tokens, H, D], got {tuple(keys.shape)}")
    bsz, ntok, heads, hd = keys.shape
    nt = temporal_complex_dims(hd)
    n_frames = max(-(-ntok // int(frame_seq_length)), 1)
    frames = int(start_frame) + torch.arange(n_frames)
    factors = factor_table(temporal_freqs[:, :nt], torch.zeros_like(frames), frames, keys.device)
    if keys.stride(-1) != 1 or keys.stride(2) != hd or keys.stride(1) != heads * hd:
        keys = keys.contiguous()
    flat = keys.view(bsz, ntok, heads * hd) if keys.is_contiguous() else keys.reshape(bsz, ntok, heads * hd)
    size = _regular_page_tokens(page_spans, ntok)
    if size is not None:
        return segment_means(flat, heads=heads, head_dim=hd, seg_tokens=size, factors=factors,
                             row_tokens=int(frame_seq_length))
    return segment_means(flat, heads=heads, head_dim=hd, spans=list(page_spans), factors=factors,
                         row_tokens=int(frame_seq_length))


def _scale_of(dim: int, scale: Optional[float]) -> float:
    if scale is None:
        scale = float(dim) ** 0.5
    return float(scale) if scale and scale > 0 else 0.0


def score_pages(query_vec: torch.Tensor, page_index: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
    """Affinity ``page_index @ query / scale`` per page (``scale`` defaults to sqrt(dim); no
    division when it is 0 or negative) -> ``[P]`` fp32."""
    if page_index.numel() == 0:
        return page_index.new_zeros((0,))
    _lib.require_gpu(page_index)
    _, _, scores = score_topk(page_index, query_vec, 1, scale=_scale_of(page_index.shape[-1], scale),
                              want_scores=True)
    return scores


def select_pages(page_index: torch.Tensor, query_vec: torch.Tensor, topk: int, *, scale: Optional[float] = None,
                 mask: Optional[torch.Tensor] = None):
    """Device-side selection: ``(sel int32 [k], scores fp32 [k])`` of the ``topk`` best pages
    (``k = min(topk, P)``), pages with ``mask != 0`` skipped (their slots then hold -1)."""
    k = min(int(topk), page_index.shape[0])
    sel, sel_scores, _ = score_topk(page_index, query_vec, k, scale=_scale_of(page_index.shape[-1], scale),
                                    mask=mask)
    return sel, sel_scores


def select_top_chunks(query_vec: torch.Tensor, chunk_index: torch.Tensor, topk: int) -> List[int]:
    """Stage 1: ids of the ``topk`` chunks whose unit prompt index is most cosine-similar."""
    if chunk_index.numel() == 0 or topk <= 0:
        return []
    sel, _ = select_pages(chunk_index, query_vec, topk, scale=0.0)
    return [int(i) for i in sel.tolist()]


def select_topk_pages(query_vec: torch.Tensor, candidates: Sequence[Tuple[int, int, torch.Tensor]], topk: int,
                      scale: Optional[float] = None) -> List[Tuple[int, int, float]]:
    """Stage 2: global top-``topk`` of ``(chunk_id, page_id, page_vector)`` candidates ->
    ``(chunk_id, page_id, score)`` highest first."""
    if topk <= 0 or len(candidates) == 0:
        return []
    index = torch.stack([c[2].reshape(-1).float() for c in candidates], dim=0)
    sel, sel_scores = select_pages(index, query_vec, topk, scale=scale)
    return [(int(candidates[i][0]), int(candidates[i][1]), float(s))
            for i, s in zip(sel.tolist(), sel_scores.tolist())]
