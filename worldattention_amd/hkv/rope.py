"""Temporal rotary re-rotation of KV pages on the GPU, with the reference's signatures.

Mirrors ``pipeline/hkv/rope.py``: ``temporal_complex_dims`` (:22-25), ``temporal_band`` (:28-30),
``shift_temporal_rope`` (:50-67) and ``derope_temporal`` (:70-82). The rotation factor
``freqs[new] * conj(freqs[orig])`` is formed exactly as the reference forms it (in the table's
precision, then complex64); the per-token complex multiply runs in ``wa_rerope`` in fp32 and the
result is rounded to the key dtype, as the reference's ``_apply_factor`` does (:33-40).
"""
from __future__ import annotations

import torch

from ._ops import factor_table, rotate_temporal

__all__ = ["temporal_complex_dims", "temporal_band", "shift_temporal_rope", "derope_temporal"]


def temporal_complex_dims(head_dim: int) -> int:
    """Complex pairs in the temporal band of a ``head_dim`` rotary embedding (``rope.py:22-25``)."""
    half = head_dim // 2
    return half - 2 * (half // 3)


def temporal_band(freqs: torch.Tensor, head_dim: int) -> torch.Tensor:
    """The temporal columns of a ``[max_positions, head_dim // 2]`` table (``rope.py:28-30``)."""
    return freqs[:, : temporal_complex_dims(head_dim)]


def _check_band(k: torch.Tensor, temporal_freqs: torch.Tensor) -> int:
    nt = temporal_complex_dims(k.shape[-1])
    if temporal_freqs.dim() != 2 or temporal_freqs.shape[1] < nt:
        raise ValueError(f"temporal_freqs must be [positions, >= {nt}] for head_dim {k.shape[-1]}, "
                         f"got {tuple(temporal_freqs.shape)}")
    return nt


def shift_temporal_rope(k: torch.Tensor, temporal_freqs: torch.Tensor, new_frame0: int,
                        orig_frame0: int) -> torch.Tensor:
    """Move a page of keys ``[..., tokens, H, head_dim]`` from ``orig_frame0`` to ``new_frame0``
    (one factor for the whole page; positions clamped to the table). Returns a new tensor."""
    nt = _check_band(k, temporal_freqs)
    ids = torch.tensor([int(new_frame0)]), torch.tensor([int(orig_frame0)])
    factors = factor_table(temporal_freqs[:, :nt], ids[0], ids[1], k.device)
    out = torch.empty_like(k, memory_format=torch.contiguous_format)
    src = k if k.stride(-1) == 1 else k.contiguous()
    return rotate_temporal(src, factors, dst=out)


def derope_temporal(k: torch.Tensor, temporal_freqs: torch.Tensor, frame_ids: torch.Tensor) -> torch.Tensor:
    """Remove each token's temporal rotation from ``k`` ``[B, tokens, H, head_dim]``;
    ``frame_ids`` ``[tokens]`` is each token's absolute frame. Returns a new tensor."""
    nt = _check_band(k, temporal_freqs)
    if frame_ids.dim() != 1 or frame_ids.shape[0] != k.shape[-3]:
        raise ValueError("frame_ids must hold one frame per token")
    frames, rows = torch.unique(frame_ids.to(k.device), return_inverse=True)
    factors = factor_table(temporal_freqs[:, :nt], torch.zeros_like(frames), frames, k.device)
    out = torch.empty_like(k, memory_format=torch.contiguous_format)
    src = k if k.stride(-1) == 1 else k.contiguous()
    return rotate_temporal(src, factors, dst=out, rows=rows.to(torch.int32))
