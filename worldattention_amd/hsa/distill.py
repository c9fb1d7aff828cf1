"""Per-layer self-distillation of HSA towards dense attention (``wan/modules/hsa/distill.py:22-71``).

While collection is switched on, each HSA forward that runs under autograd adds one scalar,
``MSE(hsa_out, dense_out)`` with the dense output detached, to a process-wide list; the trainer
takes the list, sums it and backpropagates into the gate and the low-rank projections
(``trainer/hsa_stage.py:149-165``). Switching collection off empties the list.

The dense teacher is this library's flash kernel (``wa_bsa_fwd`` over every key block, bf16
operands, fp32 softmax and accumulation), not torch SDPA: it reads ``[B, L, H, D]`` q/k/v in place
and never materialises the ``L x L`` scores.
"""
from __future__ import annotations

from typing import List

import torch
import torch.nn.functional as F

from .. import _lib
from .block_sparse import bsa_forward, padded_head_dim

__all__ = ["enable_distill", "distill_enabled", "pop_distill_losses", "record_distill_loss",
           "dense_attention", "record_against_dense"]


class _Collector:
    """The on/off switch and the losses gathered since the trainer last took them."""

    def __init__(self) -> None:
        self.on = False
        self.items: List[torch.Tensor] = []

    def switch(self, on: bool) -> None:
        self.on = bool(on)
        if not self.on:
            self.items = []

    def take(self) -> List[torch.Tensor]:
        got, self.items = self.items, []
        return got


_COLLECTOR = _Collector()


def enable_distill(flag: bool = True) -> None:
    """Switch collection on (``True``) or off (``False``, which also drops what was gathered)."""
    _COLLECTOR.switch(flag)


def distill_enabled() -> bool:
    return _COLLECTOR.on


def pop_distill_losses() -> List[torch.Tensor]:
    """The losses gathered since the previous call; the registry is left empty."""
    return _COLLECTOR.take()


def record_distill_loss(loss: torch.Tensor) -> None:
    _COLLECTOR.items.append(loss)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Softmax attention of ``[B, Lq, H, D]`` queries over all ``[B, Lkv, H, D]`` keys, scale
    ``D ** -0.5``, no mask: the target HSA is distilled towards. Runs the dense flash kernel on
    bf16 copies of the operands (head dims other than 64 and 128 zero-padded to the next one, with
    the original scale); the result has ``q``'s dtype."""
    d = q.shape[-1]
    dp = padded_head_dim(d)
    if k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)} and v {tuple(v.shape)} do not match")
    block = 128 if dp == 128 else 64
    qb, kb, vb = (_lib.kernel_ready(F.pad(t.detach(), (0, dp - d)) if dp != d else t.detach()) for t in (q, k, v))
    out, _ = bsa_forward(qb, kb, vb, index=None, num=None, block_size=block, layout="blhd",
                         out_dtype=q.dtype if q.dtype in (torch.float32, torch.bfloat16) else torch.float32,
                         scale=d ** -0.5 if dp != d else 0.0)
    out = out[..., :d].contiguous() if dp != d else out
    return out if out.dtype == q.dtype else out.to(q.dtype)


def record_against_dense(hsa_out: torch.Tensor, q, k, v) -> None:
    """Gather ``MSE(hsa_out, dense_attention(q, k, v))``; gradients reach ``hsa_out`` only."""
    with torch.no_grad():
        teacher = dense_attention(q, k, v).to(hsa_out.dtype).float()
    record_distill_loss(F.mse_loss(hsa_out.float(), teacher))
