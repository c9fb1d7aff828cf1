"""HSA parameter initialization (``trainer/hsa_stage.py:43-82``).

Only the initializer is on the attention path; the trainer knobs of the reference module are out of
scope.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .hsa.attention import HSAAttention

__all__ = ["init_hsa_parameters"]


def init_hsa_parameters(model: nn.Module) -> int:
    """Give every :class:`HSAAttention` in ``model`` its block-pooling initialization.

    Row ``r`` of each projection averages tokens ``[r*block, min((r+1)*block, seg))``; the fusion
    gate starts at zero weight and bias (an even 0.5 mix). Returns the number of modules touched.
    """
    modules = [m for m in model.modules() if isinstance(m, HSAAttention)]
    for module in modules:
        with torch.no_grad():
            for projection in (module.k_proj_mat, module.v_proj_mat):
                rank, seg_len = projection.shape
                rows = torch.zeros((rank, seg_len), dtype=torch.float32)
                for row in range(rank):
                    start = row * module.block_size
                    end = min((row + 1) * module.block_size, seg_len)
                    if end > start:
                        rows[row, start:end] = 1.0 / float(end - start)
                projection.copy_(rows.to(projection.dtype))
            module.gate_lin.weight.zero_()
            module.gate_lin.bias.zero_()
    return len(modules)
