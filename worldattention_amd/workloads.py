"""Seeded synthetic inputs at the benchmark shapes (no datasets or checkpoints are needed).

* ``cfg1`` — tests-scale plumbing: B=1, H=2, D=64, Lq=256, Lkv=1024, block 64, fp32; head 0 sparse
  top-4, head 1 elu(x)+1 linear. Q/K/V ~ N(0,1)/8; K gets one N(0, 0.5^2) offset vector per
  256-token frame and head, so routing is non-trivial.
* ``cfg2`` — Wan-1.3B chunk: B=1, H=12, D=128, bf16, Lq = 3 frames x 1560 (frames 18-20 of a
  30x52 latent grid), Lkv = 21 frames x 1560, block 128. Q/K/V ~ N(0,1); K gets one N(0, 0.5^2)
  offset per frame and head; Wan 3-D RoPE (temporal 22 / height 21 / width 21 complex pairs) is
  applied to Q and K at their frame positions. 8 sparse heads with budgets drawn from {8,16,32}
  and 4 linear heads, both chosen by the seed.
* ``cfg5`` — cfg2 shapes with top-k 16 on every sparse head, plus dO ~ N(0,1), for fwd+bwd.

The 3-D RoPE follows ``wan/modules/model.py:29-36`` and ``wan/modules/causal_model.py:34-62``.
"""
from __future__ import annotations

import math

import torch

FRAME_H, FRAME_W = 30, 52
FRAME_TOKENS = FRAME_H * FRAME_W  # 1560


def rope_freqs(max_positions: int, head_dim: int, theta: float = 10000.0) -> torch.Tensor:
    """``[max_positions, D/2]`` complex128 table: temporal | height | width bands."""
    def params(dim):
        inv = 1.0 / torch.pow(theta, torch.arange(0, dim, 2).to(torch.float64).div(dim))
        ang = torch.outer(torch.arange(max_positions), inv)
        return torch.polar(torch.ones_like(ang), ang)
    d = head_dim
    return torch.cat([params(d - 4 * (d // 6)), params(2 * (d // 6)), params(2 * (d // 6))], dim=1)


def apply_rope_3d(x: torch.Tensor, freqs: torch.Tensor, frames: int, height: int, width: int,
                  start_frame: int) -> torch.Tensor:
    """Rotate ``[B, F*H*W, heads, D]`` by the 3-D RoPE of frames ``start_frame ..`` (fp64 math)."""
    b, length, heads, d = x.shape
    c = d // 2
    ft, fh, fw = freqs.split([c - 2 * (c // 3), c // 3, c // 3], dim=1)
    per_pos = torch.cat([
        ft[start_frame:start_frame + frames].view(frames, 1, 1, -1).expand(frames, height, width, -1),
        fh[:height].view(1, height, 1, -1).expand(frames, height, width, -1),
        fw[:width].view(1, 1, width, -1).expand(frames, height, width, -1),
    ], dim=-1).reshape(length, 1, -1).to(x.device)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(b, length, heads, -1, 2))
    return torch.view_as_real(xc * per_pos).flatten(3).to(x.dtype)


def _frame_offsets(g, frames, heads, d, frame_tokens, sigma):
    off = torch.randn(1, frames, heads, d, generator=g) * sigma
    return off.repeat_interleave(frame_tokens, dim=1)


def cfg1(device="cpu", seed: int = 0) -> dict:
    g = torch.Generator().manual_seed(seed)
    h, d, lq, lkv = 2, 64, 256, 1024
    q = torch.randn(1, lq, h, d, generator=g) / math.sqrt(d)
    k = torch.randn(1, lkv, h, d, generator=g) / math.sqrt(d)
    v = torch.randn(1, lkv, h, d, generator=g) / math.sqrt(d)
    k = k + _frame_offsets(g, lkv // 256, h, d, 256, 0.5)
    return dict(q=q.to(device), k=k.to(device), v=v.to(device), block_size=64, routing="topk", topk=[4, 0],
                head_modes=["sparse", "linear"], linear_mode="elu1", proj_segment_len=256)


def _wan_chunk(seed: int, heads: int = 12, d: int = 128, q_frames: int = 3, kv_frames: int = 21,
               dtype=torch.bfloat16, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    lq, lkv = q_frames * FRAME_TOKENS, kv_frames * FRAME_TOKENS
    q = torch.randn(1, lq, heads, d, generator=g)
    k = torch.randn(1, lkv, heads, d, generator=g) + _frame_offsets(g, kv_frames, heads, d, FRAME_TOKENS, 0.5)
    v = torch.randn(1, lkv, heads, d, generator=g)
    freqs = rope_freqs(1024, d)
    q = apply_rope_3d(q, freqs, q_frames, FRAME_H, FRAME_W, start_frame=kv_frames - q_frames)
    k = apply_rope_3d(k, freqs, kv_frames, FRAME_H, FRAME_W, start_frame=0)
    return g, q.to(device=device, dtype=dtype), k.to(device=device, dtype=dtype), v.to(device=device, dtype=dtype)


def head_split(g: torch.Generator, heads: int, n_linear: int):
    """Pick ``n_linear`` linear heads with the seed; the rest are sparse."""
    linear = sorted(torch.randperm(heads, generator=g)[:n_linear].tolist())
    return ["linear" if h in linear else "sparse" for h in range(heads)]


def cfg2(device="cpu", seed: int = 0, dtype=torch.bfloat16) -> dict:
    g, q, k, v = _wan_chunk(seed, dtype=dtype, device=device)
    modes = head_split(g, 12, 4)
    choices = torch.tensor([8, 16, 32])
    ks = [int(choices[torch.randint(0, 3, (1,), generator=g)]) if m == "sparse" else 0 for m in modes]
    return dict(q=q, k=k, v=v, block_size=128, routing="topk", topk=ks, head_modes=modes, linear_mode="elu1",
                proj_segment_len=FRAME_TOKENS)


def cfg5(device="cpu", seed: int = 0, dtype=torch.bfloat16) -> dict:
    g, q, k, v = _wan_chunk(seed, dtype=dtype, device=device)
    modes = head_split(g, 12, 4)
    ks = [16 if m == "sparse" else 0 for m in modes]
    do = torch.randn(q.shape, generator=g).to(device=device, dtype=dtype)
    return dict(q=q, k=k, v=v, do=do, block_size=128, routing="topk", topk=ks, head_modes=modes,
                linear_mode="elu1", proj_segment_len=FRAME_TOKENS)


def sparse_flops(num: torch.Tensor, index: torch.Tensor, q_len: int, kv_len: int, block_size: int, d: int,
                 heads=None) -> tuple[float, float]:
    """(useful, tile) forward FLOP of the sparse branch for a routing.

    useful = 4 D sum_rows q_real(i) sum_{j in list} kv_real(j); tile = 4 D Bs^2 sum num.
    """
    num = num.detach().cpu().long()
    index = index.detach().cpu().long()
    bsz, nh, nq = num.shape
    nkv = -(-kv_len // block_size)
    kv_real = torch.full((nkv,), block_size, dtype=torch.long)
    kv_real[-1] = kv_len - (nkv - 1) * block_size
    q_real = torch.full((nq,), block_size, dtype=torch.long)
    q_real[-1] = q_len - (nq - 1) * block_size
    hs = range(nh) if heads is None else heads
    useful, tiles = 0, 0
    for b in range(bsz):
        for h in hs:
            for i in range(nq):
                n = int(num[b, h, i])
                if n <= 0:
                    continue
                ids = index[b, h, i, :n].clamp(0, nkv - 1)
                useful += int(q_real[i]) * int(kv_real[ids].sum())
                tiles += n
    return 4.0 * d * useful, 4.0 * d * block_size * block_size * tiles
