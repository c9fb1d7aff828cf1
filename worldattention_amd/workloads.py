"""Seeded synthetic inputs at the benchmark shapes (no datasets or checkpoints are needed).

* ``cfg1`` — tests-scale plumbing: B=1, H=2, D=64, Lq=256, Lkv=1024, block 64, fp32; head 0 sparse
  top-4, head 1 elu(x)+1 linear. Q/K/V ~ N(0,1)/8; K gets one N(0, 0.5^2) offset vector per
  256-token frame and head, so routing is non-trivial.
* ``cfg2`` — Wan-1.3B chunk: B=1, H=12, D=128, bf16, Lq = 3 frames x 1560 (frames 18-20 of a
  30x52 latent grid), Lkv = 21 frames x 1560, block 128. Q/K/V ~ N(0,1); K gets one N(0, 0.5^2)
  offset per frame and head; Wan 3-D RoPE (temporal 22 / height 21 / width 21 complex pairs) is
  applied to Q and K at their frame positions. 8 sparse heads with budgets drawn from {8,16,32}
  and 4 linear heads, both chosen by the seed.
* ``cfg3`` — HKV long-horizon retrieval at the Wan-1.3B shape: a 120-frame history (187,200
  tokens, H=12, D=128, bf16) per layer, one-frame pages. Frames 0..113 of every layer sit in a
  pinned host pool, frames 114..119 stay resident in the device pool; the query chunk (frames
  120..122) mixes the key clusters of 8 seeded host frames, so retrieval has a ground truth.
* ``cfg4`` — Wan-14B attention stack: H=40, D=128, model dim 5120, 40 layers with seeded
  ``Linear(5120, 3*5120)`` QKV / ``Linear(5120, 5120)`` out weights, a 28,080-token synthetic KV
  history per layer plus the chunk's own 4,680 tokens, 30 sparse (top-16) / 10 linear heads.
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


def cfg2_reference_mode(device="cpu", seed: int = 0, dtype=torch.bfloat16) -> dict:
    """The reference's own default HSA configuration on the cfg 2 chunk: the DiT's
    ``HSAAttention(block_size=64, tau_min=0.35, tau_max=1.0, proj_segment_len=1560)``
    (``wan/modules/causal_model.py:100-107``), i.e. Gini routing, the low-rank linear branch and
    both branches on every head. Projections from the block-averaging initializer
    (``trainer/hsa_stage.py:43-82``) and a seeded, trained-looking fusion gate. Returns the inputs
    and the module (on ``device``, in ``dtype``)."""
    from .hsa.attention import HSAAttention
    from .hsa_stage import init_hsa_parameters

    _, q, k, v = _wan_chunk(seed, dtype=dtype, device=device)
    heads, d = q.shape[2], q.shape[3]
    module = HSAAttention(num_heads=heads, head_dim=d, block_size=64, tau_min=0.35, tau_max=1.0,
                          proj_segment_len=FRAME_TOKENS)
    init_hsa_parameters(module)
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        module.gate_lin.weight.copy_(torch.randn(d, d, generator=gen) * 0.05)
        module.gate_lin.bias.copy_(torch.randn(d, generator=gen) * 0.05)
    return dict(q=q, k=k, v=v, module=module.to(device=device, dtype=dtype))


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


def cfg3(device, seed: int = 0, layers: int = 4, history_frames: int = 120, resident_frames: int = 6,
         retrieved: int = 8, q_frames: int = 3, heads: int = 12, d: int = 128) -> dict:
    """HKV retrieval workload (see the module docstring). Returns device / pinned-host tensors:

    host_k / host_v: per layer ``[1, host_frames * 1560, H, D]`` pinned bf16 (roped keys);
    pool_k / pool_v: per layer device ``[1, (retrieved + resident) * 1560, H, D]`` with the resident
        frames already in the last ``resident_frames`` slots;
    keys0: device ``[1, history_frames * 1560, H, D]`` layer-0 keys (the page-summary input);
    q: device roped queries ``[1, q_frames * 1560, H, D]``; q_content: pre-rope ``[1, Lq, H*D]``;
    freqs: the complex128 RoPE table (device); truth: the host frames the query was built from.
    """
    g = torch.Generator(device=device).manual_seed(seed)
    host_frames = history_frames - resident_frames
    ft = FRAME_TOKENS
    freqs = rope_freqs(1024, d).to(device)
    offsets = torch.randn(history_frames, heads, d, generator=g, device=device) * 0.5
    truth = sorted(torch.randperm(host_frames, generator=g, device=device)[:retrieved].tolist())
    host_k, host_v, pool_k, pool_v = [], [], [], []
    keys0 = None
    slots = (retrieved + resident_frames) * ft
    for layer in range(layers):
        k = torch.randn(1, history_frames * ft, heads, d, generator=g, device=device)
        k += offsets.repeat_interleave(ft, dim=0).unsqueeze(0)
        k = apply_rope_3d(k, freqs, history_frames, FRAME_H, FRAME_W, 0).to(torch.bfloat16)
        v = torch.randn(1, history_frames * ft, heads, d, generator=g, device=device).to(torch.bfloat16)
        if layer == 0:
            keys0 = k
        hk = torch.empty((1, host_frames * ft, heads, d), dtype=torch.bfloat16, pin_memory=True)
        hv = torch.empty_like(hk, pin_memory=True)
        hk.copy_(k[:, : host_frames * ft])
        hv.copy_(v[:, : host_frames * ft])
        pk = torch.zeros((1, slots, heads, d), dtype=torch.bfloat16, device=device)
        pv = torch.zeros_like(pk)
        pk[:, retrieved * ft:] = k[:, host_frames * ft:]
        pv[:, retrieved * ft:] = v[:, host_frames * ft:]
        host_k.append(hk)
        host_v.append(hv)
        pool_k.append(pk)
        pool_v.append(pv)
        del k, v
    lq = q_frames * ft
    mix = offsets[truth].mean(dim=0) * 4.0
    qc = torch.randn(1, lq, heads, d, generator=g, device=device) + mix.unsqueeze(0).unsqueeze(0)
    q = apply_rope_3d(qc, freqs, q_frames, FRAME_H, FRAME_W, history_frames).to(torch.bfloat16)
    gm = torch.Generator().manual_seed(seed + 1)
    modes = head_split(gm, heads, 4)
    return dict(host_k=host_k, host_v=host_v, pool_k=pool_k, pool_v=pool_v, keys0=keys0, q=q,
                q_content=qc.reshape(1, lq, heads * d).to(torch.bfloat16), freqs=freqs, truth=truth,
                history_frames=history_frames, host_frames=host_frames, resident_frames=resident_frames,
                retrieved=retrieved, frame_tokens=ft, block_size=128, head_modes=modes,
                topk=[16 if m == "sparse" else 0 for m in modes], linear_mode="elu1")


def cfg4_layer(seed: int = 0, heads: int = 40, d: int = 128, q_len: int = 3 * FRAME_TOKENS,
               kv_len: int = 28080 + 3 * FRAME_TOKENS, dtype=torch.bfloat16) -> dict:
    """One H=40 HSA layer call of the cfg 4 stack with seeded N(0,1) activations (CPU tensors):
    q ``[1, 4680, 40, 128]``, k / v ``[1, 32760, 40, 128]``, heads 0..29 sparse (top-16), 30..39
    elu1 linear. The stack's projections of N(0,1) inputs by 1/sqrt(dim)-scaled weights give
    unit-variance q / k / v, which is what this draws directly."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, q_len, heads, d, generator=g).to(dtype)
    k = torch.randn(1, kv_len, heads, d, generator=g).to(dtype)
    v = torch.randn(1, kv_len, heads, d, generator=g).to(dtype)
    n_sparse = heads * 3 // 4
    modes = ["sparse"] * n_sparse + ["linear"] * (heads - n_sparse)
    return dict(q=q, k=k, v=v, block_size=128, routing="topk", topk=[16 if m == "sparse" else 0 for m in modes],
                head_modes=modes, linear_mode="elu1", proj_segment_len=FRAME_TOKENS)


def cfg4(device, seed: int = 0, layers: int = 40, heads: int = 40, d: int = 128, history: int = 28080,
         chunk: int = 3 * FRAME_TOKENS) -> dict:
    """Wan-14B stack workload (see the module docstring): weights and caches on ``device``."""
    g = torch.Generator(device=device).manual_seed(seed)
    dim = heads * d
    scale = 1.0 / math.sqrt(dim)
    w_qkv = [(torch.randn(dim, 3 * dim, generator=g, device=device) * scale).to(torch.bfloat16) for _ in range(layers)]
    w_out = [(torch.randn(dim, dim, generator=g, device=device) * scale).to(torch.bfloat16) for _ in range(layers)]
    k_cache = [torch.randn(1, history + chunk, heads, d, generator=g, device=device).to(torch.bfloat16)
               for _ in range(layers)]
    v_cache = [torch.randn(1, history + chunk, heads, d, generator=g, device=device).to(torch.bfloat16)
               for _ in range(layers)]
    x = torch.randn(1, chunk, dim, generator=g, device=device).to(torch.bfloat16)
    modes = ["sparse"] * 30 + ["linear"] * 10 if heads == 40 else head_split(torch.Generator().manual_seed(seed), heads,
                                                                                heads // 4)
    return dict(w_qkv=w_qkv, w_out=w_out, k_cache=k_cache, v_cache=v_cache, x=x, history=history, chunk=chunk,
                heads=heads, d=d, block_size=128, head_modes=modes,
                topk=[16 if m == "sparse" else 0 for m in modes], linear_mode="elu1")
