"""CPU oracle for Hybrid Sparse Attention (HSA) — test infrastructure only.

Restates, with plain PyTorch CPU ops, what the reference computes in
``wan/modules/hsa/routing.py``, ``wan/modules/hsa/block_sparse_torch.py``,
``wan/modules/hsa/attention.py`` and ``trainer/hsa_stage.py``, plus the two north-star extensions
(per-head top-k routing and the ``elu(x)+1`` kernelized linear branch) that have no reference code.

Every function keeps the reference's rounding points (bf16 casts, fp32 logits, double cumsum), so
for the reference's own modes the oracle and the reference agree bit for bit on torch-CPU, except
where the reference itself is implementation-defined (``torch.sort(stable=False)`` tie order): the
oracle always sorts stably, i.e. ties go lowest block index first.

``compute=torch.float64`` variants (where offered) are the high-precision references the HIP
kernels' tolerances are stated against.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn.functional as F

HEAD_MODES = ("both", "sparse", "linear")
LINEAR_MODES = ("lowrank", "elu1")
ROUTING_MODES = ("gini", "topk")


# ----------------------------------------------------------------------------------------------
# Shapes (routing.py:121-142)
# ----------------------------------------------------------------------------------------------
def block_counts(q_len: int, kv_len: int, block_size: int):
    """Padded lengths and block counts. Follows ``routing.py:138-142``.

    pinned by: closed form (ceil division), tests/test_oracle_hsa.py::test_block_counts.
    """
    nq = -(-q_len // block_size)
    nkv = -(-kv_len // block_size)
    return nq * block_size, nkv * block_size, nq, nkv


def pad_to_len(x: torch.Tensor, target_len: int) -> torch.Tensor:
    """Zero-pad ``[B, L, H, D]`` on the token axis. Follows ``routing.py:129-135``."""
    extra = target_len - x.shape[1]
    if extra <= 0:
        return x
    return F.pad(x, (0, 0, 0, 0, 0, extra))


def variable_block_sizes(kv_len: int, kv_len_padded: int, block_size: int) -> torch.Tensor:
    """Real token count per key block (last one may be partial). Follows ``routing.py:121-126``."""
    n = kv_len_padded // block_size
    sizes = torch.full((n,), block_size, dtype=torch.int32)
    sizes[-1] = kv_len - (n - 1) * block_size
    return sizes


# ----------------------------------------------------------------------------------------------
# Routing (routing.py:25-118)
# ----------------------------------------------------------------------------------------------
class BlockRouting:
    """Routing result, same fields as the reference ``BlockRouting`` (``routing.py:25-42``)."""

    __slots__ = ("index", "num", "mask", "thresholds")

    def __init__(self, index, num, mask, thresholds):
        self.index, self.num, self.mask, self.thresholds = index, num, mask, thresholds


def block_mean_pool(x: torch.Tensor, logical_len: int, num_blocks: int, block_size: int) -> torch.Tensor:
    """Mean of each block's real tokens, ``[B, H, N*Bs, D] -> [B, H, N, D]``.

    Follows ``routing.py:45-61`` including its dtype behaviour: with no partial block the result
    is ``mean`` in the input dtype (fp32 accumulate, one rounding); with a partial trailing block
    the per-block *sum* is rounded to the input dtype and then divided in fp32, giving fp32.

    pinned by: partial-block known answer (reference ``tests/test_hsa_routing.py:86-94``), and a
    per-element brute-force loop in tests/test_oracle_hsa.py.
    """
    b, h, _, d = x.shape
    blocks = x.reshape(b, h, num_blocks, block_size, d)
    if logical_len % block_size == 0:
        return blocks.mean(dim=3)
    real = torch.full((num_blocks,), float(block_size), dtype=torch.float32)
    real[-1] = float(logical_len - (num_blocks - 1) * block_size)
    keep = (torch.arange(block_size).view(1, block_size) < real.to(torch.int64).view(num_blocks, 1))
    summed = (blocks * keep.view(1, 1, num_blocks, block_size, 1).to(x.dtype)).sum(dim=3)
    return summed / real.view(1, 1, num_blocks, 1)


def block_attention_map(q_pooled: torch.Tensor, k_pooled: torch.Tensor) -> torch.Tensor:
    """fp32 ``softmax(qp kp^T / sqrt(D))``. Follows ``routing.py:64-68``.

    pinned by: row sums are 1 (reference ``tests/test_hsa_routing.py:207``) and an fp64 einsum.
    """
    logits = torch.matmul(q_pooled.float(), k_pooled.float().transpose(-2, -1)) * (q_pooled.shape[-1] ** -0.5)
    return torch.softmax(logits, dim=-1)


def build_block_routing(block_attn: torch.Tensor, tau_min: float, tau_max: float, *,
                        return_mask: bool = False, heads: Optional[Sequence[int]] = None) -> BlockRouting:
    """Head-adaptive cumulative-mass routing. Follows ``routing.py:71-118``.

    * rows sorted descending (stable: equal weights keep ascending block order);
    * row Gini ``sum_m (N+1-2m) p_(m) / N`` (fp32 ops), head Gini = mean over (batch, q-block);
    * ``tau_h = tau_min + G_h (tau_max - tau_min)`` in fp32;
    * ``num`` = count of sorted slots whose exclusive prefix (fp32 of the double cumsum, minus the
      slot's own weight) is below ``tau_h``; ``index`` is the whole descending permutation.

    ``heads`` (extension) restricts routing to a subset of heads: the others get ``num = 0``
    (their thresholds are still reported; per-head quantities do not couple heads).

    pinned by: independent loop transcription (reference ``tests/test_hsa_routing.py:11-57``),
    known answers uniform -> 0 and one-hot -> (N-1)/N (``:60-72``), per-head thresholds
    (``:75-83``), invariants (``:196-212``); and golden vectors written from the reference module
    itself (tests/golden/routing_gini.pt).
    """
    _, nheads, _, nkv = block_attn.shape
    probs = block_attn.float()
    sorted_p, order = torch.sort(probs, dim=-1, descending=True, stable=True)
    ranks = torch.arange(1, nkv + 1, dtype=sorted_p.dtype)
    gini = torch.sum((nkv + 1 - 2 * ranks) * sorted_p, dim=-1) / nkv
    thresholds = tau_min + gini.mean(dim=(0, 2)) * (tau_max - tau_min)
    exclusive = torch.cumsum(sorted_p, dim=-1) - sorted_p
    keep = exclusive < thresholds.view(1, nheads, 1, 1)
    if heads is not None:
        routed = torch.zeros(nheads, dtype=torch.bool)
        routed[list(heads)] = True
        keep = keep & routed.view(1, nheads, 1, 1)
    num = keep.sum(dim=-1, dtype=torch.int32)
    mask = None
    if return_mask:
        mask = torch.zeros_like(probs, dtype=torch.bool).scatter_(-1, order, keep)
    return BlockRouting(order.to(torch.int32), num, mask, thresholds)


def build_topk_routing(block_attn: torch.Tensor, head_k, *, return_mask: bool = False) -> BlockRouting:
    """North-star per-head top-k routing (no reference code).

    ``index`` is the same stable descending permutation as :func:`build_block_routing`, and
    ``num[b, h, i] = min(k_h, Nkv)``; a head with ``k_h = 0`` is not routed. Thresholds are zero.

    pinned by: ``torch.topk`` agreement on tie-free rows and a brute-force lowest-index tie rule in
    tests/test_oracle_hsa.py.
    """
    bsz, nheads, nq, nkv = block_attn.shape
    ks = _per_head(head_k, nheads)
    _, order = torch.sort(block_attn.float(), dim=-1, descending=True, stable=True)
    num = torch.tensor([min(k, nkv) for k in ks], dtype=torch.int32).view(1, nheads, 1).expand(bsz, nheads, nq)
    mask = None
    if return_mask:
        slot = torch.arange(nkv).view(1, 1, 1, nkv)
        keep = slot < num.unsqueeze(-1)
        mask = torch.zeros(block_attn.shape, dtype=torch.bool).scatter_(-1, order, keep)
    return BlockRouting(order.to(torch.int32), num.contiguous(), mask, torch.zeros(nheads))


def map_to_index(block_map: torch.Tensor):
    """Boolean ``[B, H, Nq, Nkv]`` mask -> ascending ``(index, num)``, index padded with -1.

    Follows ``block_sparse_triton.py:20-57``. pinned by: brute-force nonzero() per row.
    """
    index = torch.full(block_map.shape, -1, dtype=torch.int32)
    num = block_map.sum(dim=-1, dtype=torch.int32)
    flat_map = block_map.reshape(-1, block_map.shape[-1])
    flat_idx = index.view(-1, block_map.shape[-1])
    for r in range(flat_map.shape[0]):
        sel = torch.nonzero(flat_map[r]).flatten()
        flat_idx[r, : sel.numel()] = sel.to(torch.int32)
    return index, num


def _per_head(value, nheads: int):
    if isinstance(value, int):
        return [int(value)] * nheads
    vals = [int(v) for v in value]
    if len(vals) != nheads:
        raise ValueError(f"expected {nheads} per-head values, got {len(vals)}")
    return vals


# ----------------------------------------------------------------------------------------------
# Block-sparse attention (block_sparse_torch.py:16-64; LSE convention block_sparse_triton.py:136)
# ----------------------------------------------------------------------------------------------
def block_sparse_attention(q, k, v, q2k_index, q2k_num, block_sizes, block_size, *,
                           compute_dtype=None, return_lse=False):
    """Attention of each query block over its first ``num`` listed key blocks.

    ``[B, H, N, D]`` inputs padded to ``block_size``. Follows ``block_sparse_torch.py:16-64``:
    listed ids are clamped to ``[0, Nkv-1]``, key tokens at or past ``block_sizes[j]`` are masked,
    a row with nothing selected returns 0, the math runs in fp32 (or the input's fp64) and the
    result is cast back to ``q.dtype``. A block listed twice is attended twice, as the reference's
    gather does.

    ``return_lse`` also returns the natural-log log-sum-exp of the scaled logits per query row
    (``-inf`` for empty rows).

    pinned by: SDPA equivalence on full selection, single block and partial tail (reference
    ``tests/test_hsa_routing.py:97-151``), slot invariance (``:154-178``), empty -> 0 (``:181-193``).
    """
    bsz, heads, nq_tok, d = q.shape
    nq = nq_tok // block_size
    nkv = k.shape[2] // block_size
    if compute_dtype is None:
        compute_dtype = q.dtype if q.dtype in (torch.float32, torch.float64) else torch.float32
    scale = 1.0 / math.sqrt(d)
    qc, kc, vc = q.to(compute_dtype), k.to(compute_dtype), v.to(compute_dtype)
    out = torch.zeros((bsz, heads, nq_tok, d), dtype=compute_dtype)
    lse = torch.full((bsz, heads, nq_tok), -math.inf, dtype=compute_dtype)
    sizes = [int(s) for s in block_sizes.tolist()]
    for b in range(bsz):
        for h in range(heads):
            for i in range(nq):
                n = int(q2k_num[b, h, i])
                if n <= 0:
                    continue
                ids = [min(max(int(j), 0), max(nkv - 1, 0)) for j in q2k_index[b, h, i, :n].tolist()]
                spans = [(j * block_size, j * block_size + max(min(sizes[j], block_size), 0)) for j in ids]
                keys = torch.cat([kc[b, h, s:e] for s, e in spans])
                vals = torch.cat([vc[b, h, s:e] for s, e in spans])
                if keys.shape[0] == 0:
                    continue
                qi = qc[b, h, i * block_size:(i + 1) * block_size]
                logits = torch.matmul(qi, keys.transpose(0, 1)) * scale
                out[b, h, i * block_size:(i + 1) * block_size] = torch.matmul(torch.softmax(logits, -1), vals)
                lse[b, h, i * block_size:(i + 1) * block_size] = torch.logsumexp(logits, -1)
    out = out.to(q.dtype)
    return (out, lse) if return_lse else out


def block_sparse_attention_gather(q, k, v, q2k_index, q2k_num, block_sizes, block_size):
    """Same result as :func:`block_sparse_attention`, vectorized the way the reference's torch path
    is (``block_sparse_torch.py:30-64``): every row's listed key blocks are gathered at once
    (width = the longest list), slots past ``num`` and tokens past ``block_sizes[j]`` are masked,
    rows with nothing valid give 0. Autograd through it is cheap at the benchmark shapes.

    pinned by: equality with the per-row loop of :func:`block_sparse_attention` (duplicates,
    clamped ids, partial blocks, empty rows) in tests/test_oracle_hsa.py.
    """
    bsz, heads, nq_tok, d = q.shape
    nq, nkv = nq_tok // block_size, k.shape[2] // block_size
    width = max(int(q2k_num.max()), 1)
    ids = q2k_index[..., :width].long().clamp(0, max(nkv - 1, 0))               # [B, H, Nq, W]
    comp = q.dtype if q.dtype in (torch.float32, torch.float64) else torch.float32
    tok = (ids.unsqueeze(-1) * block_size + torch.arange(block_size)).flatten(-2)  # [B, H, Nq, W*Bs]
    bi = torch.arange(bsz).view(bsz, 1, 1, 1)
    hi = torch.arange(heads).view(1, heads, 1, 1)
    keys = k.to(comp)[bi, hi, tok]                                                # [B, H, Nq, W*Bs, D]
    vals = v.to(comp)[bi, hi, tok]
    qb = q.to(comp).view(bsz, heads, nq, block_size, d)
    logits = torch.matmul(qb, keys.transpose(-1, -2)) / math.sqrt(d)              # [B, H, Nq, Bs, W*Bs]
    slot_ok = torch.arange(width).view(1, 1, 1, width) < q2k_num.long().unsqueeze(-1)
    tok_ok = torch.arange(block_size).view(1, 1, 1, 1, block_size) < block_sizes.long()[ids].unsqueeze(-1)
    ok = (slot_ok.unsqueeze(-1) & tok_ok).flatten(-2).unsqueeze(-2)               # [B, H, Nq, 1, W*Bs]
    logits = logits.masked_fill(~ok, float("-inf"))
    probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
    return torch.matmul(probs, vals).reshape(bsz, heads, nq_tok, d).to(q.dtype)


# ----------------------------------------------------------------------------------------------
# Linear branch (attention.py:64-118) and the north-star elu(x)+1 branch
# ----------------------------------------------------------------------------------------------
def compress_kv(k, v, *, segment_len, k_proj_mat, v_proj_mat, block_size):
    """Low-rank sequence projection per segment, ``[B, H, L, D] -> [B, H, sum r, D]``.

    Follows ``attention.py:64-110``: ``r = min(rank, ceil(seg_len / block_size))``, fp32 math with
    the projection cast to fp32, result cast back to the input dtype.

    pinned by: closed form ``E @ K`` (reference ``tests/test_hsa_attention.py:138-150``) and
    coarse-cache == inline (``:128-135``).
    """
    if k_proj_mat.shape != v_proj_mat.shape:
        raise ValueError("k_proj_mat and v_proj_mat must have the same shape")
    length = k.shape[2]
    if segment_len <= 0:
        segment_len = length
    outs_k, outs_v = [], []
    for start in range(0, length, segment_len):
        end = min(start + segment_len, length)
        seg = end - start
        if seg > k_proj_mat.shape[1]:
            raise ValueError(f"segment length {seg} exceeds projection length {k_proj_mat.shape[1]}")
        r = min(k_proj_mat.shape[0], -(-seg // block_size))
        ek = k_proj_mat[:r, :seg].float()
        ev = v_proj_mat[:r, :seg].float()
        outs_k.append(torch.matmul(ek, k[:, :, start:end].float()).to(k.dtype))
        outs_v.append(torch.matmul(ev, v[:, :, start:end].float()).to(v.dtype))
    return torch.cat(outs_k, dim=2), torch.cat(outs_v, dim=2)


def linear_branch_lowrank(q, k_coarse, v_coarse):
    """Softmax attention of full-resolution queries over compressed keys. ``attention.py:113-118``.

    pinned by: SDPA on (q, Kc, Vc) in fp64.
    """
    logits = torch.matmul(q.float(), k_coarse.float().transpose(-2, -1)) * (q.shape[-1] ** -0.5)
    weights = torch.softmax(logits, dim=-1)
    return torch.matmul(weights.to(v_coarse.dtype), v_coarse)


def elu1(x: torch.Tensor) -> torch.Tensor:
    """Feature map ``phi(x) = elu(x) + 1`` (positive everywhere)."""
    return F.elu(x) + 1.0


def linear_branch_elu1(q, k, v, *, compute_dtype=torch.float32, return_state=False):
    """North-star kernelized linear attention over ``[B, H, L, D]`` (no reference code).

    ``S = sum_t phi(k_t) v_t^T``, ``z = sum_t phi(k_t)``, ``o = phi(q) S / (phi(q) . z)``,
    non-causal over the whole KV window, computed in ``compute_dtype`` and cast to ``v.dtype``.

    pinned by: the quadratic form ``(phi(Q) phi(K)^T) V / rowsum`` in fp64 and a per-token loop on
    tiny shapes (tests/test_oracle_hsa.py).
    """
    fq = elu1(q.to(compute_dtype))
    fk = elu1(k.to(compute_dtype))
    state = torch.matmul(fk.transpose(-2, -1), v.to(compute_dtype))        # [B, H, D, D]
    zsum = fk.sum(dim=-2)                                                  # [B, H, D]
    num = torch.matmul(fq, state)
    den = torch.matmul(fq, zsum.unsqueeze(-1))
    out = (num / den).to(v.dtype)
    return (out, state, zsum) if return_state else out


# ----------------------------------------------------------------------------------------------
# Full composition (attention.py:153-259) with the north-star head modes
# ----------------------------------------------------------------------------------------------
def hsa_attention(q, k, v, *, k_coarse=None, v_coarse=None, k_proj_mat=None, v_proj_mat=None,
                  gate_weight=None, gate_bias=None, block_size=64, tau_min=0.35, tau_max=1.0,
                  proj_segment_len=1560, routing="gini", topk=None, head_modes=None,
                  linear_mode="lowrank", return_parts=False):
    """HSA over ``[B, L, H, D]`` tensors. Follows ``attention.py:153-259``.

    Reference behaviour is ``routing="gini"``, ``linear_mode="lowrank"``, every head ``"both"``:
    ``out = sparse + sigmoid(gate_lin(q)) * linear``. Extensions (north star): ``routing="topk"``
    with per-head ``topk``; ``linear_mode="elu1"``; ``head_modes`` per head in
    {"both", "sparse", "linear"}, where a head contributes only the branches it runs:
    ``out_h = [runs sparse] sparse_h + [runs linear] gate_h * linear_h``.

    The gate is ``sigmoid(F.linear(q.to(W.dtype), W, b))`` when ``gate_weight`` is given, else
    ``sigmoid(q)`` (``attention.py:246-251``); all branch sums happen in the linear branch's dtype
    and the result is cast to ``q.dtype``.

    pinned by: gated-sum identity (reference ``tests/test_hsa_attention.py:91-99``), coarse == inline
    (``:128-135``), and golden vectors from the reference module (tests/golden/hsa_attention.pt).
    """
    bsz, q_len, heads, d = q.shape
    kv_len = k.shape[1]
    modes = list(head_modes) if head_modes is not None else ["both"] * heads
    if len(modes) != heads or any(m not in HEAD_MODES for m in modes):
        raise ValueError(f"head_modes must list one of {HEAD_MODES} per head")
    sparse_heads = [h for h, m in enumerate(modes) if m in ("both", "sparse")]
    linear_heads = [h for h, m in enumerate(modes) if m in ("both", "linear")]
    out_dtype = q.dtype
    q_t = q.transpose(1, 2).contiguous()
    k_t = k.transpose(1, 2).contiguous()
    v_t = v.transpose(1, 2).contiguous()

    if linear_mode == "lowrank":
        if k_coarse is None:
            kc, vc = compress_kv(k_t, v_t, segment_len=proj_segment_len, k_proj_mat=k_proj_mat,
                                 v_proj_mat=v_proj_mat, block_size=block_size)
        else:
            kc, vc = k_coarse.transpose(1, 2).contiguous(), v_coarse.transpose(1, 2).contiguous()
        linear = linear_branch_lowrank(q_t, kc, vc)
    elif linear_mode == "elu1":
        linear = linear_branch_elu1(q_t, k_t, v_t)
    else:
        raise ValueError(f"linear_mode must be one of {LINEAR_MODES}")

    q_pad_len, kv_pad_len, nq, nkv = block_counts(q_len, kv_len, block_size)
    q_p = pad_to_len(q, q_pad_len).transpose(1, 2).contiguous()
    k_p = pad_to_len(k, kv_pad_len).transpose(1, 2).contiguous()
    v_p = pad_to_len(v, kv_pad_len).transpose(1, 2).contiguous()
    attn_map = block_attention_map(block_mean_pool(q_p, q_len, nq, block_size),
                                   block_mean_pool(k_p, kv_len, nkv, block_size))
    if routing == "gini":
        route = build_block_routing(attn_map, tau_min, tau_max, heads=sparse_heads)
    elif routing == "topk":
        ks = _per_head(topk, heads)
        ks = [kk if h in sparse_heads else 0 for h, kk in enumerate(ks)]
        route = build_topk_routing(attn_map, ks)
    else:
        raise ValueError(f"routing must be one of {ROUTING_MODES}")
    sizes = variable_block_sizes(kv_len, kv_pad_len, block_size)
    sparse = block_sparse_attention_gather(q_p.to(torch.bfloat16), k_p.to(torch.bfloat16),
                                           v_p.to(torch.bfloat16), route.index, route.num, sizes, block_size)

    comp = linear.dtype
    if gate_weight is not None:
        gate = torch.sigmoid(F.linear(q.to(gate_weight.dtype), gate_weight, gate_bias)).to(comp)
    else:
        gate = torch.sigmoid(q.to(comp))
    sparse_t = sparse.transpose(1, 2)[:, :q_len].to(comp)
    linear_t = linear.transpose(1, 2)
    out = torch.zeros((bsz, q_len, heads, d), dtype=comp)
    for h in range(heads):
        runs_s, runs_l = h in sparse_heads, h in linear_heads
        if runs_s and runs_l:
            out[:, :, h] = torch.addcmul(sparse_t[:, :, h], linear_t[:, :, h], gate[:, :, h])
        elif runs_s:
            out[:, :, h] = sparse_t[:, :, h]
        else:
            out[:, :, h] = torch.addcmul(torch.zeros_like(linear_t[:, :, h]), linear_t[:, :, h], gate[:, :, h])
    out = out.to(out_dtype)
    if return_parts:
        return out, {"routing": route, "attn_map": attn_map, "sparse": sparse_t, "linear": linear_t,
                     "gate": gate, "block_sizes": sizes}
    return out


# ----------------------------------------------------------------------------------------------
# Parameter init (trainer/hsa_stage.py:43-82) and module-level helpers (attention.py:331-347)
# ----------------------------------------------------------------------------------------------
def init_projection(rank: int, seg_len: int, block_size: int, dtype=torch.bfloat16) -> torch.Tensor:
    """Row ``r`` averages tokens ``[r*Bs, min((r+1)*Bs, seg))``. Follows ``hsa_stage.py:43-82``.

    pinned by: known rows (reference ``tests/test_hsa_attention.py:153-160``).
    """
    proj = torch.zeros((rank, seg_len), dtype=dtype)
    for r in range(rank):
        s, e = r * block_size, min((r + 1) * block_size, seg_len)
        if e > s:
            proj[r, s:e] = 1.0 / float(e - s)
    return proj


def coarse_cache_size(kv_cache_size: int, seg_len: int, rank: int) -> int:
    """``ceil(n / seg) * rank``. Follows ``attention.py:331-335``."""
    return 0 if kv_cache_size <= 0 else -(-kv_cache_size // seg_len) * rank


def token_range_to_coarse(start: int, end: int, seg_len: int, rank: int):
    """Segment-aligned token range -> coarse slots. Follows ``attention.py:337-347``."""
    if start % seg_len or end % seg_len:
        raise ValueError("coarse-cache access requires segment-aligned token indices")
    return (start // seg_len) * rank, (end // seg_len) * rank
