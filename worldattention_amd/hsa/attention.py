"""Hybrid Sparse Attention (HSA) on MI355X, with the reference's call signatures.

Mirrors ``wan/modules/hsa/attention.py``: ``resolve_backend`` (:47-61), ``compress_kv`` (:64-110),
``_linear_branch`` (:113-118), ``hsa_parameter_names`` (:121-132), ``require_trained_hsa``
(:135-150), ``hsa_attention`` (:153-259) and ``HSAAttention`` (:262-380).

Every branch runs in ``libworldattention_amd`` on ``[B, L, H, D]`` tensors in place (no transposes,
no pad copies): routing (``wa_block_mean_pool`` + ``wa_route``), the sparse branch (``wa_bsa_fwd``
over the routed lists), the linear branch (``wa_compress_kv`` + dense ``wa_bsa_fwd`` over the
compressed keys, or ``wa_elu1_state`` + ``wa_elu1_readout``), and the gated fusion (in the
epilogue of whichever kernel writes a head's output last).

North-star extensions (keyword-only, defaults give the reference behaviour):

* ``routing="topk"`` with ``topk`` (int or per-head list) instead of Gini routing;
* ``linear_mode="elu1"``: kernelized linear attention ``phi(q) S / (phi(q) . z)``,
  ``phi = elu + 1``, over the full-resolution KV window;
* ``head_modes``: per head ``"both"`` (reference), ``"sparse"`` or ``"linear"``; a head adds only
  the branches it runs: ``out_h = [sparse] sparse_h + [linear] gate_h * linear_h``.
"""
from __future__ import annotations

import contextlib
import math
from typing import Optional, Sequence

import torch
import torch.nn as nn

from .. import _lib
from . import distill
from .block_sparse import bsa_forward, padded_head_dim, unit_table
from .routing import BlockRouting, _route, block_counts, pool_for_routing

__all__ = [
    "HSAAttention",
    "hsa_attention",
    "compress_kv",
    "resolve_backend",
    "hsa_parameter_names",
    "require_trained_hsa",
]

_BACKENDS = ("auto", "triton", "torch")
_HSA_ATTR = "hsa_attention"
_HEAD_MODES = ("both", "sparse", "linear")
_LINEAR_MODES = ("lowrank", "elu1")
_ROUTING_MODES = ("gini", "topk")
SUPPORTED_BLOCK_SIZES = (64, 128)
# Value of a key's padding channels: the queries' padding is zero, so q . k is unchanged, and the
# elu(x)+1 feature of the padding, exp(-200), is 0 in fp32 (exactly representable in bf16).
PAD_KEY_VALUE = -200.0


def resolve_backend(backend: str) -> str:
    """Validate a backend name (``attention.py:47-61``).

    Accepts ``"auto"``, ``"triton"`` and ``"torch"`` and rejects anything else, as the reference
    does. Every name runs the same HIP kernels; the name is kept so existing configs load.
    """
    backend = str(backend or "auto").lower()
    if backend not in _BACKENDS:
        raise ValueError(f"unknown HSA backend {backend!r}; expected one of {_BACKENDS}")
    if backend != "auto":
        return backend
    return "triton" if torch.cuda.is_available() else "torch"


# ----------------------------------------------------------------------------------------------
# Low-rank compression
# ----------------------------------------------------------------------------------------------
def coarse_length(kv_len: int, segment_len: int, proj_rank: int, block_size: int) -> int:
    """Rows produced by compressing ``kv_len`` tokens (sum of per-segment ranks)."""
    if segment_len <= 0:
        segment_len = kv_len
    total = 0
    for start in range(0, kv_len, segment_len):
        seg = min(segment_len, kv_len - start)
        total += min(proj_rank, math.ceil(seg / block_size))
    return total


def _pad_channels(t: Optional[torch.Tensor], d_to: int, value: float = 0.0) -> Optional[torch.Tensor]:
    """``t`` with its last dim padded to ``d_to`` with ``value`` (differentiable)."""
    if t is None or t.shape[-1] == d_to:
        return t
    return torch.nn.functional.pad(t, (0, d_to - t.shape[-1]), value=value)


def _compress(x: torch.Tensor, proj: torch.Tensor, *, segment_len: int, block_size: int, layout: str,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out`` (optional): a view of the destination rows (same layout, dtype of ``x``), e.g. slots
    of a compressed cache, written in place. Head dims the kernel lacks run zero-padded (the
    projection acts on each channel alone)."""
    dev = _lib.require_gpu(x, proj)
    if layout == "bhld":
        bsz, heads, length, d = x.shape
    else:
        bsz, length, heads, d = x.shape
    if d not in (32, 64, 128):
        dp = padded_head_dim(d, (32, 64, 128))
        res = _compress(_pad_channels(x, dp), proj, segment_len=segment_len, block_size=block_size, layout=layout)
        res = res[..., :d]
        if out is None:
            return res.contiguous()
        out.copy_(res)
        return out
    if segment_len <= 0:
        segment_len = length
    for start in range(0, length, segment_len):
        seg = min(segment_len, length - start)
        if seg > proj.shape[1]:
            raise ValueError(
                f"segment length {seg} exceeds projection length {proj.shape[1]}; increase proj_segment_len")
    lc = coarse_length(length, segment_len, proj.shape[0], block_size)
    src = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
    if src.stride(-1) != 1:
        src = src.contiguous()
    pj = proj if proj.dtype in (torch.float32, torch.bfloat16) else proj.float()
    pj = pj.contiguous()
    shape = (bsz, heads, lc, d) if layout == "bhld" else (bsz, lc, heads, d)
    if out is None:
        out = torch.empty(shape, dtype=x.dtype, device=dev)
    elif tuple(out.shape) != shape or out.dtype != x.dtype or out.stride(-1) != 1:
        raise ValueError(f"compress output must be {x.dtype} {shape} with unit last stride, got "
                         f"{out.dtype} {tuple(out.shape)}")
    if layout == "bhld":
        xp, x_sb, x_st, x_sh = _lib.bhld(src)
        op, o_sb, o_st, o_sh = _lib.bhld(out)
    else:
        xp, x_sb, x_st, x_sh = _lib.blhd(src)
        op, o_sb, o_st, o_sh = _lib.blhd(out)
    args = _lib.CompressArgs(xp, x_sb, x_st, x_sh, _lib.dtype_code(src), pj.data_ptr(), _lib.dtype_code(pj),
                             pj.shape[0], pj.shape[1], bsz, length, heads, d, segment_len, block_size,
                             op, o_sb, o_st, o_sh, _lib.dtype_code(out))
    _lib.call("wa_compress_kv", args, _lib.stream_ptr(dev))
    return out


def compress_kv(k: torch.Tensor, v: torch.Tensor, *, segment_len: int, k_proj_mat: torch.Tensor,
                v_proj_mat: torch.Tensor, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Project ``[B, H, L, D]`` keys and values onto the low-rank sequence basis (``attention.py:64-110``)."""
    if k_proj_mat.shape != v_proj_mat.shape:
        raise ValueError(
            "k_proj_mat and v_proj_mat must have the same shape, got "
            f"{tuple(k_proj_mat.shape)} and {tuple(v_proj_mat.shape)}")
    return (_compress(k, k_proj_mat, segment_len=segment_len, block_size=block_size, layout="bhld"),
            _compress(v, v_proj_mat, segment_len=segment_len, block_size=block_size, layout="bhld"))


def _linear_branch(q: torch.Tensor, k_coarse: torch.Tensor, v_coarse: torch.Tensor) -> torch.Tensor:
    """Softmax attention of ``[B, H, L, D]`` queries over compressed keys (``attention.py:113-118``);
    other head dims than 64 / 128 run zero-padded at the original scale."""
    d = q.shape[-1]
    dp = padded_head_dim(d)
    block = 128 if dp == 128 else 64
    qx, kx, vx = (_pad_channels(t, dp) for t in (q, k_coarse, v_coarse))
    out, _ = bsa_forward(_lib.kernel_ready(qx), _lib.kernel_ready(kx), _lib.kernel_ready(vx),
                         index=None, num=None, block_size=block, out_dtype=v_coarse.dtype,
                         scale=d ** -0.5 if dp != d else 0.0)
    return out[..., :d].contiguous() if dp != d else out


# ----------------------------------------------------------------------------------------------
# Parameter bookkeeping (pure Python, identical behaviour)
# ----------------------------------------------------------------------------------------------
def hsa_parameter_names(model: nn.Module) -> list[str]:
    """State-dict keys of every HSA parameter in ``model``, found by module type (``:121-132``)."""
    names = []
    for module_name, module in model.named_modules():
        if isinstance(module, HSAAttention):
            prefix = f"{module_name}." if module_name else ""
            names.extend(prefix + name for name, _ in module.named_parameters())
    return names


def require_trained_hsa(missing_keys, checkpoint_path: str = "") -> None:
    """Raise if a checkpoint load left any HSA parameter unfilled (``:135-150``)."""
    missing_hsa = [key for key in missing_keys if _HSA_ATTR in key]
    if not missing_hsa:
        return
    where = f" in {checkpoint_path}" if checkpoint_path else ""
    raise RuntimeError(
        f"{len(missing_hsa)} HSA parameters are absent{where}, so this checkpoint has not been "
        f"through HSA training. Load a checkpoint from the HSA stage, or set attn_backend=flash to "
        f"run the dense baseline. First missing keys: {missing_hsa[:6]}")


# ----------------------------------------------------------------------------------------------
# Orchestration
# ----------------------------------------------------------------------------------------------
class HeadPlan:
    """Which heads run which branch, as cached device id lists."""

    def __init__(self, heads: int, head_modes: Optional[Sequence[str]], device):
        modes = list(head_modes) if head_modes is not None else ["both"] * heads
        if len(modes) != heads or any(m not in _HEAD_MODES for m in modes):
            raise ValueError(f"head_modes must list one of {_HEAD_MODES} for each of the {heads} heads")
        self.modes = modes
        self.both = [h for h, m in enumerate(modes) if m == "both"]
        self.sparse_only = [h for h, m in enumerate(modes) if m == "sparse"]
        self.linear_only = [h for h, m in enumerate(modes) if m == "linear"]
        self.sparse = sorted(self.both + self.sparse_only)
        self.linear = sorted(self.both + self.linear_only)
        self.t = {name: (_lib.head_list(lst, device) if lst else None)
                  for name, lst in (("both", self.both), ("sparse_only", self.sparse_only),
                                    ("linear_only", self.linear_only), ("sparse", self.sparse),
                                    ("linear", self.linear))}


_PLAN_CACHE: dict = {}


def head_plan(heads: int, head_modes: Optional[Sequence[str]], device) -> HeadPlan:
    """:class:`HeadPlan` of a head-mode list, cached per (heads, modes, device)."""
    key = (heads, tuple(head_modes) if head_modes is not None else None, str(device))
    plan = _PLAN_CACHE.get(key)
    if plan is None:
        plan = _PLAN_CACHE[key] = HeadPlan(heads, head_modes, device)
    return plan


def elu1_state(k: torch.Tensor, v: torch.Tensor, heads_t: torch.Tensor):
    """``S^T`` ([B, n, D, D], fp32) and ``z`` ([B, n, D]) of the listed heads (``wa_elu1_state``)."""
    dev = _lib.require_gpu(k, v)
    if k.dtype != v.dtype:
        v = v.to(k.dtype)
    if k.dtype not in (torch.float32, torch.bfloat16):
        k, v = k.float(), v.float()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    bsz, length, heads, d = k.shape
    n = heads_t.numel()
    state = torch.empty((bsz, n, d, d), dtype=torch.float32, device=dev)
    zsum = torch.empty((bsz, n, d), dtype=torch.float32, device=dev)
    if n == 0:
        return state, zsum
    ws = torch.empty((_lib.lib().wa_elu1_state_workspace_bytes(bsz, n, length, d),), dtype=torch.uint8, device=dev)
    kp, k_sb, k_st, k_sh = _lib.blhd(k)
    vp, v_sb, v_st, v_sh = _lib.blhd(v)
    args = _lib.Elu1StateArgs(kp, k_sb, k_st, k_sh, vp, v_sb, v_st, v_sh, _lib.dtype_code(k), bsz, heads, length, d,
                              *_lib.heads_arg(heads_t), state.data_ptr(), zsum.data_ptr(), ws.data_ptr())
    _lib.call("wa_elu1_state", args, _lib.stream_ptr(dev))
    return state, zsum


def elu1_readout(q, state, zsum, heads_t, out, *, epilogue=_lib.WA_EPI_PLAIN, gate_w=None, gate_b=None,
                 gate_pre_bf16=False, gate_out_bf16=False, lin_round_bf16=False):
    dev = _lib.require_gpu(q, state, out)
    if heads_t.numel() == 0:
        return out
    q = q if q.dtype in (torch.float32, torch.bfloat16) else q.float()
    q = q if q.stride(-1) == 1 else q.contiguous()
    bsz, length, heads, d = q.shape
    qp, q_sb, q_st, q_sh = _lib.blhd(q)
    op, o_sb, o_st, o_sh = _lib.blhd(out)
    args = _lib.Elu1ReadoutArgs(qp, q_sb, q_st, q_sh, _lib.dtype_code(q), state.data_ptr(), zsum.data_ptr(),
                                op, o_sb, o_st, o_sh, _lib.dtype_code(out), bsz, heads, length, d,
                                *_lib.heads_arg(heads_t), epilogue, _lib.ptr(gate_w), _lib.ptr(gate_b),
                                int(gate_pre_bf16), int(gate_out_bf16), int(lin_round_bf16))
    _lib.call("wa_elu1_readout", args, _lib.stream_ptr(dev))
    return out


class GateSpec:
    """Kernel-side view of the fusion gate (``attention.py:246-251``)."""

    @staticmethod
    def _converted(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """Kernel-side copy of a gate parameter, held on the parameter object itself (so it dies
        with it) and refreshed when the parameter is modified in place (its version counter)."""
        per_t = t.__dict__.setdefault("_wa_kernel_copies", {})
        hit = per_t.get(dtype)
        if hit is None or hit[0] != t._version or hit[1] != t.data_ptr():
            hit = (t._version, t.data_ptr(), t.detach().to(dtype).contiguous())
            per_t[dtype] = hit
        return hit[2]

    def __init__(self, gate_lin: Optional[nn.Module], comp_dtype: torch.dtype):
        if gate_lin is not None:
            w = gate_lin.weight
            self.w = self._converted(w, torch.bfloat16)
            b = getattr(gate_lin, "bias", None)
            self.b = self._converted(b, torch.float32) if b is not None else None
            self.pre_bf16 = w.dtype == torch.bfloat16
            self.out_bf16 = w.dtype == torch.bfloat16 or comp_dtype == torch.bfloat16
        else:
            self.w, self.b = None, None
            self.pre_bf16 = comp_dtype == torch.bfloat16
            self.out_bf16 = comp_dtype == torch.bfloat16

    def kwargs(self):
        return dict(gate_w=self.w, gate_b=self.b, gate_pre_bf16=self.pre_bf16, gate_out_bf16=self.out_bf16)


def _per_head_k(topk, heads: int):
    if topk is None:
        raise ValueError("routing='topk' needs topk (an int or one budget per head)")
    ks = [int(topk)] * heads if isinstance(topk, int) else [int(x) for x in topk]
    if len(ks) != heads:
        raise ValueError(f"expected {heads} per-head top-k budgets, got {len(ks)}")
    return ks


def hsa_forward(q, k, v, *, k_coarse, v_coarse, k_proj_mat, v_proj_mat, gate_lin, block_size, tau_min,
                tau_max, proj_segment_len, routing, topk, head_modes, linear_mode, k_block_sums=None,
                k_pooled=None, save=None, scale=0.0):
    """Forward of HSA on the GPU; ``save`` (a dict) receives what the backward needs. ``scale``:
    the logit scale of routing and of both softmax branches (0: ``head_dim ** -0.5``; a caller
    that pads the head dim passes its original one's)."""
    bsz, q_len, heads, head_dim = q.shape
    kv_len = k.shape[1]
    dev = _lib.require_gpu(q, k, v, k_coarse, v_coarse)
    if block_size not in SUPPORTED_BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {SUPPORTED_BLOCK_SIZES}, got {block_size}")
    if head_dim not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128 for the gfx950 kernels, got {head_dim}")
    if routing not in _ROUTING_MODES:
        raise ValueError(f"routing must be one of {_ROUTING_MODES}")
    if linear_mode not in _LINEAR_MODES:
        raise ValueError(f"linear_mode must be one of {_LINEAR_MODES}")
    plan = head_plan(heads, head_modes, dev)

    out_dtype = q.dtype
    if linear_mode == "lowrank":
        comp_dtype = v_coarse.dtype if v_coarse is not None else v.dtype
    else:
        comp_dtype = v.dtype
    if comp_dtype not in (torch.float32, torch.bfloat16):
        comp_dtype = torch.float32
    gate = GateSpec(gate_lin, comp_dtype)
    lin_round = comp_dtype == torch.bfloat16

    out = torch.empty((bsz, q_len, heads, head_dim), dtype=comp_dtype, device=dev)
    if not scale and native_split_eligible(q, k, v, plan, routing, linear_mode, k_block_sums, k_pooled):
        _native_split_forward(q, k, v, plan, _per_head_k(topk, heads), gate, lin_round, block_size, q_len, kv_len,
                              out, save)
        return out if out.dtype == out_dtype else out.to(out_dtype)
    qb = _lib.kernel_ready(q)
    kb = _lib.kernel_ready(k)
    vb = _lib.kernel_ready(v)
    lin_tmp = torch.empty_like(out) if plan.both else None

    # With both branches present the linear branch runs on a side stream, concurrently with
    # routing and the sparse branch on the caller's stream; the two write disjoint heads of `out`
    # (or `lin_tmp`, joined before the fused sparse epilogue reads it). Its kernels are issued
    # first (measured: 3 us per call faster in graph replay than issuing the pooling first).
    main = torch.cuda.current_stream(dev)
    side = _fork_join(dev, main)[0] if plan.linear and plan.sparse else None
    if side is not None:
        side.wait_stream(main)

    # ---- linear branch -------------------------------------------------------------------
    with torch.cuda.stream(side) if side is not None else contextlib.nullcontext():
        _run_linear_heads(plan, linear_mode, q, k, v, qb, k_coarse, v_coarse, k_proj_mat, v_proj_mat,
                          proj_segment_len, block_size, q_len, out, lin_tmp, gate, lin_round, save, scale)

    # ---- sparse branch: block pooling -----------------------------------------------------
    if plan.sparse:
        _, _, nq, nkv = block_counts(q_len, kv_len, block_size)
        sp_t = plan.t["sparse"]
        qp, kp, key_args = pool_for_routing(q, k, q_len, kv_len, block_size, sp_t, k_block_sums=k_block_sums,
                                            k_pooled=k_pooled)

    # ---- sparse branch: routing and attention ----------------------------------------------
    if plan.sparse:
        # the routing launch also zeroes the arrival counters of the attention launches below
        n_only = len(plan.sparse_only) if plan.sparse_only else 0
        rows_only, rows_both = bsz * n_only * nq, bsz * (len(plan.both) if plan.both else 0) * nq
        arrivals = torch.empty((rows_only + rows_both,), dtype=torch.int32, device=dev)
        if routing == "gini":
            route, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_GINI, tau_min=tau_min, tau_max=tau_max, heads=sp_t,
                              clear=arrivals, scale=scale, **key_args)
        else:
            ks = _per_head_k(topk, heads)
            route, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=ks, heads=sp_t, clear=arrivals,
                              scale=scale, **key_args)
        if save is not None:
            save.update(route=route)
        # top-k routing fixes every row's visit count on the host: launch exactly those units
        vis_of = (lambda hl: [min(ks[h], nkv) for h in hl]) if routing == "topk" else (lambda hl: None)
        if plan.sparse_only:
            bsa_forward(qb, kb, vb, index=route.index, num=route.num, block_size=block_size, layout="blhd",
                        heads=plan.t["sparse_only"], out=out, lq=q_len, lkv=kv_len, attn_round_bf16=True,
                        visits=vis_of(plan.sparse_only), arrivals=arrivals[:rows_only], scale=scale)
        if plan.both:
            if side is not None:
                main.wait_stream(side)
            bsa_forward(qb, kb, vb, index=route.index, num=route.num, block_size=block_size, layout="blhd",
                        heads=plan.t["both"], out=out, lq=q_len, lkv=kv_len, epilogue=_lib.WA_EPI_FUSE,
                        x=lin_tmp, attn_round_bf16=True, visits=vis_of(plan.both), arrivals=arrivals[rows_only:],
                        scale=scale, **gate.kwargs())
    if side is not None:
        main.wait_stream(side)
    return out if out.dtype == out_dtype else out.to(out_dtype)


_FORK_JOIN: dict = {}


def _fork_join(dev: torch.device, main: torch.cuda.Stream, which: int = 0):
    """The side stream of the linear branch for work issued on ``main`` (default priority), with the
    fork / join events that :func:`_native_split_forward` hands to the library: one set per caller
    stream, so calls on different streams never wait on each other's linear branch. The events are
    recorded once here so that they exist before their handles are passed on. ``which`` = 1: a
    second such set (the one-call backward's dQ stream)."""
    key = (dev.index, main.cuda_stream, which)
    ent = _FORK_JOIN.get(key)
    if ent is None:
        side = torch.cuda.Stream(device=dev)
        fork, join = torch.cuda.Event(), torch.cuda.Event()
        fork.record(side)
        join.record(side)
        ent = (side, fork, join)
        _FORK_JOIN[key] = ent
    return ent


# Whether calls the one-call library path covers take it. False runs the same entry points one
# launch at a time from Python (the same results; a reference point for comparisons).
ONE_CALL = True


def native_split_eligible(q, k, v, plan, routing, linear_mode, k_block_sums=None, k_pooled=None) -> bool:
    """Whether the one-call library path (``wa_hsa_fwd`` / ``wa_hsa_bwd``) covers this call: top-k
    sparse heads and elu1 linear heads, no head in both branches, bf16 q / k / v that the kernels
    read in place, routing from pooled keys."""
    return (ONE_CALL and routing == "topk" and linear_mode == "elu1" and bool(plan.sparse_only) and bool(plan.linear_only)
            and not plan.both and k_block_sums is None and k_pooled is None
            and all(_lib.is_kernel_ready(t) for t in (q, k, v)))


def _native_split_forward(q, k, v, plan, ks, gate, lin_round, block_size, q_len, kv_len, out, save, train=None):
    """:func:`hsa_forward` of top-k sparse heads and elu1 linear heads as one library call
    (``wa_hsa_fwd``): the same entry points with the same arguments as the Python orchestration,
    the linear heads' on a side stream of the caller's stream (see :func:`_fork_join`) that the
    call forks and joins inside (so graph capture records the same two branches). An eager call
    then pays one crossing into the library instead of ~20 (allocations, argument structs,
    launches, events): 171 -> 48 us of host time, and at cfg 2 the eager call went from 195 to
    141 us (GPU-bound).

    ``train`` (a dict): the call also writes what the one-call backward takes back (the sparse
    heads' log-sum-exp, the elu1 state, the unfused linear readout and its gate), stored in it with
    the routing and the linear heads' mode list."""
    dev = q.device
    bsz, _, heads, d = q.shape
    _, _, nq, nkv = block_counts(q_len, kv_len, block_size)
    vis = [min(ks[h], nkv) for h in plan.sparse_only]
    units, n_units = unit_table(bsz, vis, nq, _lib.bsa_default_split(block_size), dev)
    max_visits = max(max(vis), 1)
    n_sp, n_lin = len(plan.sparse_only), len(plan.linear_only)
    index = torch.empty((bsz, heads, nq, nkv), dtype=torch.int32, device=dev)
    num = torch.empty((bsz, heads, nq), dtype=torch.int32, device=dev)
    ws = torch.empty((_lib.lib().wa_hsa_fwd_workspace_bytes(bsz, heads, q_len, kv_len, d, block_size, n_sp, n_lin,
                                                             max_visits),), dtype=torch.uint8, device=dev)
    main = torch.cuda.current_stream(dev)
    side, fork, join = _fork_join(dev, main) if n_sp and n_lin else (None, None, None)
    extra = ()
    if train is not None:
        f32 = dict(dtype=torch.float32, device=dev)
        lin = torch.empty((bsz, q_len, heads, d), **f32)
        train.update(lse=torch.empty((bsz, heads, q_len), **f32), state=torch.empty((bsz, n_lin, d, d), **f32),
                     zsum=torch.empty((bsz, n_lin, d), **f32), lin=lin, gate=torch.empty_like(lin),
                     lin_modes=_lib.head_list([2 if h in plan.linear else 0 for h in range(heads)], dev),
                     index=index, num=num)
        extra = (train["lse"].data_ptr(), train["state"].data_ptr(), train["zsum"].data_ptr(), *_lib.blhd(lin),
                 *_lib.blhd(train["gate"]), train["lin_modes"].data_ptr())
    args = _lib.HsaFwdArgs(*_lib.blhd(q), *_lib.blhd(k), *_lib.blhd(v), *_lib.blhd(out), _lib.dtype_code(out),
                           bsz, heads, q_len, kv_len, d, block_size,
                           *_lib.heads_arg(plan.t["sparse_only"]), _lib.head_list(ks, dev).data_ptr(),
                           units.data_ptr(), n_units, max_visits, index.data_ptr(), num.data_ptr(),
                           *_lib.heads_arg(plan.t["linear_only"]), _lib.ptr(gate.w), _lib.ptr(gate.b),
                           int(gate.pre_bf16), int(gate.out_bf16), int(lin_round), ws.data_ptr(),
                           side.cuda_stream if side is not None else None,
                           fork.cuda_event if fork is not None else None,
                           join.cuda_event if join is not None else None, *extra)
    # the call ends with the caller's stream waiting for the side stream, so later work on it (and
    # the allocator's reuse of the workspace) is ordered after the linear branch
    _lib.call("wa_hsa_fwd", args, main.cuda_stream)
    if save is not None:  # top-k routing has no thresholds (the kernel writes zeros)
        save.update(route=BlockRouting(index=index, num=num, mask=None,
                                       thresholds=torch.zeros((heads,), dtype=torch.float32, device=dev)))


def _run_linear_heads(plan, linear_mode, q, k, v, qb, k_coarse, v_coarse, k_proj_mat, v_proj_mat, proj_segment_len,
                      block_size, q_len, out, lin_tmp, gate, lin_round, save, scale=0.0):
    """Linear-branch heads of :func:`hsa_forward`: linear-only heads straight into ``out`` with the
    gate applied, heads that also run the sparse branch into ``lin_tmp``."""
    if plan.linear:
        if linear_mode == "lowrank":
            if k_coarse is None:
                kc = _compress(k, k_proj_mat, segment_len=proj_segment_len, block_size=block_size, layout="blhd")
                vc = _compress(v, v_proj_mat, segment_len=proj_segment_len, block_size=block_size, layout="blhd")
            else:
                kc, vc = k_coarse, v_coarse
            kcb, vcb = _lib.kernel_ready(kc), _lib.kernel_ready(vc)
            if save is not None:
                save.update(kc=kc, vc=vc)
            # The dense launch over the compressed keys tiles its queries freely: 128-query units at
            # D = 128 walk the same 64-key steps in the same order (the same arithmetic per query)
            # in half the units of the routed block size 64 (one round of units instead of ~1.7).
            dense_block = 128 if qb.shape[-1] == 128 else block_size
            if plan.both:
                bsa_forward(qb, kcb, vcb, index=None, num=None, block_size=dense_block, layout="blhd",
                            heads=plan.t["both"], out=lin_tmp, lq=q_len, scale=scale)
            if plan.linear_only:
                bsa_forward(qb, kcb, vcb, index=None, num=None, block_size=dense_block, layout="blhd",
                            heads=plan.t["linear_only"], out=out, lq=q_len, epilogue=_lib.WA_EPI_GATED,
                            attn_round_bf16=lin_round, scale=scale, **gate.kwargs())
        else:
            if plan.both:
                s_b, z_b = elu1_state(k, v, plan.t["both"])
                elu1_readout(q, s_b, z_b, plan.t["both"], lin_tmp)
            if plan.linear_only:
                s_l, z_l = elu1_state(k, v, plan.t["linear_only"])
                elu1_readout(q, s_l, z_l, plan.t["linear_only"], out, epilogue=_lib.WA_EPI_GATED,
                             lin_round_bf16=lin_round, **gate.kwargs())


def hsa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    k_coarse: Optional[torch.Tensor] = None,
    v_coarse: Optional[torch.Tensor] = None,
    k_proj_mat: torch.Tensor,
    v_proj_mat: torch.Tensor,
    gate_lin: Optional[nn.Module] = None,
    block_size: int = 64,
    tau_min: float = 0.35,
    tau_max: float = 1.0,
    proj_segment_len: int = 1560,
    backend: str = "auto",
    routing: str = "gini",
    topk=None,
    head_modes: Optional[Sequence[str]] = None,
    linear_mode: str = "lowrank",
    k_block_sums: Optional[torch.Tensor] = None,
    k_pooled: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Run HSA over ``[B, L, H, D]`` queries, keys and values (``attention.py:153-259``).

    ``k_coarse`` / ``v_coarse`` supply an already-compressed view of the same KV range (the
    decoding loop's compressed cache); when omitted the compression runs here.

    ``k_block_sums`` (no reference counterpart): the fp32 key block sums that
    :func:`worldattention_amd.hsa.kvcache.kv_append` keeps beside a KV cache whose first
    ``k.shape[1]`` tokens are ``k``; ``k_pooled``: fp32 block means of exactly ``k`` (the routing
    pool of ``routing.py:45-61``). With either, routing pools only the queries; the result is
    identical to pooling ``k``.

    Head dims other than 64 and 128 (the reference's functional API takes any) run padded to the
    next of them: queries, values, coarse caches and the gate layer with zeros, keys with
    ``PAD_KEY_VALUE``, routing and both softmax branches at the original ``head_dim ** -0.5``; the
    padding changes no logit, no elu(x)+1 feature and no gate of a real channel, and the output is
    cut back to ``head_dim`` (gradients flow through the padding to the unpadded tensors).
    """
    if (k_coarse is None) != (v_coarse is None):
        raise ValueError("k_coarse and v_coarse must be provided together")
    if k_block_sums is not None and k_pooled is not None:
        raise ValueError("pass k_block_sums or k_pooled, not both")
    bsz, q_len, heads, head_dim = q.shape
    kv_len = k.shape[1]
    if q_len <= 0 or kv_len <= 0:
        raise ValueError("q_len and kv_len must be positive")
    if k_coarse is not None:
        if k_coarse.shape[0] != bsz or tuple(k_coarse.shape[2:]) != (heads, head_dim):
            raise ValueError(
                f"expected k_coarse shaped [B, Lc, {heads}, {head_dim}], got {tuple(k_coarse.shape)}")
        if v_coarse.shape != k_coarse.shape:
            raise ValueError("v_coarse must have the same shape as k_coarse")
    resolve_backend(backend)
    needs_grad = torch.is_grad_enabled() and (
        any(t is not None and t.requires_grad for t in (q, k, v, k_coarse, v_coarse, k_proj_mat, v_proj_mat))
        or (gate_lin is not None and any(p.requires_grad for p in gate_lin.parameters())))
    dp = padded_head_dim(head_dim)
    qx, kx, vx, scale = q, k, v, 0.0
    if dp != head_dim:
        scale = head_dim ** -0.5
        qx, kx, vx = _pad_channels(q, dp), _pad_channels(k, dp, PAD_KEY_VALUE), _pad_channels(v, dp)
        k_coarse, v_coarse = _pad_channels(k_coarse, dp), _pad_channels(v_coarse, dp)
        k_block_sums, k_pooled = _pad_channels(k_block_sums, dp), _pad_channels(k_pooled, dp)
        gate_lin = _PaddedGate(gate_lin, dp) if gate_lin is not None else None
    cfg = dict(k_coarse=k_coarse, v_coarse=v_coarse, k_proj_mat=k_proj_mat, v_proj_mat=v_proj_mat,
               gate_lin=gate_lin, block_size=block_size, tau_min=tau_min, tau_max=tau_max,
               proj_segment_len=proj_segment_len, routing=routing, topk=topk, head_modes=head_modes,
               linear_mode=linear_mode, k_block_sums=k_block_sums, k_pooled=k_pooled, scale=scale)
    if needs_grad:
        from ._autograd import hsa_attention_autograd
        output = hsa_attention_autograd(qx, kx, vx, **cfg)
    else:
        output = hsa_forward(qx, kx, vx, **cfg)
    if dp != head_dim:
        output = output[..., :head_dim].contiguous()
    if distill.distill_enabled() and torch.is_grad_enabled():
        distill.record_against_dense(output, q, k, v)
    return output


class _PaddedGate:
    """A gate layer's weight ``[D, D]`` and bias ``[D]`` zero-padded to ``dp`` channels (padding
    channels get sigmoid(0) and gate nothing: their linear-branch output is zero)."""

    def __init__(self, gate_lin: nn.Module, dp: int):
        w = gate_lin.weight
        self.weight = torch.nn.functional.pad(w, (0, dp - w.shape[1], 0, dp - w.shape[0]))
        b = getattr(gate_lin, "bias", None)
        self.bias = _pad_channels(b, dp) if b is not None else None


class HSAAttention(nn.Module):
    """Hybrid Sparse Attention over a KV window (``attention.py:262-380``).

    Owns the low-rank projections ``k_proj_mat`` / ``v_proj_mat`` (``[ceil(seg/block), seg]`` bf16)
    and the fusion gate ``gate_lin`` (``Linear(D, D)``), all zero until loaded or initialized, so
    state dicts are interchangeable with the reference's.

    ``block_size`` may be 64 (reference) or 128 (north-star configs). The extension keywords
    ``routing``, ``topk``, ``head_modes`` and ``linear_mode`` are forwarded to :func:`hsa_attention`.
    """

    def __init__(self, num_heads: int, head_dim: int, block_size: int = 64, tau_min: float = 0.35,
                 tau_max: float = 1.0, proj_segment_len: int = 1560, backend: str = "auto", *,
                 routing: str = "gini", topk=None, head_modes: Optional[Sequence[str]] = None,
                 linear_mode: str = "lowrank"):
        super().__init__()
        if block_size not in SUPPORTED_BLOCK_SIZES:
            raise ValueError(f"the sparse-branch kernels are specialized for block_size in {SUPPORTED_BLOCK_SIZES}")
        if proj_segment_len <= 0:
            raise ValueError(f"proj_segment_len must be positive, got {proj_segment_len}")
        if routing not in _ROUTING_MODES:
            raise ValueError(f"routing must be one of {_ROUTING_MODES}")
        if linear_mode not in _LINEAR_MODES:
            raise ValueError(f"linear_mode must be one of {_LINEAR_MODES}")
        if head_modes is not None and (len(head_modes) != num_heads or any(m not in _HEAD_MODES for m in head_modes)):
            raise ValueError(f"head_modes must list one of {_HEAD_MODES} per head")
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.tau_min = tau_min
        self.tau_max = tau_max
        self.proj_segment_len = proj_segment_len
        self.proj_rank = math.ceil(proj_segment_len / block_size)
        self.backend = backend
        self.routing = routing
        self.topk = topk
        self.head_modes = list(head_modes) if head_modes is not None else None
        self.linear_mode = linear_mode
        self.k_proj_mat = nn.Parameter(torch.zeros((self.proj_rank, proj_segment_len), dtype=torch.bfloat16))
        self.v_proj_mat = nn.Parameter(torch.zeros((self.proj_rank, proj_segment_len), dtype=torch.bfloat16))
        self.gate_lin = nn.Linear(head_dim, head_dim, bias=True)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """Return every HSA parameter to its zero placeholder (``attention.py:318-329``)."""
        with torch.no_grad():
            self.k_proj_mat.zero_()
            self.v_proj_mat.zero_()
            self.gate_lin.weight.zero_()
            self.gate_lin.bias.zero_()

    def coarse_cache_size(self, kv_cache_size: int) -> int:
        """Compressed slots needed to mirror a token cache of ``kv_cache_size`` (``:331-335``)."""
        if kv_cache_size <= 0:
            return 0
        return math.ceil(kv_cache_size / self.proj_segment_len) * self.proj_rank

    def token_range_to_coarse(self, start_index: int, end_index: int) -> tuple[int, int]:
        """Map a segment-aligned token range onto compressed-cache slots (``:337-347``)."""
        if start_index % self.proj_segment_len != 0 or end_index % self.proj_segment_len != 0:
            raise ValueError(
                "coarse-cache access requires segment-aligned token indices, got "
                f"start={start_index}, end={end_index}, proj_segment_len={self.proj_segment_len}")
        return ((start_index // self.proj_segment_len) * self.proj_rank,
                (end_index // self.proj_segment_len) * self.proj_rank)

    def compress_kv_cache(self, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Compress ``[B, L, H, D]`` keys and values for the compressed cache (``:349-361``)."""
        if k.shape != v.shape:
            raise ValueError(f"k and v must match, got {tuple(k.shape)} and {tuple(v.shape)}")
        if k.ndim != 4:
            raise ValueError(f"expected [B, L, H, D] tensors, got ndim={k.ndim}")
        if torch.is_grad_enabled() and (self.k_proj_mat.requires_grad or k.requires_grad or v.requires_grad):
            from ._autograd import compress_autograd
            return (compress_autograd(k, self.k_proj_mat, self.proj_segment_len, self.block_size),
                    compress_autograd(v, self.v_proj_mat, self.proj_segment_len, self.block_size))
        return (_compress(k, self.k_proj_mat, segment_len=self.proj_segment_len, block_size=self.block_size,
                          layout="blhd"),
                _compress(v, self.v_proj_mat, segment_len=self.proj_segment_len, block_size=self.block_size,
                          layout="blhd"))

    def forward(self, q, k, v, k_coarse=None, v_coarse=None, *, k_block_sums=None, k_pooled=None) -> torch.Tensor:
        return hsa_attention(
            q, k, v, k_coarse=k_coarse, v_coarse=v_coarse, k_proj_mat=self.k_proj_mat,
            v_proj_mat=self.v_proj_mat, gate_lin=self.gate_lin, block_size=self.block_size,
            tau_min=self.tau_min, tau_max=self.tau_max, proj_segment_len=self.proj_segment_len,
            backend=self.backend, routing=self.routing, topk=self.topk, head_modes=self.head_modes,
            linear_mode=self.linear_mode, k_block_sums=k_block_sums, k_pooled=k_pooled)
