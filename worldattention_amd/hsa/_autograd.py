"""Differentiable HSA on the GPU (the training path of ``wan/modules/hsa/attention.py:153-259``).

The reference differentiates its torch path with autograd (and the Triton kernels with
``block_sparse_triton.py:353-368``). Here the forward keeps the two branch outputs and the gate
apart (fp32), fuses them with ``wa_hsa_fuse_fwd``, and the backward runs
``wa_hsa_fuse_bwd`` -> ``wa_bsa_bwd`` (sparse branch) -> ``wa_elu1_bwd`` or a dense ``wa_bsa_bwd``
over the compressed keys (linear branch), all accumulating into fp32 gradient buffers. Routing is
not differentiated, as in the reference (its ``argsort`` / thresholds carry no gradient).
"""
from __future__ import annotations


import torch

from .. import _lib
from ._bwd import bsa_backward
from .attention import _fork_join
from .block_sparse import bsa_forward
from .routing import _route, block_counts, pool_for_routing

__all__ = ["hsa_attention_autograd", "compress_autograd", "elu1_backward", "fuse_forward", "fuse_backward"]

MODE_SPARSE, MODE_LINEAR = 1, 2


def _blhd(t):
    return _lib.blhd(t) if t is not None else (None, 0, 0, 0)


def _fuse_args(q, sparse, lin, modes_t, gate, spec, *, out=None, dout=None, dlin=None, dq=None, dgw=None, dgb=None,
               ws=None, attn_round, lin_round, dq_accumulate=True):
    bsz, length, heads, d = q.shape
    return _lib.HsaFuseArgs(
        *_lib.blhd(q), *_blhd(sparse), *_blhd(lin), modes_t.data_ptr(),
        *_blhd(out), _lib.dtype_code(out) if out is not None else 0,
        *_blhd(gate), _lib.ptr(spec.w), _lib.ptr(spec.b),
        int(spec.pre_bf16), int(spec.out_bf16), int(attn_round), int(lin_round),
        *_blhd(dout), _lib.dtype_code(dout) if dout is not None else 0,
        *_blhd(dlin), *_blhd(dq), int(dq_accumulate),
        _lib.ptr(dgw), _lib.ptr(dgb), _lib.ptr(ws),
        bsz, heads, length, d)


def fuse_forward(q, sparse, lin, modes_t, gate, spec, out, *, attn_round, lin_round):
    """``out = [sparse] + [gate * lin]`` per head mode (``wa_hsa_fuse_fwd``); fills ``gate``."""
    dev = _lib.require_gpu(q, out)
    args = _fuse_args(q, sparse, lin, modes_t, gate, spec, out=out, attn_round=attn_round, lin_round=lin_round)
    _lib.call("wa_hsa_fuse_fwd", args, _lib.stream_ptr(dev))


def fuse_backward(q, lin, modes_t, gate, spec, dout, dlin, dq, *, lin_round, dq_accumulate=True):
    """``dlin = dout * gate``; adds the gate path into ``dq`` (writes it with ``dq_accumulate=False``);
    returns ``(dW, db)`` or ``(None, None)``."""
    dev = _lib.require_gpu(q, dout)
    bsz, length, heads, d = q.shape
    dgw = dgb = ws = None
    if spec.w is not None:
        dgw = torch.empty((d, d), dtype=torch.float32, device=dev)
        dgb = torch.empty((d,), dtype=torch.float32, device=dev)
        ws = torch.empty((_lib.lib().wa_hsa_fuse_bwd_workspace_bytes(bsz, heads, length, d),), dtype=torch.uint8,
                         device=dev)
    args = _fuse_args(q, None, lin, modes_t, gate, spec, dout=dout, dlin=dlin, dq=dq, dgw=dgw, dgb=dgb, ws=ws,
                      attn_round=False, lin_round=lin_round, dq_accumulate=dq_accumulate)
    _lib.call("wa_hsa_fuse_bwd", args, _lib.stream_ptr(dev))
    return dgw, dgb


def elu1_backward(q, k, v, dout, state, zsum, heads_t, dq, dk, dv, *, dq_accumulate=True, kv_accumulate=True):
    """Adds the elu(x)+1 branch's gradients into fp32 ``dq``, ``dk``, ``dv`` (``wa_elu1_bwd``); with
    an ``*_accumulate`` flag off the gradient is written instead (then ``dk`` / ``dv`` may be bf16)."""
    dev = _lib.require_gpu(q, k, v, dout)
    if heads_t.numel() == 0:
        return
    if k.dtype != v.dtype:
        v = v.to(k.dtype)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    bsz, lq, heads, d = q.shape
    lkv = k.shape[1]
    n = heads_t.numel()
    ws = torch.empty((_lib.lib().wa_elu1_bwd_workspace_bytes(bsz, n, lq, d),), dtype=torch.uint8, device=dev)
    args = _lib.Elu1BwdArgs(
        *_lib.blhd(q), _lib.dtype_code(q), *_lib.blhd(k), *_lib.blhd(v), _lib.dtype_code(k),
        *_lib.blhd(dout), _lib.dtype_code(dout), state.data_ptr(), zsum.data_ptr(),
        *_lib.blhd(dq), int(dq_accumulate), *_lib.blhd(dk), int(kv_accumulate), *_lib.blhd(dv), int(kv_accumulate),
        *_lib.heads_arg(heads_t), bsz, heads, lq, lkv, d, ws.data_ptr(), _lib.dtype_code(dk))
    _lib.call("wa_elu1_bwd", args, _lib.stream_ptr(dev))


# ----------------------------------------------------------------------------------------------
# low-rank compression (attention.py:64-110) under autograd
# ----------------------------------------------------------------------------------------------
def _compress_backward(grad, x, proj, segment_len, block_size, dx=None):
    """Gradients of ``out_seg = E[:r, :len] @ x_seg`` per segment (``wa_compress_kv_bwd``):
    ``dx_seg = E^T dout_seg`` and ``dE[:r, :len] = sum_{b, h} dout_seg x_seg^T``, fp32, for a
    ``[B, L, H, D]`` x and a ``[B, Lc, H, D]`` gradient. ``dx`` (optional): an fp32 ``[B, L, H, D]``
    tensor with unit last stride that the x gradient is added to; otherwise a new one is returned.
    Returns ``(dx, dproj)``, dproj fp32 of the projection's shape."""
    dev = _lib.require_gpu(x, proj)
    bsz, length, heads, d = x.shape
    seg = segment_len if segment_len > 0 else length
    g = grad if grad.dtype == torch.float32 and grad.is_contiguous() else grad.float().contiguous()
    xs = x if x.dtype in (torch.float32, torch.bfloat16) and x.is_contiguous() else (
        x.contiguous() if x.dtype in (torch.float32, torch.bfloat16) else x.float().contiguous())
    pj = proj if proj.dtype in (torch.float32, torch.bfloat16) else proj.float()
    pj = pj.contiguous()
    accumulate = dx is not None
    if dx is None:
        dx = torch.empty((bsz, length, heads, d), dtype=torch.float32, device=dev)
    elif dx.dtype != torch.float32 or tuple(dx.shape) != (bsz, length, heads, d) or dx.stride(-1) != 1:
        raise ValueError(f"dx must be float32 {(bsz, length, heads, d)} with unit last stride")
    dproj = torch.empty(pj.shape, dtype=torch.float32, device=dev)
    ws = torch.empty((max(_lib.lib().wa_compress_kv_bwd_workspace_bytes(length, pj.shape[0], seg, block_size), 4),),
                     dtype=torch.uint8, device=dev)
    args = _lib.CompressBwdArgs(*_lib.blhd(g), *_lib.blhd(xs), _lib.dtype_code(xs), pj.data_ptr(),
                                _lib.dtype_code(pj), pj.shape[0], pj.shape[1], bsz, length, heads, d, seg,
                                block_size, *_lib.blhd(dx), int(accumulate), dproj.data_ptr(), 0, ws.data_ptr())
    _lib.call("wa_compress_kv_bwd", args, _lib.stream_ptr(dev))
    return dx, dproj


class _Compress(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, proj, segment_len, block_size):
        from .attention import _compress
        ctx.save_for_backward(x, proj)
        ctx.cfg = (segment_len, block_size)
        return _compress(x, proj, segment_len=segment_len, block_size=block_size, layout="blhd")

    @staticmethod
    def backward(ctx, grad):
        x, proj = ctx.saved_tensors
        dx, dproj = _compress_backward(grad, x, proj, *ctx.cfg)
        return dx.to(x.dtype), dproj.to(proj.dtype), None, None


def compress_autograd(x, proj, segment_len, block_size):
    """Differentiable ``compress_kv`` of a ``[B, L, H, D]`` tensor (``attention.py:64-110``)."""
    return _Compress.apply(x, proj, segment_len, block_size)


# ----------------------------------------------------------------------------------------------
# hsa_attention under autograd
# ----------------------------------------------------------------------------------------------
class _GateParams:
    """The gate layer's weight and bias as the autograd function receives them."""
    __slots__ = ("weight", "bias")

    def __init__(self, weight, bias):
        self.weight, self.bias = weight, bias


class _HSA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, k_coarse, v_coarse, k_proj_mat, v_proj_mat, gate_w, gate_b, cfg):
        from .attention import (GateSpec, _compress, _native_split_forward, _per_head_k, elu1_readout, elu1_state,
                                head_plan, native_split_eligible)

        block_size, routing, topk, linear_mode = cfg["block_size"], cfg["routing"], cfg["topk"], cfg["linear_mode"]
        bsz, q_len, heads, d = q.shape
        kv_len = k.shape[1]
        dev = _lib.require_gpu(q, k, v, k_coarse, v_coarse)
        plan = head_plan(heads, cfg["head_modes"], dev)
        if linear_mode == "lowrank":
            comp = v_coarse.dtype if v_coarse is not None else v.dtype
        else:
            comp = v.dtype
        if comp not in (torch.float32, torch.bfloat16):
            comp = torch.float32

        spec = GateSpec(_GateParams(gate_w, gate_b) if gate_w is not None else None, comp)
        lin_round = comp == torch.bfloat16
        modes = [(MODE_SPARSE if h in plan.sparse else 0) | (MODE_LINEAR if h in plan.linear else 0)
                 for h in range(heads)]
        modes_t = _lib.head_list(modes, dev)

        ctx.cfg = cfg
        ctx.has_coarse = k_coarse is not None
        ctx.dtypes = tuple(t.dtype if t is not None else None
                           for t in (q, k, v, k_coarse, v_coarse, k_proj_mat, v_proj_mat, gate_w, gate_b))
        scale = cfg.get("scale", 0.0)
        if not scale and native_split_eligible(q, k, v, plan, routing, linear_mode, cfg["k_block_sums"],
                                               cfg["k_pooled"]):
            # one library call (wa_hsa_fwd with its training outputs); the backward is wa_hsa_bwd
            out = torch.empty((bsz, q_len, heads, d), dtype=comp, device=dev)
            tr = {}
            _native_split_forward(q, k, v, plan, _per_head_k(topk, heads), spec, lin_round, block_size, q_len,
                                  kv_len, out, None, train=tr)
            ctx.native = True
            ctx.extra = dict(plan=plan, spec=spec, lin_round=lin_round, lin_modes=tr["lin_modes"])
            ctx.save_for_backward(q, k, v, out, tr["lse"], tr["state"], tr["zsum"], tr["lin"], tr["gate"],
                                  tr["index"], tr["num"])
            return out if out.dtype == q.dtype else out.to(q.dtype)
        ctx.native = False

        qb, kb, vb = _lib.kernel_ready(q), _lib.kernel_ready(k), _lib.kernel_ready(v)
        f32 = dict(dtype=torch.float32, device=dev)
        out = torch.empty((bsz, q_len, heads, d), dtype=comp, device=dev)
        # Split heads (each head in one branch): a sparse head's output is its attention rounded to
        # bf16, which the sparse kernel writes straight into `out`; that output is also the O whose
        # row sums with dO the backward takes (as the reference's backward takes its bf16 output).
        # Heads with both branches keep the fp32 sparse output for the fusion.
        split = not plan.both
        sparse = torch.empty((bsz, q_len, heads, d), **f32) if plan.sparse and not split else None
        lin = torch.empty((bsz, q_len, heads, d), **f32) if plan.linear else None
        gate = torch.empty((bsz, q_len, heads, d), **f32) if plan.linear else None
        saved = dict(plan=plan, spec=spec, modes_t=modes_t, lin_round=lin_round, comp=comp)
        lse_s = lse_l = kc = vc = kcb = vcb = state = zsum = route = None

        if plan.linear:
            lt = plan.t["linear"]
            if linear_mode == "elu1":
                state, zsum = elu1_state(k, v, lt)
                elu1_readout(q, state, zsum, lt, lin)
            else:
                if k_coarse is None:
                    kc = _compress(k, k_proj_mat, segment_len=cfg["proj_segment_len"], block_size=block_size,
                                   layout="blhd")
                    vc = _compress(v, v_proj_mat, segment_len=cfg["proj_segment_len"], block_size=block_size,
                                   layout="blhd")
                else:
                    kc, vc = k_coarse, v_coarse
                kcb, vcb = _lib.kernel_ready(kc), _lib.kernel_ready(vc)
                _, lse_l = bsa_forward(qb, kcb, vcb, index=None, num=None, block_size=block_size, layout="blhd",
                                       heads=lt, out=lin, lq=q_len, want_lse=True, scale=scale)
        if plan.sparse:
            _, _, nq, nkv = block_counts(q_len, kv_len, block_size)
            st = plan.t["sparse"]
            qp, kp, key_args = pool_for_routing(q, k, q_len, kv_len, block_size, st,
                                                k_block_sums=cfg["k_block_sums"], k_pooled=cfg["k_pooled"])
            visits = None
            # the routing launch also zeroes the arrival counters of the sparse launch
            arrivals = torch.empty((bsz * len(plan.sparse) * nq,), dtype=torch.int32, device=dev)
            if routing == "gini":
                route, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_GINI, tau_min=cfg["tau_min"],
                                  tau_max=cfg["tau_max"], heads=st, clear=arrivals, scale=scale, **key_args)
            else:
                ks = _per_head_k(topk, heads)
                route, _ = _route(None, qp, kp, mode=_lib.WA_ROUTE_TOPK, head_k=ks, heads=st, clear=arrivals,
                                  scale=scale, **key_args)
                visits = [min(ks[h], nkv) for h in plan.sparse]
            _, lse_s = bsa_forward(qb, kb, vb, index=route.index, num=route.num, block_size=block_size,
                                   layout="blhd", heads=st, out=out if split else sparse, lq=q_len, lkv=kv_len,
                                   want_lse=True, visits=visits, attn_round_bf16=split, arrivals=arrivals,
                                   scale=scale)
        if split:
            if plan.linear:  # gate and gated output of the linear heads; the sparse heads are written
                lin_modes = _lib.head_list([MODE_LINEAR if h in plan.linear else 0 for h in range(heads)], dev)
                fuse_forward(qb, None, lin, lin_modes, gate, spec, out, attn_round=True, lin_round=lin_round)
        else:
            fuse_forward(qb, sparse, lin, modes_t, gate, spec, out, attn_round=True, lin_round=lin_round)
        sparse_o = out if split else sparse  # the sparse heads' O for the backward

        ctx.extra = saved
        ctx.save_for_backward(q, k, v, qb, kb, vb, sparse_o if plan.sparse else None, lin, gate, lse_s, lse_l, kc,
                              vc, kcb, vcb, state, zsum,
                              route.index if route is not None else None,
                              route.num if route is not None else None, k_proj_mat, v_proj_mat)
        return out if out.dtype == q.dtype else out.to(q.dtype)

    @staticmethod
    def backward(ctx, dout):
        if ctx.native:
            return _native_split_backward(ctx, dout)
        (q, k, v, qb, kb, vb, sparse, lin, gate, lse_s, lse_l, kc, vc, kcb, vcb, state, zsum, index, num,
         k_proj_mat, v_proj_mat) = ctx.saved_tensors
        cfg, ex = ctx.cfg, ctx.extra
        plan, spec = ex["plan"], ex["spec"]
        dev = q.device
        bsz, q_len, heads, d = q.shape
        kv_len = k.shape[1]
        block_size = cfg["block_size"]
        dout = dout if dout.stride(-1) == 1 and dout.dtype in (torch.float32, torch.bfloat16) else dout.float().contiguous()
        f32 = dict(dtype=torch.float32, device=dev)
        # Split heads (each head in exactly one branch, elu1 linear heads): every gradient element
        # has one first writer (gate for dq of linear heads, the sparse backward for its heads,
        # elu1 for dk / dv of linear heads), which writes instead of adding, so the buffers need no
        # zero fill. Otherwise they start at zero and every kernel accumulates.
        fresh = (not plan.both and len(plan.sparse_only) + len(plan.linear_only) == heads
                 and (not plan.linear or cfg["linear_mode"] == "elu1"))
        alloc = torch.empty if fresh else torch.zeros
        dq = alloc((bsz, q_len, heads, d), **f32)
        # written once in their final type when that is bf16 (no fp32 buffer, no cast pass)
        kd, vd = ctx.dtypes[1], ctx.dtypes[2]
        kv_dt = torch.bfloat16 if fresh and kd == vd == torch.bfloat16 else torch.float32
        dk = alloc((bsz, kv_len, heads, d), dtype=kv_dt, device=dev)
        dv = alloc((bsz, kv_len, heads, d), dtype=kv_dt, device=dev)
        dgw = dgb = dkc = dvc = dEk = dEv = None
        if plan.linear:
            dlin = torch.empty((bsz, q_len, heads, d), **f32)
            dgw, dgb = fuse_backward(qb, lin, ex["modes_t"], gate, spec, dout, dlin, dq, lin_round=ex["lin_round"],
                                     dq_accumulate=not fresh)
        if plan.sparse:
            bsa_backward(qb, kb, vb, sparse, lse_s, dout, index=index, num=num, block_size=block_size,
                         layout="blhd", heads=plan.t["sparse"], lq=q_len, lkv=kv_len, dq=dq, dk=dk, dv=dv,
                         accumulate=not fresh, scale=cfg.get("scale", 0.0))
        if plan.linear:
            lt = plan.t["linear"]
            if cfg["linear_mode"] == "elu1":
                elu1_backward(q, k, v, dlin, state, zsum, lt, dq, dk, dv, dq_accumulate=True,
                              kv_accumulate=not fresh)
            else:
                lc = kcb.shape[1]
                dkc = torch.zeros((bsz, lc, heads, d), **f32)
                dvc = torch.zeros((bsz, lc, heads, d), **f32)
                bsa_backward(qb, kcb, vcb, lin, lse_l, dlin, index=None, num=None, block_size=block_size,
                             layout="blhd", heads=lt, lq=q_len, lkv=lc, dq=dq, dk=dkc, dv=dvc, accumulate=True,
                             scale=cfg.get("scale", 0.0))
                if not ctx.has_coarse:
                    _, dEk = _compress_backward(dkc, k, k_proj_mat, cfg["proj_segment_len"], block_size, dx=dk)
                    _, dEv = _compress_backward(dvc, v, v_proj_mat, cfg["proj_segment_len"], block_size, dx=dv)
        qd, kd, vd, kcd, vcd, ekd, evd, gwd, gbd = ctx.dtypes

        def cast(t, dt):
            return None if t is None or dt is None else t.to(dt)
        return (cast(dq, qd), cast(dk, kd), cast(dv, vd),
                cast(dkc, kcd) if ctx.has_coarse else None, cast(dvc, vcd) if ctx.has_coarse else None,
                cast(dEk, ekd), cast(dEv, evd), cast(dgw, gwd), cast(dgb, gbd), None)


# The one-call backward runs the sparse heads' dQ pass on a stream of its own, beside their dK/dV
# pass and the linear heads (False: after the transposed lists, on the caller's stream).
DQ_STREAM = True


def _native_split_backward(ctx, dout):
    """The backward of the one-call forward in one library call (``wa_hsa_bwd``): the sparse heads'
    ``wa_bsa_bwd`` on the caller's stream, the linear heads' gate and elu1 backward on its side
    stream (:func:`_fork_join`); dq, dk and dv are written once, in bf16 when their inputs are."""
    q, k, v, out, lse, state, zsum, lin, gate, index, num = ctx.saved_tensors
    cfg, ex = ctx.cfg, ctx.extra
    plan, spec = ex["plan"], ex["spec"]
    dev = q.device
    bsz, q_len, heads, d = q.shape
    kv_len = k.shape[1]
    dout = dout if dout.stride(-1) == 1 and dout.dtype in (torch.float32, torch.bfloat16) else dout.float().contiguous()
    qd, kd, vd = ctx.dtypes[:3]
    dq = torch.empty(q.shape, dtype=torch.bfloat16 if qd == torch.bfloat16 else torch.float32, device=dev)
    kv_dt = torch.bfloat16 if kd == vd == torch.bfloat16 else torch.float32
    dk = torch.empty(k.shape, dtype=kv_dt, device=dev)
    dv = torch.empty(v.shape, dtype=kv_dt, device=dev)
    dgw = dgb = None
    if spec.w is not None:
        dgw = torch.empty((d, d), dtype=torch.float32, device=dev)
        dgb = torch.empty((d,), dtype=torch.float32, device=dev)
    n_sp, n_lin = len(plan.sparse_only), len(plan.linear_only)
    block_size = cfg["block_size"]
    ws = torch.empty((_lib.lib().wa_hsa_bwd_workspace_bytes(bsz, heads, q_len, kv_len, d, block_size, n_sp, n_lin),),
                     dtype=torch.uint8, device=dev)
    main = torch.cuda.current_stream(dev)
    side, fork, join = _fork_join(dev, main)
    dqs, dq_fork, dq_join = _fork_join(dev, main, 1) if DQ_STREAM else (None, None, None)
    args = _lib.HsaBwdArgs(
        *_lib.blhd(q), *_lib.blhd(k), *_lib.blhd(v), *_lib.blhd(out), _lib.dtype_code(out),
        *_lib.blhd(dout), _lib.dtype_code(dout),
        bsz, heads, q_len, kv_len, d, block_size,
        *_lib.heads_arg(plan.t["sparse_only"]), index.data_ptr(), num.data_ptr(), lse.data_ptr(),
        *_lib.heads_arg(plan.t["linear_only"]), ex["lin_modes"].data_ptr(), *_lib.blhd(lin), *_lib.blhd(gate),
        state.data_ptr(), zsum.data_ptr(),
        _lib.ptr(spec.w), _lib.ptr(spec.b), int(spec.pre_bf16), int(spec.out_bf16), int(ex["lin_round"]),
        *_lib.blhd(dq), _lib.dtype_code(dq), *_lib.blhd(dk), *_lib.blhd(dv), _lib.dtype_code(dk),
        _lib.ptr(dgw), _lib.ptr(dgb), ws.data_ptr(), side.cuda_stream, fork.cuda_event, join.cuda_event,
        dqs.cuda_stream if dqs is not None else None, dq_fork.cuda_event if dq_fork is not None else None,
        dq_join.cuda_event if dq_join is not None else None)
    _lib.call("wa_hsa_bwd", args, main.cuda_stream)
    qd, kd, vd, kcd, vcd, ekd, evd, gwd, gbd = ctx.dtypes

    def cast(t, dt):
        return None if t is None or dt is None else t.to(dt)
    return (cast(dq, qd), cast(dk, kd), cast(dv, vd), None, None, None, None, cast(dgw, gwd), cast(dgb, gbd), None)


def hsa_attention_autograd(q, k, v, *, k_coarse, v_coarse, k_proj_mat, v_proj_mat, gate_lin, block_size, tau_min,
                           tau_max, proj_segment_len, routing, topk, head_modes, linear_mode, k_block_sums=None,
                           k_pooled=None, scale=0.0):
    """Differentiable :func:`hsa_attention` (q, k, v, coarse caches, projections and gate)."""
    if block_size not in (64, 128) or q.shape[-1] not in (64, 128):
        raise ValueError("block_size and head_dim must each be 64 or 128 for the gfx950 kernels")
    gate_w = gate_lin.weight if gate_lin is not None else None
    gate_b = getattr(gate_lin, "bias", None) if gate_lin is not None else None
    cfg = dict(block_size=block_size, tau_min=tau_min, tau_max=tau_max, proj_segment_len=proj_segment_len,
               routing=routing, topk=topk, head_modes=head_modes, linear_mode=linear_mode,
               k_block_sums=k_block_sums, k_pooled=k_pooled, scale=scale)
    return _HSA.apply(q, k, v, k_coarse, v_coarse, k_proj_mat, v_proj_mat, gate_w, gate_b, cfg)
