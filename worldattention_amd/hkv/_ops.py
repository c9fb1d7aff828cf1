"""Tensor-level wrappers of the HKV entry points of ``libworldattention_amd`` (no CPU path).

``segment_means`` -> ``wa_hkv_page_summary``, ``score_topk`` -> ``wa_hkv_score_topk``,
``rotate_temporal`` -> ``wa_rerope``, ``copy_pages`` -> ``wa_hkv_gather_async`` /
``wa_hkv_store_async``. Every launch goes on the current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from .. import _lib

__all__ = ["segment_means", "score_topk", "rotate_temporal", "copy_pages", "factor_table", "PageCopy"]


def factor_table(temporal_freqs: torch.Tensor, new_ids: torch.Tensor, orig_ids: torch.Tensor,
                 device: torch.device) -> torch.Tensor:
    """``freqs[new] * conj(freqs[orig])`` (positions clamped to the table) as complex64 on ``device``,
    viewed as float pairs ``[n, n_temporal, 2]``. The product is taken in the table's own precision
    and then narrowed to complex64, the order of ``pipeline/hkv/rope.py:35-40, 43-47``."""
    top = temporal_freqs.shape[0] - 1
    new = new_ids.to(temporal_freqs.device).clamp(0, top)
    orig = orig_ids.to(temporal_freqs.device).clamp(0, top)
    f = (temporal_freqs[new] * temporal_freqs[orig].conj()).to(torch.complex64)
    return torch.view_as_real(f.to(device)).contiguous()


def segment_means(x: torch.Tensor, *, heads: int, head_dim: int, seg_tokens: Optional[int] = None,
                  spans: Optional[Sequence[Tuple[int, int]]] = None, factors: Optional[torch.Tensor] = None,
                  row_tokens: int = 1, normalize: bool = False) -> torch.Tensor:
    """fp32 ``[n_seg, heads * head_dim]`` means over batch and the tokens of each segment of
    ``x`` ``[B, T, heads * head_dim]`` (channels contiguous), optionally de-rotated by ``factors``
    (``[n_rows, n_temporal, 2]``, row of token t = t // row_tokens) first."""
    dev = _lib.require_gpu(x, factors)
    if x.dim() != 3 or x.shape[-1] != heads * head_dim:
        raise ValueError(f"expected [B, T, {heads}*{head_dim}], got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    if x.stride(-1) != 1:
        x = x.contiguous()
    bsz, ntok, chans = x.shape
    if spans is not None:
        n_seg = len(spans)
        max_len = max(max(int(e) - int(s) for s, e in spans), 1)
        span_t = torch.tensor([v for se in spans for v in se], dtype=torch.int32).to(dev, non_blocking=True)
        seg = 0
    else:
        seg = int(seg_tokens) if seg_tokens else max(ntok, 1)
        n_seg = max(-(-ntok // seg), 1)
        max_len, span_t = seg, None
    out = torch.empty((n_seg, chans), dtype=torch.float32, device=dev)
    ws = torch.empty((max(_lib.lib().wa_hkv_summary_workspace_bytes(bsz, n_seg, chans, max_len), 1),),
                     dtype=torch.uint8, device=dev)
    if factors is not None:
        factors = factors.to(torch.float32).contiguous()
        n_rows, n_temporal = factors.shape[0], factors.shape[1]
    else:
        n_rows = n_temporal = 0
    args = _lib.HkvSummaryArgs(
        x.data_ptr(), x.stride(0), x.stride(1), _lib.dtype_code(x),
        bsz, ntok, heads, head_dim,
        seg, _lib.ptr(span_t), n_seg, max_len,
        _lib.ptr(factors), n_temporal, int(row_tokens), n_rows,
        int(bool(normalize)), out.data_ptr(), ws.data_ptr())
    _lib.call("wa_hkv_page_summary", ctypes.byref(args), _lib.stream_ptr(dev))
    return out


def _score_topk_chunked(index, query, k, *, scale, mask, want_scores):
    """:func:`score_topk` over more rows than one selection launch takes: each run of
    ``HKV_MAX_PAGES`` rows selects its own top-k, then the candidates (in row order, each run's
    best first) are ordered by a stable descending sort of their scores, which keeps the lowest
    row first among equal scores."""
    n_pages = index.shape[0]
    dev = index.device
    sels, vals, parts = [], [], []
    for r0 in range(0, n_pages, _lib.HKV_MAX_PAGES):
        r1 = min(n_pages, r0 + _lib.HKV_MAX_PAGES)
        kk = min(k, r1 - r0)
        sel, val, sc = score_topk(index[r0:r1], query, kk, scale=scale,
                                  mask=None if mask is None else mask[r0:r1], want_scores=want_scores)
        sels.append(torch.where(sel >= 0, sel + r0, sel))
        vals.append(val)
        if want_scores:
            parts.append(sc)
    cand, cval = torch.cat(sels), torch.cat(vals)
    order = torch.sort(cval, descending=True, stable=True).indices[:k]
    sel, sel_scores = cand[order].to(torch.int32).contiguous(), cval[order].contiguous()
    return sel, sel_scores, torch.cat(parts) if want_scores else None


def score_topk(index: torch.Tensor, query: torch.Tensor, k: int, *, scale: float = 0.0,
               mask: Optional[torch.Tensor] = None, want_scores: bool = False):
    """Device ``(sel int32 [k], sel_scores fp32 [k], scores fp32 [P] or None)``: the ``k`` highest
    of ``index @ query / scale`` (no division for ``scale <= 0``), lowest page index first among
    equal scores; masked pages are skipped and empty slots hold -1 / -inf. More rows than one
    selection launch takes (``HKV_MAX_PAGES``) are selected in runs and merged."""
    dev = _lib.require_gpu(index, query, mask)
    if index.dim() != 2:
        raise ValueError(f"page index must be [P, dim], got {tuple(index.shape)}")
    n_pages, dim = index.shape
    if n_pages < 1:
        raise ValueError("no pages to select from")
    if not 1 <= k <= n_pages:
        raise ValueError(f"k={k} outside [1, {n_pages}]")
    if n_pages > _lib.HKV_MAX_PAGES:
        return _score_topk_chunked(index, query, k, scale=scale, mask=mask, want_scores=want_scores)
    index = index.to(torch.float32)
    if index.stride(-1) != 1:
        index = index.contiguous()
    query = query.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if query.shape[0] != dim:
        raise ValueError(f"query dim {query.shape[0]} does not match page index dim {dim}")
    if mask is not None:
        mask = mask.to(device=dev, dtype=torch.uint8).contiguous()
    sel = torch.empty((k,), dtype=torch.int32, device=dev)
    sel_scores = torch.empty((k,), dtype=torch.float32, device=dev)
    scores = torch.empty((n_pages,), dtype=torch.float32, device=dev) if want_scores else None
    args = _lib.HkvTopkArgs(index.data_ptr(), index.stride(0), query.data_ptr(), n_pages, dim,
                            float(scale) if scale and scale > 0 else 0.0, _lib.ptr(mask), int(k),
                            _lib.ptr(scores), sel.data_ptr(), sel_scores.data_ptr())
    _lib.call("wa_hkv_score_topk", ctypes.byref(args), _lib.stream_ptr(dev))
    return sel, sel_scores, scores


def _as_blhd(t: torch.Tensor) -> torch.Tensor:
    """A [B, T, H, D] view (never a copy: in-place rotation must reach the caller's tensor)."""
    if t.dim() < 3:
        raise ValueError(f"expected [..., tokens, H, D], got {tuple(t.shape)}")
    if t.dim() == 3:
        return t.unsqueeze(0)
    return t if t.dim() == 4 else t.view(-1, *t.shape[-3:])


def rotate_temporal(src: torch.Tensor, factors: torch.Tensor, *, dst: Optional[torch.Tensor] = None,
                    rows: Optional[torch.Tensor] = None, row_tokens: int = 1 << 30, t0: int = 0,
                    t1: Optional[int] = None) -> torch.Tensor:
    """Rotate the temporal band of tokens ``[t0, t1)`` of ``src`` ``[..., T, H, D]`` by ``factors``
    ``[n_rows, n_temporal, 2]`` into ``dst`` (``src`` itself when omitted: in place). The row of
    token t is ``rows[t - t0]`` or ``(t - t0) // row_tokens``."""
    dst = src if dst is None else dst
    dev = _lib.require_gpu(src, dst, factors, rows)
    s4, d4 = _as_blhd(src), _as_blhd(dst)
    if s4.shape != d4.shape or src.dtype != dst.dtype:
        raise ValueError("src and dst must have the same shape and dtype")
    bsz, ntok, heads, hd = s4.shape
    t1 = ntok if t1 is None else t1
    if not 0 <= t0 <= t1 <= ntok:
        raise ValueError(f"token range [{t0}, {t1}) outside [0, {ntok}]")
    if rows is not None:
        rows = rows.to(device=dev, dtype=torch.int32).contiguous()
        if rows.numel() < t1 - t0:
            raise ValueError("rows must hold one entry per rotated token")
    factors = factors.to(torch.float32).contiguous()
    ps, sb, st, sh = _lib.blhd(s4)
    pd, db, dt, dh = _lib.blhd(d4)
    args = _lib.RopeArgs(ps, sb, st, sh, pd, db, dt, dh, _lib.dtype_code(src),
                         bsz, t0, t1, heads, hd, factors.data_ptr(), factors.shape[1], factors.shape[0],
                         _lib.ptr(rows), int(row_tokens))
    _lib.call("wa_rerope", ctypes.byref(args), _lib.stream_ptr(dev))
    return dst


def gather_rotate(pages, dst: torch.Tensor, factors: Optional[torch.Tensor] = None, *, stream=None) -> None:
    """Install pinned host pages into ``dst`` ``[B, cap, H, D]`` (device) with one kernel launch per
    32 pages (``wa_hkv_gather_rotate``): ``pages`` is a list of ``(src, dst_token)`` with ``src`` a
    pinned ``[B, tokens, H, D]`` view; page i's temporal band is multiplied by ``factors[i]``
    (``[n_pages, n_temporal, 2]`` fp32, device) on the way, or copied as is when ``factors`` is None."""
    dev = _lib.require_gpu(dst, factors)
    d4 = _as_blhd(dst)
    bsz, cap, heads, hd = d4.shape
    arr = (_lib.HkvPage * max(len(pages), 1))()
    for i, (src, dst_token) in enumerate(pages):
        if src.is_cuda or not src.is_pinned():
            raise ValueError("gather_rotate reads pinned host pages")
        if src.dtype != dst.dtype:
            raise ValueError(f"page dtype {src.dtype} differs from the cache's {dst.dtype}")
        s4 = _as_blhd(src)
        if s4.shape[0] != bsz or tuple(s4.shape[2:]) != (heads, hd):
            raise ValueError(f"page {tuple(src.shape)} does not fit a [B={bsz}, *, H={heads}, D={hd}] cache")
        p, sb, st, sh = _lib.blhd(s4)
        arr[i] = _lib.HkvPage(p, sb, st, sh, s4.shape[1], int(dst_token))
    nt = 0
    if factors is not None:
        factors = factors.to(torch.float32).contiguous()
        if factors.shape[0] != len(pages):
            raise ValueError("one factor row per page")
        nt = factors.shape[1]
    pd, db, dt, dh = _lib.blhd(d4)
    args = _lib.HkvGatherRotateArgs(ctypes.cast(arr, ctypes.c_void_p), len(pages), pd, db, dt, dh,
                                    _lib.dtype_code(dst), bsz, cap, heads, hd, _lib.ptr(factors), nt)
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    _lib.call("wa_hkv_gather_rotate", ctypes.byref(args), s.cuda_stream)


class PageCopy:
    """One 2-D copy: ``rows`` rows of ``width`` bytes (pitches in bytes)."""

    __slots__ = ("src", "src_pitch", "dst", "dst_pitch", "width", "rows")

    def __init__(self, src: int, src_pitch: int, dst: int, dst_pitch: int, width: int, rows: int):
        self.src, self.src_pitch, self.dst, self.dst_pitch = src, src_pitch, dst, dst_pitch
        self.width, self.rows = width, rows

    def follows(self, other: "PageCopy") -> bool:
        """True when this copy continues ``other`` in both buffers (mergeable into one)."""
        return (self.rows == other.rows and self.src_pitch == other.src_pitch and self.dst_pitch == other.dst_pitch
                and self.src == other.src + other.width and self.dst == other.dst + other.width)


def coalesce(copies: Sequence[PageCopy]) -> list:
    """Merge runs of copies that continue each other (adjacent pages of one chunk)."""
    out: list = []
    for c in copies:
        if out and c.follows(out[-1]):
            prev = out[-1]
            out[-1] = PageCopy(prev.src, prev.src_pitch, prev.dst, prev.dst_pitch, prev.width + c.width, prev.rows)
        else:
            out.append(c)
    return out


def copy_pages(copies: Sequence[PageCopy], *, to_device: bool, stream: torch.cuda.Stream,
               done: Optional[torch.cuda.Event] = None) -> int:
    """Enqueue the copies on ``stream`` (pinned host <-> device) and record ``done`` after them.
    Returns the number of copy commands issued after coalescing."""
    merged = coalesce(copies)
    arr = (_lib.HkvCopy * max(len(merged), 1))()
    for i, c in enumerate(merged):
        arr[i] = _lib.HkvCopy(c.src, c.src_pitch, c.dst, c.dst_pitch, c.width, c.rows)
    name = "wa_hkv_gather_async" if to_device else "wa_hkv_store_async"
    _lib.call(name, arr, len(merged), stream.cuda_stream, None)
    if done is not None:
        done.record(stream)  # torch creates its events lazily: record through torch, same stream order
    return len(merged)
