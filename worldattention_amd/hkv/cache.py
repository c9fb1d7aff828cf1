"""Hierarchical KV cache (HKV) on the GPU, with the reference's signatures.

Mirrors ``pipeline/hkv/cache.py:39-299`` — ``HKVCache(frame_seq_length, page_size_frames,
topk_pages, stage1_topk_chunks, cpu_max_chunks, nvme_enabled, nvme_dir, rerope)`` with ``store`` /
``retrieve`` / ``apply`` / ``reset`` / ``len`` / ``page_tokens`` and the same online-cache dict
contract (``k``, ``v`` ``[B, capacity, H, D]``, ``global_end_index``, ``local_end_index``,
optional ``k_coarse`` / ``v_coarse``). What moves to the GPU path:

* ``store``: page summaries (``wa_hkv_page_summary``) straight from the GPU-resident layer-0
  keys; every layer's valid tokens copied into pinned host blobs on a side stream
  (``wa_hkv_store_async``) instead of synchronous pageable ``.to("cpu")``.
* ``retrieve``: stage-1 and stage-2 scoring + top-k in ``wa_hkv_score_topk``.
* ``apply``: per layer, on the side stream, the selected key pages are read from the pinned tier
  by one kernel that writes them into the online cache already re-rotated
  (``wa_hkv_gather_rotate``, one factor per page from the reference's move plan) when the caller
  waits for the install; with ``wait=False`` they are DMA copies re-rotated in HBM by one short
  pass (``wa_rerope``), which leaves the CUs to the attention that overlaps the install. The value
  pages are DMA copies (``wa_hkv_gather_async``, adjacent pages of a chunk merged into one copy), the
  compressed tier is rebuilt (``wa_compress_kv``) and a per-layer event recorded; the caller's stream
  waits for the last one (or, with ``wait=False``, per layer through :meth:`wait_layer`, so layer
  l's attention overlaps the gather of the layers after it).
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from .. import _lib
from ..hsa.kvcache import refresh_block_sums
from ._ops import PageCopy, copy_pages, factor_table, gather_rotate, rotate_temporal
from .retrieval import page_key_index, prompt_index, select_pages, select_top_chunks
from .rope import temporal_complex_dims
from .tiering import HKVTierManager

__all__ = ["HKVCache"]


def _slab(t: torch.Tensor):
    """(ptr, pitch bytes, row bytes, rows) when each batch row of ``[B, T, H, D]`` is one contiguous
    run of T*H*D elements; None otherwise."""
    bsz, ntok, heads, hd = t.shape
    if ntok > 1 and t.stride(1) != heads * hd or heads > 1 and t.stride(2) != hd or t.stride(3) != 1:
        return None
    es = t.element_size()
    width = ntok * heads * hd * es
    return t.data_ptr(), (t.stride(0) * es if bsz > 1 else width), width, bsz


def _copy(src: torch.Tensor, dst: torch.Tensor) -> PageCopy:
    s, d = _slab(src), _slab(dst)
    return PageCopy(s[0], s[1], d[0], d[1], s[2], s[3])


def _runs_beside(candidate: torch.cuda.Stream, other: torch.cuda.Stream) -> bool:
    """Whether work on ``candidate`` runs while ``other`` is busy: a bounded spin kernel (~1 ms) is
    queued on ``other`` and an event on ``candidate``; the event completes first only when the two
    streams are on different hardware queues (on a shared queue it waits behind the kernel)."""
    busy = torch.cuda.Event()
    with torch.cuda.stream(other):
        torch.cuda._sleep(2_000_000)
        busy.record(other)
    mark = torch.cuda.Event()
    mark.record(candidate)
    beside = False
    while not busy.query():
        if mark.query():
            beside = True
            break
    busy.synchronize()
    return beside


def _copy_stream(device: torch.device, main: torch.cuda.Stream) -> torch.cuda.Stream:
    """The page-copy stream (default priority): one whose work runs beside the caller's stream and
    beside the side streams the attention call uses on it (its linear branch and dQ pass). The
    runtime maps streams onto a few hardware queues (4 by default), so a new stream may share one
    of theirs, depending on how many streams the process created before it; the installs would
    then run in submission order with attention instead of beside it. Up to eight pooled streams
    are tried; the first that runs beside all of them is kept (else the last). Not probed while a
    graph is being captured."""
    if torch.cuda.is_current_stream_capturing():
        return torch.cuda.Stream(device=device)
    from ..hsa.attention import _fork_join
    others = [main, _fork_join(device, main)[0], _fork_join(device, main, 1)[0]]
    for _ in range(8):
        cand = torch.cuda.Stream(device=device)
        if all(cand.cuda_stream != o.cuda_stream for o in others) and all(_runs_beside(cand, o) for o in others):
            return cand
    return cand


class HKVCache:
    """KV bank with two-stage page retrieval and multi-tier residency.

    Args:
        frame_seq_length: tokens per latent frame.
        page_size_frames: frames per page.
        topk_pages: page budget installed per retrieval.
        stage1_topk_chunks: prompt-similar chunks that feed stage 2.
        cpu_max_chunks: host-resident chunk capacity.
        nvme_enabled, nvme_dir: enable and locate the NVMe tier.
        rerope: re-rotate retrieved keys to the cache slots they are replayed at.
    """

    def __init__(self, *, frame_seq_length: int, page_size_frames: int = 8, topk_pages: int = 4,
                 stage1_topk_chunks: int = 1, cpu_max_chunks: int = 64, nvme_enabled: bool = False,
                 nvme_dir: Optional[str] = None, rerope: bool = True):
        self.frame_seq_length = int(frame_seq_length)
        self.page_size_frames = int(page_size_frames)
        self.topk_pages = int(topk_pages)
        self.stage1_topk_chunks = int(stage1_topk_chunks)
        self.rerope = bool(rerope)
        # How apply installs keys. None: by the gather + re-rope kernel when apply waits for the
        # install (the fastest install alone), and by DMA copies followed by the in-HBM rotation
        # pass with wait=False, where the install overlaps attention: the copy engines leave every
        # CU to the attention kernels (the gather kernel's workgroups compete with them for CUs).
        # True / False force one path.
        self.fused_install: Optional[bool] = None
        self._tier_kwargs = dict(cpu_max_chunks=cpu_max_chunks, nvme_enabled=nvme_enabled, nvme_dir=nvme_dir)
        self._side_stream: Optional[torch.cuda.Stream] = None
        self._inflight: list = []   # (event, objects) kept alive until the event completes
        self.layer_events: List[torch.cuda.Event] = []
        self.reset()

    # -- bookkeeping ---------------------------------------------------------------------------
    def reset(self) -> None:
        """Drop the bank and start a fresh rollout."""
        self._drain()
        self.chunks: List[dict] = []
        self.prompt_bank: List[torch.Tensor] = []
        self.tier = HKVTierManager(**self._tier_kwargs)
        self.layer_events = []

    def __len__(self) -> int:
        return len(self.chunks)

    @property
    def page_tokens(self) -> int:
        return self.page_size_frames * self.frame_seq_length

    def _side(self, device: torch.device) -> torch.cuda.Stream:
        if self._side_stream is None or self._side_stream.device != device:
            self._side_stream = _copy_stream(device, torch.cuda.current_stream(device))
        return self._side_stream

    def _keep(self, event, objs) -> None:
        self._inflight = [(e, o) for e, o in self._inflight if not e.query()]
        self._inflight.append((event, objs))

    def _drain(self) -> None:
        for event, _ in self._inflight:
            event.synchronize()
        self._inflight = []

    def wait_layer(self, block_idx: int) -> None:
        """Make the current stream wait until layer ``block_idx`` of the last :meth:`apply` is
        installed (for ``apply(..., wait=False)``)."""
        torch.cuda.current_stream().wait_event(self.layer_events[block_idx])

    # -- store ---------------------------------------------------------------------------------
    def store(self, kv_cache: Sequence[dict], *, prompt_embeds: torch.Tensor, current_start_frame: int,
              temporal_freqs: torch.Tensor) -> int:
        """Write the populated part of the online cache into the bank as a new chunk. Returns the
        chunk id, or -1 when the cache holds nothing."""
        valid = int(kv_cache[0]["local_end_index"].item())
        if valid <= 0:
            return -1
        k0 = kv_cache[0]["k"]
        device = _lib.require_gpu(k0)
        chunk_id = len(self.chunks)
        spans = [(s, min(s + self.page_tokens, valid)) for s in range(0, valid, self.page_tokens)]
        start_frame = int(current_start_frame - valid // self.frame_seq_length)
        index_device = self.prompt_bank[0].device if self.prompt_bank else device
        page_index = page_key_index(k0[:, :valid], spans, frame_seq_length=self.frame_seq_length,
                                    start_frame=start_frame, temporal_freqs=temporal_freqs)

        main, side = torch.cuda.current_stream(device), self._side(device)
        sources, blob, copies = [], {"k": [], "v": []}, []
        for block in kv_cache:
            for name in ("k", "v"):
                src = block[name][:, :valid]
                if _slab(src) is None:
                    src = src.contiguous()
                host = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
                sources.append(src)
                blob[name].append(host)
                copies.append(_copy(src, host))
        side.wait_stream(main)
        done = torch.cuda.Event()
        copy_pages(copies, to_device=False, stream=side, done=done)
        main.wait_event(done)   # later writes into the online cache come after the copy
        self._keep(done, sources)

        self.chunks.append({"chunk_id": chunk_id, "valid_tokens": valid, "page_spans": spans,
                            "start_frame": start_frame, "page_index": page_index})
        self.prompt_bank.append(prompt_index(prompt_embeds.to(device)).detach().to(index_device))
        self.tier.put(chunk_id, blob, ready=done)
        return chunk_id

    # -- retrieve ------------------------------------------------------------------------------
    def retrieve(self, *, prompt_embeds: torch.Tensor, query_vec: torch.Tensor) -> List[Tuple[int, int]]:
        """``(chunk_id, page_id)`` pairs to install for the incoming prompt, chronological."""
        if not self.chunks:
            return []
        bank = torch.stack(self.prompt_bank, dim=0)
        candidates = select_top_chunks(prompt_index(prompt_embeds.to(bank.device)).detach(), bank,
                                       self.stage1_topk_chunks)
        rows, owners = [], []
        for cid in candidates:
            pidx = self.chunks[cid].get("page_index")
            if pidx is None or pidx.numel() == 0:
                continue
            rows.append(pidx)
            owners.extend((cid, p) for p in range(pidx.shape[0]))
        if not rows:
            return []
        index = torch.cat(rows, dim=0)
        query = query_vec.reshape(-1)
        if query.shape[0] != index.shape[1]:
            raise ValueError(f"query dim {query.shape[0]} does not match page index dim {index.shape[1]}")
        if self.topk_pages <= 0:
            return []
        sel, _ = select_pages(index, query.to(index.device), self.topk_pages)
        picked = [owners[i] for i in sel.tolist() if i >= 0]
        return sorted(picked, key=lambda pr: (self.chunks[pr[0]]["start_frame"],
                                              self.chunks[pr[0]]["page_spans"][pr[1]][0]))

    # -- apply ---------------------------------------------------------------------------------
    def _resolve_pages(self, selected_pairs, side):
        entries, blobs = [], {}
        self.tier.prefetch(sorted({cid for cid, _ in selected_pairs}))  # spilled chunks read in parallel
        for chunk_id, page_id in selected_pairs:
            if not 0 <= chunk_id < len(self.chunks):
                continue
            spans = self.chunks[chunk_id]["page_spans"]
            if not 0 <= page_id < len(spans):
                continue
            if chunk_id not in blobs:
                pending = self.tier.ready_event(chunk_id)
                blob = self.tier.get(chunk_id, wait=False)
                if blob is None:
                    continue
                if pending is not None:
                    side.wait_event(pending)   # GPU-side order after the store's copy
                blobs[chunk_id] = blob
            start, end = spans[page_id]
            entries.append((chunk_id, start, end))
        return entries, blobs

    def _plan_rerope(self, installed, current_start_frame):
        """(orig_frame, new_frame) of every installed page: the pages fill consecutive frames that
        end at ``current_start_frame`` (cache.py:273-286)."""
        fsl = self.frame_seq_length
        base = current_start_frame - sum(e - s for _, s, e in installed) // fsl
        moves, offset = [], 0
        for chunk_id, start, end in installed:
            moves.append((self.chunks[chunk_id]["start_frame"] + start // fsl, base + offset // fsl))
            offset += end - start
        return moves

    def apply(self, kv_cache: Sequence[dict], selected_pairs: Sequence[Tuple[int, int]], *, current_start_frame: int,
              temporal_freqs: torch.Tensor, hsa_modules: Optional[Sequence] = None, wait: bool = True) -> int:
        """Install the selected pages into the online cache, replacing its contents; returns the
        number of tokens installed. ``hsa_modules`` (one per block) is required when the cache
        carries a compressed tier."""
        k0 = kv_cache[0]["k"]
        device = _lib.require_gpu(k0)
        main, side = torch.cuda.current_stream(device), self._side(device)
        entries, blobs = self._resolve_pages(selected_pairs, side)
        if not entries:
            return 0
        capacity, dtype = int(k0.shape[1]), k0.dtype
        installed, budget = [], capacity
        for chunk_id, start, end in entries:
            if budget <= 0:
                break
            take = min(end - start, budget)
            installed.append((chunk_id, start, start + take))
            budget -= take
        total = sum(e - s for _, s, e in installed)
        moves = self._plan_rerope(installed, current_start_frame) if self.rerope else None
        has_coarse = "k_coarse" in kv_cache[0] and "v_coarse" in kv_cache[0]
        if has_coarse and hsa_modules is None:
            raise ValueError("the online cache carries a compressed tier, so hsa_modules must be supplied so it "
                             "can be rebuilt for the installed pages")

        side.wait_stream(main)
        keep = [blobs]
        self.layer_events = []
        with torch.cuda.stream(side):
            factors = rows = None
            if moves and total > 0:
                nt = temporal_complex_dims(k0.shape[-1])
                factors = factor_table(temporal_freqs[:, :nt], torch.tensor([m[1] for m in moves]),
                                       torch.tensor([m[0] for m in moves]), device)
                lens = torch.tensor([e - s for _, s, e in installed], device=device)
                rows = torch.repeat_interleave(torch.arange(len(installed), device=device, dtype=torch.int32),
                                               lens, output_size=total)
                keep += [factors, rows]
            for block_idx, block in enumerate(kv_cache):
                kc, vc = block["k"], block["v"]
                targets = [kc, vc] + ([block["k_coarse"], block["v_coarse"]] if has_coarse else [])
                for t in targets:
                    if t.is_cuda:
                        t.record_stream(side)
                if total < capacity:
                    kc[:, total:].zero_()
                    vc[:, total:].zero_()
                if has_coarse:
                    block["k_coarse"].zero_()
                    block["v_coarse"].zero_()
                if total > 0:
                    fused = self._gather_layer(block_idx, installed, blobs, kc, vc, total, keep, factors,
                                               use_kernel=wait if self.fused_install is None else self.fused_install)
                    if factors is not None and not fused:
                        rotate_temporal(kc, factors, rows=rows, t0=0, t1=total)
                    if has_coarse:
                        self._write_coarse(block, hsa_modules[block_idx], kc[:, :total], vc[:, :total])
                    refresh_block_sums(block, total)  # key block sums kept for routing, if any
                block["global_end_index"].fill_(current_start_frame * self.frame_seq_length)
                block["local_end_index"].fill_(total)
                ev = torch.cuda.Event()
                ev.record(side)
                self.layer_events.append(ev)
        self._keep(self.layer_events[-1], keep)
        if wait:
            main.wait_event(self.layer_events[-1])
        return total

    def _gather_layer(self, block_idx, installed, blobs, kc, vc, total, keep, factors=None, use_kernel=True) -> bool:
        """Pinned-tier pages of one layer -> cache tokens [0, total). With ``use_kernel``, keys of the
        cache's dtype are read by one kernel that also applies each page's re-rope factors (returns
        True); otherwise they are DMA copies like the values (neighbouring pages of a chunk
        coalesce) and the caller rotates afterwards."""
        k_srcs = [blobs[cid]["k"][block_idx] for cid, _, _ in installed]
        fused = use_kernel and all(src.dtype == kc.dtype for src in k_srcs)
        if fused:
            pages, off = [], 0
            for (cid, s, e), src in zip(installed, k_srcs):
                pages.append((src[:, s:e], off))
                off += e - s
            gather_rotate(pages, kc, factors, stream=torch.cuda.current_stream(kc.device))
        plans = []
        for name, dst in ((("v", vc),) if fused else (("k", kc), ("v", vc))):
            srcs = [blobs[cid][name][block_idx] for cid, _, _ in installed]
            direct = all(s.dtype == dst.dtype for s in srcs) and _slab(dst[:, :total]) is not None
            stage = dst[:, :total] if direct else torch.empty((dst.shape[0], total) + tuple(srcs[0].shape[2:]),
                                                              dtype=srcs[0].dtype, device=dst.device)
            if not all(s.dtype == stage.dtype for s in srcs):
                raise TypeError("pages of one layer must share a dtype")
            copies, off = [], 0
            for (cid, s, e), src in zip(installed, srcs):
                copies.append(_copy(src[:, s:e], stage[:, off:off + e - s]))
                off += e - s
            plans.append((copies, stage, dst, direct))
        copy_pages([c for plan in plans for c in plan[0]], to_device=True,
                   stream=torch.cuda.current_stream(kc.device))
        for _, stage, dst, direct in plans:
            if not direct:
                dst[:, :total].copy_(stage)
                keep.append(stage)
        return fused

    @staticmethod
    def _write_coarse(block: dict, hsa, loaded_k: torch.Tensor, loaded_v: torch.Tensor) -> None:
        """Rebuild the compressed tier for pages installed at cache offset 0 (cache.py:288-299)."""
        start, end = hsa.token_range_to_coarse(0, int(loaded_k.shape[1]))
        with torch.no_grad():
            k_coarse, v_coarse = hsa.compress_kv_cache(loaded_k, loaded_v)
        block["k_coarse"][:, start:end] = k_coarse.to(dtype=block["k_coarse"].dtype, device=block["k_coarse"].device)
        block["v_coarse"][:, start:end] = v_coarse.to(dtype=block["v_coarse"].dtype, device=block["v_coarse"].device)
