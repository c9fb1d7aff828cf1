"""Multi-tier residency of KV chunk blobs (pinned host DRAM, optional NVMe spill).

The observable behaviour of ``pipeline/hkv/tiering.py:18-127`` is kept, since the cache and its
tests depend on it: ``put`` / ``get`` / ``location`` / ``stats`` / ``cleanup``; least recently used
host chunks leave first; with NVMe a spilled chunk keeps its file as a backup, so spilling it again
writes nothing; without NVMe it is dropped. Additions for the GPU path: a blob may carry the event
of the device->host copy that fills it (``put(..., ready=event)``); host readers and spills wait
for it.

The NVMe tier replaces the reference's synchronous ``torch.save`` / ``torch.load`` with
asynchronous direct I/O (``wa_io_*``): a spill starts writing the blob's tensors (raw bytes, one
4 KiB-aligned region each, O_DIRECT where the file system takes it) on a worker thread and returns;
the blob is released once the write has completed (checked on every put, get, prefetch and stats
call); a write that fails leaves the chunk in host memory and raises. A reload reads into freshly allocated (pinned, when
a GPU is present) tensors of the recorded shapes; :meth:`HKVTierManager.prefetch` starts reloads
ahead of their ``get``. A chunk requested while its spill is still being written is served from
memory.
"""
from __future__ import annotations

import ctypes
import os
from collections import OrderedDict
from typing import Dict, Iterable, List, Optional

import torch

from .. import _lib

__all__ = ["HKVTierManager"]

_HOST, _DISK = "cpu", "nvme"


def _leaves(obj, out: List[torch.Tensor]) -> List[torch.Tensor]:
    """The tensors of a blob (dicts in key order, lists in order)."""
    if isinstance(obj, torch.Tensor):
        out.append(obj)
    elif isinstance(obj, dict):
        for key in sorted(obj):
            _leaves(obj[key], out)
    elif isinstance(obj, (list, tuple)):
        for val in obj:
            _leaves(val, out)
    return out


def _spec(obj):
    """The blob's structure with each tensor replaced by its (shape, dtype)."""
    if isinstance(obj, torch.Tensor):
        return ("t", tuple(obj.shape), obj.dtype)
    if isinstance(obj, dict):
        return ("d", {key: _spec(val) for key, val in obj.items()})
    if isinstance(obj, (list, tuple)):
        return ("l", type(obj), [_spec(val) for val in obj])
    return ("o", obj)


def _build(spec, pin: bool):
    """Empty tensors (pinned when ``pin``) in the structure of ``spec``."""
    kind = spec[0]
    if kind == "t":
        return torch.empty(spec[1], dtype=spec[2], pin_memory=pin)
    if kind == "d":
        return {key: _build(val, pin) for key, val in spec[1].items()}
    if kind == "l":
        return spec[1](_build(val, pin) for val in spec[2])
    return spec[1]


def _start_io(write: bool, path: str, tensors: List[torch.Tensor], direct: bool) -> int:
    n = len(tensors)
    bufs = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in tensors])
    sizes = (ctypes.c_int64 * max(n, 1))(*[t.numel() * t.element_size() for t in tensors])
    fn = "wa_io_write_async" if write else "wa_io_read_async"
    handle = getattr(_lib.lib(), fn)(os.fsencode(path), bufs, sizes, n, int(direct))
    if handle <= 0:
        msg = _lib.lib().wa_last_error().decode(errors="replace")
        raise (OSError if handle == _lib.WA_ERR_IO else ValueError)(f"{fn}: {msg}")
    return handle


class HKVTierManager:
    """Chunk blobs across host DRAM and NVMe with LRU migration.

    Args:
        cpu_max_chunks: host-resident chunk capacity (at least 1).
        nvme_enabled: spill over-capacity chunks to disk instead of dropping them.
        nvme_dir: directory of spill files; required when ``nvme_enabled``.
    """

    def __init__(self, cpu_max_chunks: int, nvme_enabled: bool = False, nvme_dir: Optional[str] = None):
        self.cpu_max_chunks = max(int(cpu_max_chunks), 1)
        self.nvme_enabled = bool(nvme_enabled)
        self.nvme_dir = nvme_dir
        if self.nvme_enabled:
            if not nvme_dir:
                raise ValueError("nvme_dir is required when nvme_enabled=True")
            os.makedirs(nvme_dir, exist_ok=True)
        self._where: Dict[int, str] = {}            # chunk -> tier
        self._recency: "OrderedDict[int, None]" = OrderedDict()  # least recent first
        self._blobs: Dict[int, dict] = {}            # host-resident blobs
        self._files: Dict[int, str] = {}             # spill file (backup) per chunk ever spilled
        self._pending: Dict[int, object] = {}        # fill event per host blob
        self._specs: Dict[int, tuple] = {}           # structure of each spilled blob
        self._writes: Dict[int, tuple] = {}          # spill in flight: (handle, blob, tensors)
        self._reads: Dict[int, tuple] = {}           # reload in flight: (handle, blob)
        self.direct_io = True
        self.n_spills = self.n_loads = self.n_drops = 0

    # -- residency -------------------------------------------------------------------------
    def _use(self, chunk_id: int) -> None:
        self._recency.pop(chunk_id, None)
        self._recency[chunk_id] = None

    def _wait_filled(self, chunk_id: int) -> None:
        event = self._pending.pop(chunk_id, None)
        if event is not None:
            event.synchronize()

    def _host_count(self) -> int:
        return sum(1 for tier in self._where.values() if tier == _HOST)

    def _make_room(self) -> None:
        while self._host_count() > self.cpu_max_chunks:
            victim = next(cid for cid in self._recency if self._where.get(cid) == _HOST)
            self._wait_filled(victim)
            blob = self._blobs.pop(victim)
            if not self.nvme_enabled:
                del self._where[victim]
                del self._recency[victim]
                self.n_drops += 1
                continue
            if victim not in self._files:
                path = os.path.join(self.nvme_dir, f"hkv_chunk_{victim}.bin")
                tensors = [t if t.is_contiguous() else t.contiguous() for t in _leaves(blob, [])]
                self._specs[victim] = _spec(blob)
                self._writes[victim] = (_start_io(True, path, tensors, self.direct_io), blob, tensors)
                self._files[victim] = path
            self._where[victim] = _DISK
            self.n_spills += 1
        self._reap()

    def _reap(self) -> None:
        """Finish the spills whose writes have completed, releasing their blobs. A spill that failed
        leaves its chunk in host memory (without a backup file, which is deleted) and raises
        ``OSError`` naming the chunk."""
        for cid in [c for c, (h, _, _) in self._writes.items() if _lib.lib().wa_io_done(h) == 1]:
            handle, blob, _ = self._writes.pop(cid)
            try:
                _lib.call("wa_io_wait", handle)
            except OSError as exc:
                path = self._files.pop(cid, None)
                self._specs.pop(cid, None)
                if path is not None:
                    try:
                        os.remove(path)
                    except OSError:
                        pass
                if self._where.get(cid) == _DISK:
                    self._blobs[cid] = blob
                    self._where[cid] = _HOST
                    self.n_spills -= 1
                raise OSError(f"HKVTierManager: spilling chunk {cid} failed; it stays in host memory: {exc}") from exc

    def _read(self, chunk_id: int) -> dict:
        """Reload a spilled chunk: the blob still in memory if its spill is being written, else the
        prefetched or a fresh read of its file."""
        if chunk_id in self._writes:
            return self._writes[chunk_id][1]
        if chunk_id in self._reads:
            handle, blob = self._reads.pop(chunk_id)
        else:
            blob = _build(self._specs[chunk_id], torch.cuda.is_available())
            handle = _start_io(False, self._files[chunk_id], _leaves(blob, []), self.direct_io)
        _lib.call("wa_io_wait", handle)
        return blob

    def prefetch(self, chunk_ids: Iterable[int]) -> None:
        """Start reading spilled chunks back so later ``get`` calls only wait for them."""
        self._reap()
        for cid in chunk_ids:
            if self._where.get(cid) == _DISK and cid not in self._reads and cid not in self._writes:
                blob = _build(self._specs[cid], torch.cuda.is_available())
                self._reads[cid] = (_start_io(False, self._files[cid], _leaves(blob, []), self.direct_io), blob)

    # -- API -------------------------------------------------------------------------------
    def put(self, chunk_id: int, blob: dict, ready=None) -> None:
        """Register a freshly produced chunk as host-resident (``ready``: event of its fill)."""
        self._blobs[chunk_id] = blob
        self._where[chunk_id] = _HOST
        if ready is None:
            self._pending.pop(chunk_id, None)
        else:
            self._pending[chunk_id] = ready
        self._use(chunk_id)
        self._make_room()

    def get(self, chunk_id: int, wait: bool = True) -> Optional[dict]:
        """The chunk's blob, reloaded from NVMe if it was spilled (None if unknown). With ``wait``
        the copy that filled it has completed; ``wait=False`` suits consumers ordered after that
        copy on the same stream."""
        self._reap()
        tier = self._where.get(chunk_id)
        if tier is None:
            return None
        if tier == _DISK:
            blob = self._read(chunk_id)
            self.n_loads += 1
            self._blobs[chunk_id] = blob
            self._where[chunk_id] = _HOST
            self._use(chunk_id)
            self._make_room()
            return blob
        self._use(chunk_id)
        if wait:
            self._wait_filled(chunk_id)
        return self._blobs[chunk_id]

    def ready_event(self, chunk_id: int):
        """Pending fill event of a host-resident blob, or None."""
        return self._pending.get(chunk_id)

    def location(self, chunk_id: int) -> str:
        """``"cpu"``, ``"nvme"`` or ``"absent"``."""
        return self._where.get(chunk_id, "absent")

    def stats(self) -> dict:
        self._reap()
        on_disk = sum(1 for tier in self._where.values() if tier == _DISK)
        return {"cpu_resident": self._host_count(), "nvme_resident": on_disk, "backups": len(self._files),
                "n_spills": self.n_spills, "n_loads": self.n_loads, "n_drops": self.n_drops}

    def cleanup(self) -> None:
        """Delete spill files and forget every chunk."""
        for cid in list(self._pending):
            self._wait_filled(cid)
        errors = []
        for table in (self._writes, self._reads):
            for handle, *_ in table.values():
                try:
                    _lib.call("wa_io_wait", handle)
                except OSError as exc:  # the files go anyway
                    errors.append(exc)
            table.clear()
        self._specs.clear()
        for path in set(self._files.values()):
            try:
                os.remove(path)
            except OSError:
                pass
        self._where.clear()
        self._recency.clear()
        self._blobs.clear()
        self._files.clear()
        if errors:
            raise errors[0]
