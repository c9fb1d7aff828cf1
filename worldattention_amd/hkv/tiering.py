"""Multi-tier residency of KV chunk blobs (pinned host DRAM, optional NVMe spill).

The observable behaviour of ``pipeline/hkv/tiering.py:18-127`` is kept, since the cache and its
tests depend on it: ``put`` / ``get`` / ``location`` / ``stats`` / ``cleanup``; least recently used
host chunks leave first; with NVMe a spilled chunk keeps its file as a backup, so spilling it again
writes nothing; without NVMe it is dropped. Additions for the GPU path: a blob may carry the event
of the device->host copy that fills it (``put(..., ready=event)``); host readers and spills wait
for it. Spill files are written by ``torch.save`` and read with ``torch.load(weights_only=True)``
(dicts / lists of tensors), then re-pinned when a GPU is present so page gathers stay asynchronous.
"""
from __future__ import annotations

import os
from collections import OrderedDict
from typing import Dict, Optional

import torch

__all__ = ["HKVTierManager"]

_HOST, _DISK = "cpu", "nvme"


def _pinned(obj):
    """``obj`` with every tensor in page-locked host memory."""
    if isinstance(obj, torch.Tensor):
        return obj if obj.is_pinned() else obj.pin_memory()
    if isinstance(obj, dict):
        return {key: _pinned(val) for key, val in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_pinned(val) for val in obj)
    return obj


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
                path = os.path.join(self.nvme_dir, f"hkv_chunk_{victim}.pt")
                torch.save(blob, path)
                self._files[victim] = path
            self._where[victim] = _DISK
            self.n_spills += 1

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
        tier = self._where.get(chunk_id)
        if tier is None:
            return None
        if tier == _DISK:
            blob = torch.load(self._files[chunk_id], map_location="cpu", weights_only=True)
            if torch.cuda.is_available():
                blob = _pinned(blob)
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
        on_disk = sum(1 for tier in self._where.values() if tier == _DISK)
        return {"cpu_resident": self._host_count(), "nvme_resident": on_disk, "backups": len(self._files),
                "n_spills": self.n_spills, "n_loads": self.n_loads, "n_drops": self.n_drops}

    def cleanup(self) -> None:
        """Delete spill files and forget every chunk."""
        for cid in list(self._pending):
            self._wait_filled(cid)
        for path in set(self._files.values()):
            try:
                os.remove(path)
            except OSError:
                pass
        self._where.clear()
        self._recency.clear()
        self._blobs.clear()
        self._files.clear()
