"""Host tier bookkeeping of worldattention_amd.hkv.HKVTierManager (CPU only): the behaviour the
reference's tests/test_hkv_tiering.py fixes — LRU order, NVMe spill and reload, free re-spills via
backups, cleanup — plus the fill-event handshake used by the GPU store path."""
import os

import pytest
import torch

from worldattention_amd.hkv import HKVTierManager


def blob(tag):
    return {"k": [torch.full((2, 2), float(tag))], "v": [torch.full((2, 2), -float(tag))]}


def test_resident_chunks_round_trip():
    tier = HKVTierManager(cpu_max_chunks=4)
    for cid in range(3):
        tier.put(cid, blob(cid))
    for cid in range(3):
        assert tier.location(cid) == "cpu"
        assert torch.equal(tier.get(cid)["k"][0], torch.full((2, 2), float(cid)))
    assert tier.get(99) is None and tier.location(99) == "absent"


def test_over_capacity_drops_the_least_recently_used_without_nvme():
    tier = HKVTierManager(cpu_max_chunks=2)
    tier.put(0, blob(0))
    tier.put(1, blob(1))
    tier.get(0)
    tier.put(2, blob(2))
    assert [tier.location(c) for c in range(3)] == ["cpu", "absent", "cpu"]
    assert tier.stats()["n_drops"] == 1 and tier.stats()["n_spills"] == 0


def test_capacity_is_never_below_one():
    tier = HKVTierManager(cpu_max_chunks=0)
    tier.put(0, blob(0))
    assert tier.location(0) == "cpu"


def test_nvme_spills_and_reloads(tmp_path):
    tier = HKVTierManager(cpu_max_chunks=2, nvme_enabled=True, nvme_dir=str(tmp_path))
    for cid in range(3):
        tier.put(cid, blob(cid))
    assert tier.location(0) == "nvme" and tier.stats()["n_spills"] == 1
    assert len(os.listdir(tmp_path)) == 1
    assert torch.equal(tier.get(0)["k"][0], torch.zeros(2, 2))
    assert tier.location(0) == "cpu"
    st = tier.stats()
    assert st["n_loads"] == 1 and st["n_drops"] == 0 and st["nvme_resident"] == 1   # chunk 1 went out


def test_nvme_backup_makes_respilling_free(tmp_path):
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    tier.put(0, blob(0))
    tier.put(1, blob(1))
    assert tier.stats()["n_spills"] == 1
    tier.get(0)                       # reload 0, spilling 1
    tier.put(2, blob(2))              # spills 0 again, reusing its file
    assert tier.stats()["backups"] == len(os.listdir(tmp_path)) == 2
    assert torch.equal(tier.get(0)["k"][0], torch.zeros(2, 2))


def test_nvme_requires_a_directory():
    with pytest.raises(ValueError):
        HKVTierManager(cpu_max_chunks=1, nvme_enabled=True)


def test_cleanup_removes_files_and_state(tmp_path):
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    tier.put(0, blob(0))
    tier.put(1, blob(1))
    assert len(os.listdir(tmp_path)) == 1
    tier.cleanup()
    assert os.listdir(tmp_path) == [] and tier.stats()["cpu_resident"] == 0 and tier.location(0) == "absent"


class _Event:
    """Stand-in for a device event: counts host waits."""

    def __init__(self):
        self.waits = 0

    def synchronize(self):
        self.waits += 1


def test_fill_events_are_waited_on_by_readers_and_before_a_spill(tmp_path):
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    e0, e1 = _Event(), _Event()
    tier.put(0, blob(0), ready=e0)
    assert tier.ready_event(0) is e0
    tier.get(0, wait=False)
    assert e0.waits == 0
    tier.put(1, blob(1), ready=e1)      # spilling 0 waits for its fill first
    assert e0.waits == 1 and tier.ready_event(0) is None
    tier.get(1)
    assert e1.waits == 1 and tier.ready_event(1) is None
    tier.get(1)
    assert e1.waits == 1
