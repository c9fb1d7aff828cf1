"""The NVMe tier's asynchronous file I/O (``wa_io_*``) and how the tier manager uses it: byte-exact
round trips of aligned, unaligned and empty buffers, several transfers in flight, reloads started
ahead of ``get``, a chunk requested while its spill is still being written, and I/O errors raised
as ``OSError``. Runs on the CPU (host code of the library)."""
import ctypes
import os

import pytest
import torch

from worldattention_amd import _lib
from worldattention_amd.hkv.tiering import HKVTierManager, _leaves, _start_io


def _wait(handle):
    _lib.call("wa_io_wait", handle)


@pytest.mark.parametrize("direct", [True, False])
def test_round_trip_of_aligned_unaligned_and_empty_buffers(tmp_path, direct):
    torch.manual_seed(0)
    big = torch.randn(3 * 4096 + 77)               # a page-aligned start, a ragged tail
    base = torch.randint(0, 255, (20000,), dtype=torch.uint8)
    tensors = [big, base[13:13 + 9000], torch.empty(0), torch.randn(5, 7).bfloat16(), base[1:2]]
    handles = []
    for i in range(3):                              # three files written at once
        handles.append(_start_io(True, str(tmp_path / f"f{i}.bin"), tensors, direct))
    for h in handles:
        _wait(h)
    for i in range(3):
        back = [torch.empty_like(t) for t in tensors]
        _wait(_start_io(False, str(tmp_path / f"f{i}.bin"), back, direct))
        for a, b in zip(tensors, back):
            assert torch.equal(a, b)
        # each buffer starts at a 4 KiB boundary of the file
        sizes = [t.numel() * t.element_size() for t in tensors]
        assert os.path.getsize(tmp_path / f"f{i}.bin") == sum(-(-s // 4096) * 4096 for s in sizes)


def test_read_errors_are_os_errors(tmp_path):
    path = tmp_path / "short.bin"
    path.write_bytes(b"x" * 100)
    dst = [torch.empty(4096 * 3, dtype=torch.uint8)]  # buffers live until the wait
    with pytest.raises(OSError, match="end of file"):
        _wait(_start_io(False, str(path), dst, False))
    with pytest.raises(OSError, match="cannot open"):
        _start_io(False, str(tmp_path / "missing.bin"), dst, True)


def _blob(i, layers=3):
    return {"k": [torch.full((1, 37, 2, 16), float(i + l)) for l in range(layers)],
            "v": [torch.full((1, 37, 2, 16), -float(i + l)) for l in range(layers)]}


def test_spill_reload_prefetch_and_in_flight_reuse(tmp_path):
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    for i in range(4):
        tier.put(i, _blob(i))                       # 0, 1, 2 spill; 3 stays
    assert [tier.location(i) for i in range(4)] == ["nvme"] * 3 + ["cpu"]
    assert len(os.listdir(tmp_path)) == 3           # files exist as soon as the spill returns
    tier.prefetch([0, 1, 3, 99])                    # only spilled chunks start reading
    got = tier.get(0)                               # a spill still in flight, or the prefetch
    assert all(torch.equal(t, torch.full_like(t, float(l))) for l, t in enumerate(got["k"]))
    assert all(torch.equal(t, torch.full_like(t, -float(l))) for l, t in enumerate(got["v"]))
    tier._reap()
    got1 = tier.get(1)
    assert torch.equal(got1["k"][2], torch.full((1, 37, 2, 16), 3.0))
    assert tier.stats()["n_loads"] == 2
    tier.cleanup()
    assert os.listdir(tmp_path) == [] and not tier._writes and not tier._reads


def test_a_finished_spill_is_read_back_from_its_file(tmp_path, monkeypatch):
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    monkeypatch.setattr(tier, "_reap", lambda: None)  # keep the write in flight-tracking for the test
    tier.put(0, _blob(5))
    tier.put(1, _blob(6))
    monkeypatch.undo()
    handle, blob, _ = tier._writes[0]
    _wait(handle)                                   # let the write finish, then forget it
    del tier._writes[0]
    del blob
    got = tier.get(0)
    assert torch.equal(got["k"][1], torch.full((1, 37, 2, 16), 6.0))
    assert len(_leaves(got, [])) == 6
    tier.cleanup()


def test_a_failed_spill_keeps_the_chunk_in_host_memory_and_raises(tmp_path, monkeypatch):
    """A spill whose write fails is reported, with the chunk's id, by the next tier call; the chunk
    stays host-resident with its blob, and its partial file is deleted and forgotten (so a later
    eviction writes it again instead of trusting a short file)."""
    import time
    from worldattention_amd.hkv import tiering
    tier = HKVTierManager(cpu_max_chunks=1, nvme_enabled=True, nvme_dir=str(tmp_path))
    monkeypatch.setattr(tier, "_reap", lambda: None)  # the puts must not reap the spill themselves
    tier.put(0, _blob(1))
    tier.put(1, _blob(2))                          # evicts chunk 0: its spill starts
    monkeypatch.undo()
    path = tier._files[0]
    handle = tier._writes[0][0]
    while _lib.lib().wa_io_done(handle) != 1:
        time.sleep(0.001)
    real_call = tiering._lib.call

    def failing(name, *args):
        if name == "wa_io_wait":
            real_call(name, *args)                  # release the handle, then report a failure
            raise OSError("injected write failure")
        return real_call(name, *args)

    monkeypatch.setattr(tiering._lib, "call", failing)
    with pytest.raises(OSError, match="chunk 0"):
        tier.stats()
    monkeypatch.undo()
    assert tier.location(0) == "cpu"
    assert 0 not in tier._files and not os.path.exists(path)
    got = tier.get(0)
    assert all(torch.equal(t, torch.full_like(t, float(1 + l))) for l, t in enumerate(got["k"]))
    tier.cleanup()
