"""The benchmark's host-side contract, without a GPU: more than one GPU is refused with a message
and exit status 2, the kernel-source fingerprint is what the committed counter summaries record
(so the bench line's traffic figure is a measurement of the kernel it times), and the roofline
traffic is read from that summary."""
import json
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _recorded_fingerprint(name):
    text = open(os.path.join(ROOT, "profiles", name)).read()
    m = re.search(r"kernel_source_fingerprint:\s*([0-9a-f]{16})", text)
    assert m, f"{name} records no kernel source fingerprint"
    return m.group(1)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


@pytest.mark.parametrize("summary", ["bsa_fwd_cfg2_traffic.md", "bsa_fwd_cfg2_counters.md"])
def test_committed_sparse_kernel_summaries_match_the_kernel_sources(summary):
    fp = bench.kernel_source_fingerprint()
    assert re.fullmatch(r"[0-9a-f]{16}", fp)
    assert _recorded_fingerprint(summary) == fp, (
        f"profiles/{summary} was measured on other sparse-kernel sources; re-collect it")


def test_roofline_traffic_comes_from_the_summary():
    traffic = bench.measured_traffic()
    assert traffic is not None and 1e8 < traffic < 1e9
