"""The fabric measurements behind the batch-1 kernels' per-phase latency budget (tests/fabric_probe.hip,
built by ``flashact_amd.build``), run as a child process on the MI355X and printed:

* a 1 KB hand-off and its reply between two CUs of one XCD (plain stores, and sc1 stores) and across
  two XCDs (sc1 stores): the data stores' acknowledgement and the round trip;
* streaming reads with all 256 CUs: every XCD on the same data, every XCD on its own data, one XCD
  alone (GB/s per XCD and in total).

The assertions are structural, not timing gates: no stale read, no capped wait, every workgroup on
the XCD its index implies, a cross-XCD round trip slower than a same-XCD one with plain stores, and
one XCD alone reaching less than all eight together.
"""
import os
import re
import subprocess

import pytest

from flashact_amd.build import FABRIC_PATH

pytestmark = pytest.mark.gpu


def test_fabric_latency_and_bandwidth(gpu):
    if not os.path.exists(FABRIC_PATH):
        pytest.fail(f"{FABRIC_PATH} is missing: run __graft_entry__.build() first")
    res = subprocess.run([FABRIC_PATH], capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0 and "FABRIC OK" in res.stdout, res.stdout + res.stderr
    rt = {(m.group(1), m.group(2)): float(m.group(4)) for m in
          re.finditer(r"handoff (\S+) (\S+): store_ack_ns (\S+) round_trip_ns (\S+)", res.stdout)}
    bw = {m.group(1): float(m.group(3)) for m in re.finditer(r"stream (\S+): per_xcd_GBs (\S+) total_GBs (\S+)", res.stdout)}
    assert set(rt) == {("same-xcd", "plain"), ("same-xcd", "sc1"), ("cross-xcd", "sc1")}, rt
    assert rt[("cross-xcd", "sc1")] > rt[("same-xcd", "plain")], rt
    assert bw["xcd0-alone"] < bw["same-data"] and bw["xcd0-alone"] < bw["own-data"], bw
