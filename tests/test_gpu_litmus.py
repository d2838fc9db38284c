"""Litmus tests of the message passing every kernel relies on (tests/litmus_xcd.hip, built by
``flashact_amd.build``), run as a child process on the MI355X:

* across XCDs: sc1 data stores, a wait for them, an sc1 flag store; the reader polls the flag and reads
  the data with sc1 loads (the grid barriers and the fixups of the stage engine);
* inside one XCD: plain stores (they stay in the XCD's L2) and sc1 loads (the batch-1 kernels' XCD
  barriers and targeted waits);
* the batch-1 exchange: fp16 values carrying the round's parity in their lowest bit, polled with sc1
  loads and accepted only when every value carries it.

2000 rounds on 8 channels per case, every ordered XCD distance for the flag test; a reader stops at
its first stale value. Any stale read, capped wait or workgroup placed off its XCD fails the test.
"""
import os
import subprocess

import pytest

from flashact_amd.build import LITMUS_PATH

pytestmark = pytest.mark.gpu


def test_cross_xcd_message_passing(gpu):
    if not os.path.exists(LITMUS_PATH):
        pytest.fail(f"{LITMUS_PATH} is missing: run __graft_entry__.build() first")
    res = subprocess.run([LITMUS_PATH], capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0 and "LITMUS OK" in res.stdout, res.stdout + res.stderr
