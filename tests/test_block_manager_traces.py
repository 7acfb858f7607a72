"""BlockManager id semantics against the reference implementation.

tests/golden/block_manager_traces.json holds operation scripts and the outputs
of the reference's own src/core/block_manager.cpp (compiled from the reference
sources by oracle/Makefile; recorded by tests/golden/make_bm_traces.py).  The
same driver compiled against this repository's BlockManager must print the
same lines.  Where the reference tree is present, fresh random scripts are
also compared live.
"""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OURS = os.path.join(ROOT, "oracle", "_build", "bm_trace_ours")
REF = os.path.join(ROOT, "oracle", "_ref", "bm_trace_ref")
GOLDEN = os.path.join(ROOT, "tests", "golden", "block_manager_traces.json")


def run(exe, script):
    return subprocess.run([exe], input=script, capture_output=True, text=True, check=True, timeout=60).stdout


@pytest.fixture(scope="module")
def ours():
    if not os.path.exists(OURS):
        pytest.fail(f"{OURS} not built: run make -C oracle")
    return OURS


def test_matches_recorded_reference_traces(ours):
    cases = json.load(open(GOLDEN))["cases"]
    assert len(cases) >= 10
    for c in cases:
        assert run(ours, c["script"]) == c["expected"], f"seed {c['seed']}"


@pytest.mark.skipif(not os.path.exists(REF), reason="reference build not present (oracle/_ref)")
def test_matches_reference_live(ours):
    import sys
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_bm_traces
    for seed in range(100, 104):
        script = make_bm_traces.make_script(seed, n_ops=60)
        assert run(ours, script) == run(REF, script), f"seed {seed}"
