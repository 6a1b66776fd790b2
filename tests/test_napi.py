"""The Node host side on the CPU: the N-API addon (g4hip.node) and
HipBackend (gemma4-webgpu_amd/node/hip_backend.js), checked by
tests/node/test_napi_cpu.js under Node."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "gemma4-webgpu_amd", "node", "g4hip.node")


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_addon_and_backend_on_cpu():
    assert os.path.exists(ADDON), "g4hip.node is not built (run __graft_entry__.build())"
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "test_napi_cpu.js")], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all node CPU checks passed" in r.stdout
