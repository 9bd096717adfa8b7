"""GPU test of the C++ shim (edgeforge_amd/host, EdgeForge's ef::kern / ef::Sampler signatures over
the C-ABI): tests/cpp/shim_forward runs a decode step written like Transformer::forward with the
products on the GPU and checks it against the oracle's Transformer and Sampler."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(__file__), "cpp", "shim_forward")


def test_shim_forward_matches_oracle():
    assert os.path.exists(BIN), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")
