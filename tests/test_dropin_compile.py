"""The reference's call sites compile against the drop-in headers (CPU only:
nothing runs).  tests/dropin/reference_callsites.cpp repeats them as the
reference writes them (BinaryWeightLoader(gpu, dir) and loader->load,
BufferWrapper<float> caches of the reference's layout, BucketMul::shared,
TransformerLayer::forward over those caches, MistralModel(gpu, dir)); the
GPU run of the same program is in test_dropin_gpu.py."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_reference_callsites_compile():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "dropin"), "syntax"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "warning" not in r.stderr, r.stderr
