"""The benchmark CLI (the reference's mtlattn-bench, mtlattn/bench.py) and the
wheel metadata, on the CPU."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_pairs_match_reference_formula():
    """Attended pairs as mtlattn/bench.py:27-35 counts them (its window sum
    written out per query)."""
    from mtlattn_amd.bench import _pairs
    for M in (1, 7, 64, 1000):
        assert _pairs(M, False, 0) == M * M
        assert _pairs(M, True, 0) == M * (M + 1) // 2
        for w in (1, 5, 64, 5000):
            assert _pairs(M, True, w) == sum(min(i + 1, w) for i in range(M))


def test_cli_without_device_exits_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present: the GPU test runs the CLI")
    r = subprocess.run([sys.executable, "-m", "mtlattn.bench", "--sizes", "128"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "no HIP device" in r.stderr


def test_cli_rejects_bad_gqa():
    from mtlattn_amd.bench import main
    import torch
    if not torch.cuda.is_available():
        with pytest.raises(SystemExit):
            main(["--heads", "12", "--kv-heads", "5"])


def test_wheel_metadata():
    """setup.py carries the metadata (setuptools < 61 reads no [project]
    table): name, version, both packages and the mtlattn-bench script."""
    r = subprocess.run([sys.executable, "setup.py", "--name", "--version"], cwd=ROOT, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split()[-2:] == ["mtlattn", "0.4.0+mi355x"]
    text = open(os.path.join(ROOT, "setup.py")).read()
    assert '"mtlattn-bench = mtlattn.bench:main"' in text
    assert 'packages=["mtlattn", "mtlattn_amd"]' in text
