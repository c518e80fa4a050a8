"""The benchmark CLI on the device: every mode runs and prints its table."""

import pytest

pytestmark = pytest.mark.gpu


def test_cli_modes(capsys):
    from mtlattn_amd.bench import main
    main(["--sizes", "256", "512", "--iters", "2", "--paths", "both", "--vs-sdpa"])
    main(["--sizes", "512", "--iters", "2", "--heads", "8", "--kv-heads", "2", "--causal", "--backward",
          "--vs-sdpa"])
    main(["--sizes", "512", "--iters", "2", "--causal", "--window", "128", "--dtype", "fp16"])
    main(["--decode", "--sizes", "4096", "--iters", "2", "--heads", "16", "--kv-heads", "2"])
    out = capsys.readouterr().out
    print(out, flush=True)
    assert out.count("mtlattn.bench") == 4
    assert "TF" in out and "GB/s" in out
