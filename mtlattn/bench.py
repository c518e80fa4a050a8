"""``python -m mtlattn.bench`` / ``mtlattn-bench``: the benchmark CLI under the
reference's module name (mtlattn/bench.py); implemented in mtlattn_amd.bench."""

from mtlattn_amd.bench import main  # noqa: F401

if __name__ == "__main__":
    main()
