"""Benchmark CLI (the reference's ``mtlattn-bench``, mtlattn/bench.py).

    python -m mtlattn.bench                          # default sweep
    python -m mtlattn.bench --paths both             # matrix-core and portable kernels
    python -m mtlattn.bench --causal --vs-sdpa       # causal, next to torch SDPA
    python -m mtlattn.bench --sizes 1024 8192 --dtype fp16 --window 256
    python -m mtlattn.bench --kv-heads 8 --backward  # GQA, forward + backward
    python -m mtlattn.bench --decode --sizes 8192 65536 --heads 64 --kv-heads 8

Square self-attention of one sequence per size, as the reference measures it
(mtlattn/bench.py:27-35,43-56): per-call latency (best of 4 timed rounds) and
effective TFLOP/s over the attended pairs, 4*pairs*D*H for the forward
(QK + PV) and 14*pairs*D*H with --backward (the backward's 10*pairs*D*H on
top). --decode times one query row per sequence against a KV cache of each
size (8 sequences) and reports HBM GB/s over the K/V bytes read.

Paths: ``auto`` is the production routing (matrix-core kernels for fp16/bf16
and the supported head dims); ``generic`` forces the portable kernels with
MTLATTN_NO_MFMA (the reference's --paths simdgroup equivalent, which forces
its portable Metal path with MTLATTN_NO_MPP).
"""

import argparse
import math
import os
import time

import torch

from . import varlen_attention

_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _pairs(M, causal, window):
    """Attended (query, key) pairs of square self-attention (reference:
    mtlattn/bench.py:27-35): a window limits each query to `window` keys
    ending at its own position."""
    if window > 0:
        w = min(M, window)
        return w * (w + 1) // 2 + (M - w) * w
    if causal:
        return M * (M + 1) // 2
    return M * M


def _time(fn, iters, warmup=5):
    """Best average over 4 rounds of `iters` calls (reference:
    mtlattn/bench.py:38-48), synchronising the device around each round."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(4):
        t = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        best = min(best, (time.perf_counter() - t) / iters)
    return best


class _ForcedPath:
    """Selects the kernel family for the calls inside the block through the
    library's routing switch (read on every call)."""

    def __init__(self, generic):
        self.generic = generic

    def __enter__(self):
        self.prev = os.environ.get("MTLATTN_NO_MFMA")
        os.environ.pop("MTLATTN_NO_MFMA", None)
        if self.generic:
            os.environ["MTLATTN_NO_MFMA"] = "1"

    def __exit__(self, *exc):
        os.environ.pop("MTLATTN_NO_MFMA", None)
        if self.prev is not None:
            os.environ["MTLATTN_NO_MFMA"] = self.prev


def _bench_mtlattn(M, H, Hkv, D, dtype, causal, window, backward, generic, iters):
    with _ForcedPath(generic):
        q = torch.randn(M, H, D, dtype=dtype, device="cuda")
        k = torch.randn(M, Hkv, D, dtype=dtype, device="cuda")
        v = torch.randn(M, Hkv, D, dtype=dtype, device="cuda")
        cu = torch.tensor([0, M], dtype=torch.int32, device="cuda")
        scale = 1.0 / math.sqrt(D)
        if not backward:
            return _time(lambda: varlen_attention(q, k, v, cu, cu, M, scale, causal=causal, window=window),
                         iters)
        q.requires_grad_()
        k.requires_grad_()
        v.requires_grad_()
        do = torch.randn(M, H, D, dtype=dtype, device="cuda")

        def step():
            out = varlen_attention(q, k, v, cu, cu, M, scale, causal=causal, window=window)
            torch.autograd.grad(out, (q, k, v), do)
        return _time(step, iters)


def _bench_sdpa(M, H, Hkv, D, dtype, causal, backward, iters):
    q = torch.randn(1, H, M, D, dtype=dtype, device="cuda", requires_grad=backward)
    k = torch.randn(1, Hkv, M, D, dtype=dtype, device="cuda", requires_grad=backward)
    v = torch.randn(1, Hkv, M, D, dtype=dtype, device="cuda", requires_grad=backward)
    kw = {"is_causal": causal}
    if Hkv != H:
        kw["enable_gqa"] = True
    f = torch.nn.functional.scaled_dot_product_attention
    if not backward:
        return _time(lambda: f(q, k, v, **kw), iters)
    do = torch.randn(1, H, M, D, dtype=dtype, device="cuda")
    return _time(lambda: torch.autograd.grad(f(q, k, v, **kw), (q, k, v), do), iters)


def _bench_decode(L, H, Hkv, D, dtype, iters, batch=8):
    q = torch.randn(batch, H, D, dtype=dtype, device="cuda")
    k = torch.randn(batch * L, Hkv, D, dtype=dtype, device="cuda")
    v = torch.randn(batch * L, Hkv, D, dtype=dtype, device="cuda")
    cu_q = torch.arange(0, batch + 1, dtype=torch.int32, device="cuda")
    cu_kv = torch.arange(0, (batch + 1) * L, L, dtype=torch.int32, device="cuda")
    s = _time(lambda: varlen_attention(q, k, v, cu_q, cu_kv, 1, causal=True), iters)
    return s, batch * L * Hkv * D * k.element_size() * 2


def main(argv=None):
    ap = argparse.ArgumentParser(prog="mtlattn.bench", description="Benchmark mtlattn attention on MI355X.")
    ap.add_argument("--sizes", type=int, nargs="+", default=[1024, 2048, 4096],
                    help="sequence lengths (square self-attention; KV lengths with --decode)")
    ap.add_argument("--heads", type=int, default=12)
    ap.add_argument("--kv-heads", type=int, default=None, help="kv heads for GQA (default: --heads)")
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--dtype", default="bf16", choices=list(_DT))
    ap.add_argument("--causal", action="store_true")
    ap.add_argument("--window", type=int, default=0, help="sliding-window size (0 = off)")
    ap.add_argument("--paths", default="auto", choices=["auto", "generic", "both"],
                    help="auto = production routing; generic = portable kernels; both = side by side")
    ap.add_argument("--vs-sdpa", action="store_true", help="also time torch SDPA on the same device")
    ap.add_argument("--backward", action="store_true", help="time forward + backward")
    ap.add_argument("--decode", action="store_true", help="one query per sequence against KV of each size")
    ap.add_argument("--iters", type=int, default=10)
    args = ap.parse_args(argv)

    if not torch.cuda.is_available():
        raise SystemExit("mtlattn.bench: no HIP device available")

    dtype = _DT[args.dtype]
    H, D = args.heads, args.head_dim
    Hkv = args.kv_heads or H
    if H % Hkv:
        raise SystemExit("mtlattn.bench: --heads must be a multiple of --kv-heads")
    if args.decode:
        print(f"mtlattn.bench decode - {args.dtype}, Hq={H}, Hkv={Hkv}, D={D}, 8 sequences, q_len 1")
        print("  " + "kv_len".rjust(8) + "latency".rjust(12) + "HBM".rjust(14))
        for L in args.sizes:
            s, nbytes = _bench_decode(L, H, Hkv, D, dtype, args.iters)
            print("  " + f"{L:8d}" + f"{s * 1e3:10.3f}ms" + f"{nbytes / s / 1e9:10.1f}GB/s")
        return

    paths = {"auto": [("auto", False)], "generic": [("generic", True)],
             "both": [("auto", False), ("generic", True)]}[args.paths]
    tag = f"{args.dtype}, H={H}" + (f", Hkv={Hkv}" if Hkv != H else "") + f", D={D}" + \
          (", causal" if args.causal else "") + (f", window={args.window}" if args.window else "") + \
          (", fwd+bwd" if args.backward else "")
    cols = [name for name, _ in paths] + (["sdpa"] if args.vs_sdpa else [])
    print(f"mtlattn.bench - {tag}")
    print("  " + "size".rjust(7) + "".join(c.rjust(22) for c in cols))
    for M in args.sizes:
        flops = (14 if args.backward else 4) * _pairs(M, args.causal, args.window) * D * H
        cells = []
        for _, generic in paths:
            s = _bench_mtlattn(M, H, Hkv, D, dtype, args.causal, args.window, args.backward, generic, args.iters)
            cells.append(f"{s * 1e3:7.2f}ms {flops / s / 1e12:7.2f}TF")
        if args.vs_sdpa:
            try:
                if args.window:
                    raise ValueError("no window in torch SDPA")
                s = _bench_sdpa(M, H, Hkv, D, dtype, args.causal, args.backward, args.iters)
                cells.append(f"{s * 1e3:7.2f}ms {flops / s / 1e12:7.2f}TF")
            except Exception:  # unsupported combination, or out of memory at large sizes
                cells.append(f"{'n/a':>16}")
        print("  " + f"{M:7d}" + "".join(c.rjust(22) for c in cells))


if __name__ == "__main__":
    main()
