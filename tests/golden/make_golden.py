"""Writes tests/golden/golden_small.npz: tiny varlen-attention cases with their
outputs computed by ``oracle.brute_force`` (element-by-element fp64 loops).

The reference ships no golden vectors for this path (all of its tests draw
seeded inputs and compare in the same run, tests/test_correctness.py:48-65),
so these fixtures are generated here. They pin the torch oracle forms against
an independent statement of the mathematics, and pin all of it against drift.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

# (name, q_lens, kv_lens, Hq, Hkv, D, causal, window, bias_mode)
CASES = [
    ("full_ragged", [3, 1, 5], [3, 1, 5], 2, 2, 8, False, 0, None),
    ("causal_ragged", [3, 1, 5], [3, 1, 5], 2, 2, 8, True, 0, None),
    ("causal_cross", [2, 3], [5, 3], 2, 1, 8, True, 0, None),
    ("causal_q_gt_kv", [4, 2], [2, 2], 2, 2, 4, True, 0, None),
    ("window_causal", [6], [6], 2, 1, 8, True, 2, None),
    ("window_noncausal", [5], [5], 1, 1, 4, False, 2, None),
    ("gqa_4_2", [4, 3], [4, 6], 4, 2, 8, False, 0, None),
    ("bias_perhead", [3, 4], [3, 4], 2, 2, 8, False, 0, "perhead"),
    ("bias_broadcast_causal", [4, 2], [4, 3], 2, 1, 8, True, 0, "broadcast"),
]


def make_case(seed, q_lens, kv_lens, Hq, Hkv, D, bias_mode):
    g = torch.Generator().manual_seed(seed)
    Mq, Mk = sum(q_lens), sum(kv_lens)
    q = torch.randn(Mq, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(Mk, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(Mk, Hkv, D, generator=g, dtype=torch.float64)
    do = torch.randn(Mq, Hq, D, generator=g, dtype=torch.float64)
    bias = None
    if bias_mode is not None:
        hb = Hq if bias_mode == "perhead" else 1
        bias = torch.randn(Mq, hb, max(kv_lens), generator=g, dtype=torch.float64)
        bias[:, :, ::3] -= 5.0
    return q, k, v, do, bias


def main():
    arrays = {}
    for i, (name, ql, kl, Hq, Hkv, D, causal, window, bm) in enumerate(CASES):
        q, k, v, do, bias = make_case(100 + i, ql, kl, Hq, Hkv, D, bm)
        cq = [0]
        for n in ql:
            cq.append(cq[-1] + n)
        ck = [0]
        for n in kl:
            ck.append(ck[-1] + n)
        scale = 1.0 / D ** 0.5
        out, lse, dq, dk, dv = oracle.brute_force(q, k, v, do, cq, ck, scale, causal, window, bias)
        p = f"{name}/"
        arrays[p + "q"] = q.numpy()
        arrays[p + "k"] = k.numpy()
        arrays[p + "v"] = v.numpy()
        arrays[p + "dout"] = do.numpy()
        arrays[p + "cu_q"] = np.array(cq, dtype=np.int32)
        arrays[p + "cu_kv"] = np.array(ck, dtype=np.int32)
        arrays[p + "meta"] = np.array([Hq, Hkv, D, int(causal), window], dtype=np.int64)
        if bias is not None:
            arrays[p + "bias"] = bias.numpy()
        arrays[p + "out"] = np.array(out, dtype=np.float64)
        arrays[p + "lse"] = np.array(lse, dtype=np.float64)
        arrays[p + "dq"] = np.array(dq, dtype=np.float64)
        arrays[p + "dk"] = np.array(dk, dtype=np.float64)
        arrays[p + "dv"] = np.array(dv, dtype=np.float64)
    path = os.path.join(HERE, "golden_small.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({len(CASES)} cases)")


if __name__ == "__main__":
    main()
