"""mtlattn_varlen_fwd_noalloc (no counterpart in the reference; for callers
that cannot allocate): through the C ABI, its outputs must equal
mtlattn_varlen_fwd's with a caller workspace, bitwise (same routing, same
kernels), on two calls in a row -- the second smaller, reusing the static
scratch the first one filled -- plus a prefill call (no scratch needed), an
fp32 small-grid call (key-split partials in the scratch) and a call whose
partials would exceed the static scratch (refused before any launch)."""

import ctypes
import math

import pytest
import torch

from mtlattn_amd import capi
from tests.helpers import cu_of

pytestmark = pytest.mark.gpu


def _decode_inputs(B, kv_lo, kv_hi, Hq, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    kv_lens = torch.randint(kv_lo, kv_hi + 1, (B,), generator=g).tolist()
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(sum(kv_lens), Hkv, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(sum(kv_lens), Hkv, D, generator=g).to(torch.bfloat16).cuda()
    return q, k, v, cu_of([1] * B, "cuda"), cu_of(kv_lens, "cuda")


def _both(q, k, v, cq, ck, max_q, causal=True):
    """(out, lse) of mtlattn_varlen_fwd with a workspace and of the noalloc
    entry, both through the C ABI on torch's current stream."""
    D = q.shape[2]
    p = capi.problem_for(q, k, cq, ck, max_q, 1.0 / math.sqrt(D), causal=causal)
    sh = torch.cuda.current_stream().cuda_stream
    L = capi.lib()
    need = L.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    rs, rk = q.stride(0), k.stride(0)
    outs = []
    for noalloc in (False, True):
        out = torch.full_like(q, float("nan"))
        lse = torch.full((q.shape[0], q.shape[1]), float("nan"), dtype=torch.float32, device="cuda")
        if noalloc:
            capi.call("mtlattn_varlen_fwd_noalloc", p, q.data_ptr(), rs, k.data_ptr(), rk, v.data_ptr(), rk,
                      out.data_ptr(), lse.data_ptr(), sh)
        else:
            capi.call("mtlattn_varlen_fwd", p, q.data_ptr(), rs, k.data_ptr(), rk, v.data_ptr(), rk, out.data_ptr(),
                      lse.data_ptr(), ws.data_ptr(), need, sh)
        outs.append((out, lse))
    torch.cuda.synchronize()
    return need, outs


def test_noalloc_forward_matches_workspace_entry():
    print("\n[case] noalloc forward: decode 16 seqs kv U[4096,16384] GQA 32/8, then 3 seqs kv U[2048,5000]",
          flush=True)
    L = capi.lib()
    limit = 64 << 20
    for B, lo, hi, seed in ((16, 4096, 16384, 1), (3, 2048, 5000, 2)):
        q, k, v, cq, ck = _decode_inputs(B, lo, hi, 32, 8, 128, seed)
        p = capi.problem_for(q, k, cq, ck, 1, 1.0 / math.sqrt(128), causal=True)
        assert L.mtlattn_decode_num_splits(ctypes.byref(p)) > 0, "not routed to split-KV"
        need, ((o_ws, l_ws), (o_na, l_na)) = _both(q, k, v, cq, ck, 1)
        print(f"  B={B}: scratch bytes {need} of {limit}", flush=True)
        assert 0 < need <= limit
        assert torch.isfinite(o_ws.float()).all() and torch.isfinite(l_ws).all()
        assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na), f"B={B}: noalloc differs from workspace entry"
    # a prefill call (flash forward, no scratch) through the same entry
    print("[case] noalloc forward: prefill 2 seqs causal (no scratch)", flush=True)
    g = torch.Generator().manual_seed(3)
    lens = [300, 77]
    q = torch.randn(sum(lens), 8, 128, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(sum(lens), 2, 128, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(sum(lens), 2, 128, generator=g).to(torch.bfloat16).cuda()
    cu = cu_of(lens, "cuda")
    need, ((o_ws, l_ws), (o_na, l_na)) = _both(q, k, v, cu, cu, max(lens))
    assert need == 0
    assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na)
    # fp32 on a small grid: the forward splits its key tiles, with the
    # partials in the caller's workspace or in the static scratch
    print("[case] noalloc forward: fp32 small grid (key splits in the scratch)", flush=True)
    lens = [250, 129, 17]
    q = torch.randn(sum(lens), 4, 64, generator=g).cuda()
    k = torch.randn(sum(lens), 4, 64, generator=g).cuda()
    v = torch.randn(sum(lens), 4, 64, generator=g).cuda()
    cu = cu_of(lens, "cuda")
    need, ((o_ws, l_ws), (o_na, l_na)) = _both(q, k, v, cu, cu, max(lens), causal=False)
    print(f"  scratch bytes {need} of {limit}", flush=True)
    assert 0 < need <= limit
    assert torch.isfinite(o_ws).all() and torch.isfinite(l_ws).all()
    assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na)


def test_noalloc_forward_refuses_oversized_scratch():
    """A decode call whose partials exceed the static scratch is refused
    with MTLATTN_ERR_WORKSPACE before anything is launched. The tensors are
    the full size the problem describes (768 sequences of one query against
    2048 keys, 8 kv heads: 2 x 3.2 GB of K and V), so that a regression in
    the host-side refusal would run an in-bounds forward, not read past an
    allocation."""
    print("\n[case] noalloc forward: oversized split-KV request refused", flush=True)
    L = capi.lib()
    nseq, kv_len, hq, hkv, d = 768, 2048, 64, 8, 128
    q = torch.zeros(nseq, hq, d, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(nseq * kv_len, hkv, d, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    o = torch.empty_like(q)
    cq = cu_of([1] * nseq, "cuda")
    ck = cu_of([kv_len] * nseq, "cuda")
    p = capi.problem_for(q, k, cq, ck, 1, 0.1, causal=True)
    need = L.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p))
    print(f"  split-KV scratch needed {need} bytes", flush=True)
    assert need > (64 << 20)
    sh = torch.cuda.current_stream().cuda_stream
    rc = L.mtlattn_varlen_fwd_noalloc(ctypes.byref(p), q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0),
                                      v.data_ptr(), v.stride(0), o.data_ptr(), None, sh)
    assert rc == capi.ERR_WORKSPACE
    assert b"static" in L.mtlattn_last_error()
