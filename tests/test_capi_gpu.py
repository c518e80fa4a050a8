"""GPU parity through the raw C ABI (mtlattn_amd/capi.py -> libmtlattn_hip.so),
with no torch extension in between: forward + LSE, full backward, the
per-kernel backward entries, and split-KV decode, each against the CPU oracle
on the same seeded inputs. Device memory comes from torch; the library is
called with plain pointers and torch's current stream handle."""

import math

import pytest
import torch

import oracle
from mtlattn_amd import capi
from tests.helpers import LSE_TOL, cu_of, err_stats, randn

pytestmark = pytest.mark.gpu

_DT = {torch.float16: capi.DTYPE_F16, torch.bfloat16: capi.DTYPE_BF16}


def _case(q_lens, kv_lens, Hq, Hkv, D, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = randn((sum(q_lens), Hq, D), dtype, g)
    k = randn((sum(kv_lens), Hkv, D), dtype, g)
    v = randn((sum(kv_lens), Hkv, D), dtype, g)
    do = randn((sum(q_lens), Hq, D), dtype, g)
    return q, k, v, do, cu_of(q_lens), cu_of(kv_lens)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _check(name, pairs, dtype, floors32=None):
    for i, (nm, got, ref) in enumerate(pairs):
        f32 = 0.0 if floors32 is None else floors32[i]
        st = err_stats(got, ref, dtype, f32)
        print(f"  {name} {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e} "
              f"floor32={f32:.3e}", flush=True)
        assert st["ok_elem"], (name, nm, st)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_capi_forward_backward(dtype):
    print(f"\n[case] capi fwd+bwd {dtype} ragged GQA causal D=128", flush=True)
    q_lens, kv_lens, Hq, Hkv, D = [77, 300, 1], [77, 420, 9], 8, 2, 128
    q, k, v, do, cq, ck = _case(q_lens, kv_lens, Hq, Hkv, D, dtype)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod, cqd, ckd = (t.cuda() for t in (q, k, v, do, cq, ck))
    p = capi.problem_for(qd, kd, cqd, ckd, max(q_lens), scale, causal=True)
    out = torch.empty_like(qd)
    lse = torch.empty(qd.shape[0], Hq, dtype=torch.float32, device="cuda")
    # prefill: no workspace, except fp32 on a small grid (key-split partials)
    fws_n = capi.lib().mtlattn_varlen_fwd_workspace_size(p)
    assert fws_n == 0 or dtype == torch.float32
    fws = torch.empty(max(fws_n, 1), dtype=torch.uint8, device="cuda")
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), fws.data_ptr(), fws_n, _stream())
    ws_n = capi.lib().mtlattn_varlen_bwd_workspace_size(p)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    capi.call("mtlattn_varlen_bwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
              dv.data_ptr(), ws.data_ptr(), ws_n, _stream())
    torch.cuda.synchronize()
    ref = oracle.varlen_forward_backward(q, k, v, do, cq, ck, scale, True)
    floors = None
    if dtype == torch.float32:
        # fp32: judge against fp64, allowing for the fp32 oracle's own deviation
        r64 = oracle.varlen_forward_backward(q, k, v, do, cq, ck, scale, True, dtype=torch.float64)
        floors = [err_stats(ref[i], r64[i], torch.float32)["rel"] for i in (0, 2, 3, 4)]
        ref = r64
    ro, rl, rq, rk, rv = ref
    _check("capi", [("out", out.cpu(), ro), ("dq", dq.cpu(), rq), ("dk", dk.cpu(), rk), ("dv", dv.cpu(), rv)],
           dtype, floors)
    assert (lse.cpu() - rl).abs().max().item() < LSE_TOL[dtype]


def test_capi_backward_kernels_fp32_out():
    """mtlattn_bwd_preprocess + mtlattn_bwd_dq + mtlattn_bwd_dkv with fp32
    outputs equal the fused backward entry's gradients (same kernels)."""
    print("\n[case] capi per-kernel backward bf16 window GQA", flush=True)
    q_lens, Hq, Hkv, D = [200, 333], 4, 2, 64
    q, k, v, do, cq, ck = _case(q_lens, q_lens, Hq, Hkv, D, torch.bfloat16, seed=3)
    scale = 0.2
    qd, kd, vd, dod, cqd, ckd = (t.cuda() for t in (q, k, v, do, cq, ck))
    p = capi.problem_for(qd, kd, cqd, ckd, max(q_lens), scale, causal=True, window=50)
    out = torch.empty_like(qd)
    lse = torch.empty(qd.shape[0], Hq, dtype=torch.float32, device="cuda")
    s = _stream()
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), None, 0, s)
    delta = torch.empty(qd.shape[0], Hq, dtype=torch.float32, device="cuda")
    capi.call("mtlattn_bwd_preprocess", p, out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, delta.data_ptr(), s)
    dq = torch.zeros(qd.shape, dtype=torch.float32, device="cuda")
    dk = torch.zeros(kd.shape, dtype=torch.float32, device="cuda")
    dv = torch.zeros_like(dk)
    capi.call("mtlattn_bwd_dq", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), capi.DTYPE_F32, s)
    capi.call("mtlattn_bwd_dkv", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), delta.data_ptr(), dk.data_ptr(), dv.data_ptr(),
              capi.DTYPE_F32, s)
    torch.cuda.synchronize()
    od = (dod.float() * out.float()).sum(-1)
    assert torch.allclose(delta, od, rtol=1e-5, atol=1e-4)
    ro, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, do, cq, ck, scale, True, 50)
    _check("capi-kern", [("dq", dq.cpu(), rq), ("dk", dk.cpu(), rk), ("dv", dv.cpu(), rv)], torch.bfloat16)


@pytest.mark.parametrize("D,dtype,causal,window,bias", [
    (128, torch.bfloat16, True, 0, False),
    (64, torch.float16, False, 0, False),
    (128, torch.float16, True, 40, True),
    (64, torch.bfloat16, True, 0, True),
])
def test_capi_fused_delta_matches_separate_kernels(D, dtype, causal, window, bias):
    """At head dims 64 and 128 mtlattn_varlen_bwd lets the dQ kernel compute
    delta = rowsum(dO * O) itself and leave it in the workspace for dK/dV.
    The delta, dQ, dK and dV it produces must be bitwise equal to those of the
    separate mtlattn_bwd_preprocess + mtlattn_bwd_dq + mtlattn_bwd_dkv calls,
    on ragged GQA input with an empty sequence and rows outside every sequence;
    and the gradients must match the oracle."""
    print(f"\n[case] capi fused delta D={D} {dtype} causal={causal} window={window} bias={bias}", flush=True)
    q_lens, kv_lens, Hq, Hkv = [70, 0, 131, 1, 64], [90, 5, 131, 33, 64], 8, 2
    q, k, v, do, cq, ck = _case(q_lens, kv_lens, Hq, Hkv, D, dtype, seed=11)
    # 3 trailing rows in q/k/v that no sequence owns
    g = torch.Generator().manual_seed(12)
    q, do = (torch.cat([t, randn((3, Hq, D), dtype, g)]) for t in (q, do))
    k, v = (torch.cat([t, randn((3, Hkv, D), dtype, g)]) for t in (k, v))
    scale = 1.0 / math.sqrt(D)
    bias_t = None
    if bias:
        bias_t = torch.randn(q.shape[0], 1, max(kv_lens), generator=g)
    qd, kd, vd, dod, cqd, ckd = (t.cuda() for t in (q, k, v, do, cq, ck))
    bd = bias_t.cuda() if bias else None
    p = capi.problem_for(qd, kd, cqd, ckd, max(q_lens), scale, causal=causal, window=window, bias=bd)
    out = torch.empty_like(qd)
    lse = torch.empty(qd.shape[0], Hq, dtype=torch.float32, device="cuda")
    s = _stream()
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), None, 0, s)
    ws_n = capi.lib().mtlattn_varlen_bwd_workspace_size(p)
    ws = torch.full((ws_n // 4,), float("nan"), dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    capi.call("mtlattn_varlen_bwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
              dv.data_ptr(), ws.data_ptr(), ws_n, s)
    delta = torch.full((qd.shape[0], Hq), float("nan"), dtype=torch.float32, device="cuda")
    capi.call("mtlattn_bwd_preprocess", p, out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, delta.data_ptr(), s)
    dq2, dk2, dv2 = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    capi.call("mtlattn_bwd_dq", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), delta.data_ptr(), dq2.data_ptr(), _DT[dtype], s)
    capi.call("mtlattn_bwd_dkv", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), delta.data_ptr(), dk2.data_ptr(), dv2.data_ptr(),
              _DT[dtype], s)
    torch.cuda.synchronize()
    # every row a sequence owns: delta bitwise equal (rows outside are not read)
    owned = int(cq[-1])
    wsd = ws.view(-1, Hq)[:owned].cpu()
    assert torch.equal(wsd, delta[:owned].cpu()), (wsd - delta[:owned].cpu()).abs().max()
    for nm, a, b, n in (("dq", dq, dq2, owned), ("dk", dk, dk2, int(ck[-1])), ("dv", dv, dv2, int(ck[-1]))):
        assert torch.equal(a[:n].cpu(), b[:n].cpu()), nm
    assert not dq[owned:].any() and not dk[int(ck[-1]):].any() and not dv[int(ck[-1]):].any()
    ro, _, rq, rk, rv = oracle.varlen_forward_backward(q[:owned], k[:int(ck[-1])], v[:int(ck[-1])], do[:owned],
                                                       cq, ck, scale, causal, window,
                                                       bias=bias_t[:owned] if bias else None)
    _check("fused-delta", [("dq", dq[:owned].cpu(), rq), ("dk", dk[:int(ck[-1])].cpu(), rk),
                           ("dv", dv[:int(ck[-1])].cpu(), rv)], dtype)


def test_capi_fp32_split_dkv():
    """fp32 on the fp32 matrix-core kernels: when the dQ or dK/dV grid (one
    workgroup per 128 rows and head) would leave CUs idle, the backward
    workspace query adds room for fp32 partials and mtlattn_varlen_bwd splits
    each workgroup's key tiles (dQ) or (query head, query tile) iterations
    (dK/dV), summing the splits in a fixed order; its dQ kernel computes
    delta itself. Checked: the split path is taken (workspace larger than
    delta), its gradients against the fp64 oracle, bitwise equal on a second
    call, a NaN-filled workspace does not leak into owned rows, rows outside
    every sequence are zero, the in-kernel delta against the preprocess's,
    and a delta-sized workspace (unsplit) gives bitwise the separate
    mtlattn_bwd_dq / mtlattn_bwd_dkv entries' results on that delta."""
    print("\n[case] capi fp32 split dK/dV: ragged GQA causal window, empty sequence, trailing rows", flush=True)
    q_lens, kv_lens, Hq, Hkv, D = [300, 0, 131, 1, 700], [300, 5, 200, 33, 700], 16, 2, 128
    dtype = torch.float32
    q, k, v, do, cq, ck = _case(q_lens, kv_lens, Hq, Hkv, D, dtype, seed=21)
    g = torch.Generator().manual_seed(22)
    q, do = (torch.cat([t, randn((3, Hq, D), dtype, g)]) for t in (q, do))
    k, v = (torch.cat([t, randn((3, Hkv, D), dtype, g)]) for t in (k, v))
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod, cqd, ckd = (t.cuda() for t in (q, k, v, do, cq, ck))
    p = capi.problem_for(qd, kd, cqd, ckd, max(q_lens), scale, causal=True, window=250)
    out = torch.empty_like(qd)
    lse = torch.empty(qd.shape[0], Hq, dtype=torch.float32, device="cuda")
    s = _stream()
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), None, 0, s)
    # the forward with its workspace splits its key tiles (merged by LSE):
    # equal to the unsplit forward above up to fp32 rounding
    fws_n = capi.lib().mtlattn_varlen_fwd_workspace_size(p)
    assert fws_n > 0, "expected the split forward workspace for this small grid"
    fws = torch.full((fws_n // 4,), float("nan"), dtype=torch.float32, device="cuda")
    out_s = torch.full_like(qd, float("nan"))
    lse_s = torch.full_like(lse, float("nan"))
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out_s.data_ptr(), lse_s.data_ptr(), fws.data_ptr(), fws_n, s)
    torch.cuda.synchronize()
    nq0 = int(cq[-1])
    rms_o = out[:nq0].pow(2).mean().sqrt().item()
    oerr = (out_s[:nq0] - out[:nq0]).abs().max().item() / rms_o
    fin = torch.isfinite(lse[:nq0])
    assert torch.equal(fin, torch.isfinite(lse_s[:nq0]))
    lerr = (lse_s[:nq0][fin] - lse[:nq0][fin]).abs().max().item()
    print(f"  split vs unsplit forward: out max|diff| / RMS = {oerr:.3e}, lse max|diff| = {lerr:.3e}", flush=True)
    assert oerr < 1e-5 and lerr < 2e-5
    ws_n = capi.lib().mtlattn_varlen_bwd_workspace_size(p)
    delta_n = qd.shape[0] * Hq * 4
    assert ws_n > delta_n, "expected the split dK/dV workspace for this small grid"
    runs = []
    for n in (ws_n, ws_n, delta_n):
        ws = torch.full((n // 4,), float("nan"), dtype=torch.float32, device="cuda")
        dq, dk, dv = (torch.full_like(t, float("nan")) for t in (qd, kd, vd))
        capi.call("mtlattn_varlen_bwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
                  out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                  dv.data_ptr(), ws.data_ptr(), n, s)
        torch.cuda.synchronize()
        runs.append([t.cpu() for t in (dq, dk, dv)])
    nq, nk = int(cq[-1]), int(ck[-1])
    wdelta = ws[:qd.shape[0] * Hq].clone()          # delta the last (unsplit) call left in its workspace
    delta = torch.empty((qd.shape[0], Hq), dtype=torch.float32, device="cuda")
    capi.call("mtlattn_bwd_preprocess", p, out.data_ptr(), Hq * D, dod.data_ptr(), Hq * D, delta.data_ptr(), s)
    dq2, dk2, dv2 = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    capi.call("mtlattn_bwd_dq", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), wdelta.data_ptr(), dq2.data_ptr(), capi.DTYPE_F32, s)
    capi.call("mtlattn_bwd_dkv", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              dod.data_ptr(), Hq * D, lse.data_ptr(), wdelta.data_ptr(), dk2.data_ptr(), dv2.data_ptr(),
              capi.DTYPE_F32, s)
    torch.cuda.synchronize()
    dl_w, dl_p = wdelta.view(-1, Hq)[:nq].cpu(), delta[:nq].cpu()
    derr = ((dl_w - dl_p).abs().max() / dl_p.pow(2).mean().sqrt()).item()
    print(f"  in-kernel delta vs preprocess: max|diff| / RMS = {derr:.3e}", flush=True)
    assert derr < 1e-5
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b), "split dQ / dK/dV not bitwise repeatable"
    assert torch.equal(runs[2][0][:nq], dq2[:nq].cpu())
    assert torch.equal(runs[2][1][:nk], dk2[:nk].cpu()) and torch.equal(runs[2][2][:nk], dv2[:nk].cpu())
    for r in runs:
        assert not r[0][nq:].any() and not r[1][nk:].any() and not r[2][nk:].any()
    args = (q[:nq], k[:nk], v[:nk], do[:nq], cq, ck, scale, True, 250)
    r64 = oracle.varlen_forward_backward(*args, dtype=torch.float64)
    r32 = oracle.varlen_forward_backward(*args, dtype=torch.float32)
    floors = [err_stats(r32[i], r64[i], dtype)["rel"] for i in (2, 3, 4)]
    for name, r in (("split", runs[0]), ("unsplit", runs[2])):
        _check(f"fp32 {name}", [("dq", r[0][:nq], r64[2]), ("dk", r[1][:nk], r64[3]), ("dv", r[2][:nk], r64[4])],
               dtype, floors)


def test_capi_splitkv_and_workspace_errors():
    print("\n[case] capi split-KV decode bf16 + workspace check", flush=True)
    kv_lens, Hq, Hkv, D = [3000, 5000, 2048], 16, 2, 128
    q, k, v, _, cq, ck = _case([1, 1, 1], kv_lens, Hq, Hkv, D, torch.bfloat16, seed=5)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, cqd, ckd = (t.cuda() for t in (q, k, v, cq, ck))
    p = capi.problem_for(qd, kd, cqd, ckd, 1, scale, causal=True)
    ns = 6
    need = capi.lib().mtlattn_attn_splitkv_workspace_size(p, ns)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(qd)
    lse = torch.empty(3, Hq, dtype=torch.float32, device="cuda")
    with pytest.raises(capi.MtlattnError, match="workspace"):
        capi.call("mtlattn_attn_splitkv", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(),
                  Hkv * D, out.data_ptr(), lse.data_ptr(), ns, ws.data_ptr(), need - 1, _stream())
    capi.call("mtlattn_attn_splitkv", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), ns, ws.data_ptr(), need, _stream())
    torch.cuda.synchronize()
    ro, rl = oracle.varlen_forward(q, k, v, cq, ck, scale, True)
    _check("capi-splitkv", [("out", out.cpu(), ro)], torch.bfloat16)
    assert (lse.cpu() - rl).abs().max().item() < LSE_TOL[torch.bfloat16]
