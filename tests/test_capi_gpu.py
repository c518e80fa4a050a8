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
    assert capi.lib().mtlattn_varlen_fwd_workspace_size(p) == 0
    capi.call("mtlattn_varlen_fwd", p, qd.data_ptr(), Hq * D, kd.data_ptr(), Hkv * D, vd.data_ptr(), Hkv * D,
              out.data_ptr(), lse.data_ptr(), None, 0, _stream())
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
