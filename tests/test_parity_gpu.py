"""GPU parity: the HIP kernels (through mtlattn's public API and _C) against
the CPU oracle on the same seeded inputs.

Ports the reference's case matrix (tests/test_correctness.py:312-465) with its
absolute tolerances, and adds LSE, split-KV, determinism and bookkeeping
checks. Every case prints its name first so a failing run names its case.
"""

import math
import os

import pytest
import torch

import oracle
from tests.helpers import LSE_TOL, REF_ATOL, RMS_BOUND, cu_of, err_stats, randn

pytestmark = pytest.mark.gpu

torch.set_num_threads(min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def mt():
    import mtlattn
    return mtlattn


def _banner(name):
    print(f"\n[case] {name}", flush=True)


def _inputs(q_lens, kv_lens, Hq, Hkv, D, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = randn((sum(q_lens), Hq, D), dtype, g)
    k = randn((sum(kv_lens), Hkv, D), dtype, g)
    v = randn((sum(kv_lens), Hkv, D), dtype, g)
    return q, k, v


def _make_bias(Mq, H, max_kv, broadcast, seed=7):
    """Additive bias as tests/test_correctness.py:214-223 builds it: randn with
    every 7th key pushed down by 30."""
    g = torch.Generator().manual_seed(seed)
    b = torch.randn((Mq, 1 if broadcast else H, max_kv), generator=g)
    b[:, :, ::7] -= 30.0
    return b


def _fwd(mt, name, q_lens, kv_lens, Hq, Hkv, D, dtype, atol=None, causal=False, window=0,
         bias=None, check_lse=True, seed=0):
    _banner(name)
    atol = REF_ATOL[dtype] if atol is None else atol
    q, k, v = _inputs(q_lens, kv_lens, Hq, Hkv, D, dtype, seed)
    cq, ck = cu_of(q_lens), cu_of(kv_lens)
    scale = 1.0 / math.sqrt(D)
    dev = "cuda"
    lse = torch.empty(sum(q_lens), Hq, dtype=torch.float32, device=dev)
    bdev = None if bias is None else bias.to(dev)
    out = mt._C.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cq.to(dev), ck.to(dev),
                                 max(q_lens), scale, causal, window, lse, bdev)
    out2 = mt.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cq.to(dev), ck.to(dev),
                               max(q_lens), scale, causal=causal, window=window, attn_bias=bdev)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.varlen_forward(q, k, v, cq, ck, scale, causal, window, bias)
    err = (out.cpu().float() - ref).abs().max().item()
    st = err_stats(out, ref, dtype)
    print(f"  max_err={err:.3e} atol={atol} rel={st['rel']:.3e} floor={st['floor']:.3e} "
          f"rms_rel={st['rms_rel']:.3e}", flush=True)
    assert torch.isfinite(out.float()).all()
    assert err < atol, f"{name}: max_err {err} >= {atol}"
    assert torch.equal(out.cpu(), out2.cpu()), f"{name}: _C and public API disagree"
    if check_lse:
        fin = torch.isfinite(ref_lse)
        lse_c = lse.cpu()
        assert torch.equal(torch.isfinite(lse_c), fin), f"{name}: LSE -inf pattern differs"
        lerr = (lse_c[fin] - ref_lse[fin]).abs().max().item() if fin.any() else 0.0
        print(f"  lse_err={lerr:.3e}", flush=True)
        assert lerr < LSE_TOL[dtype], f"{name}: lse err {lerr}"
    return out


def _bwd(mt, name, q_lens, kv_lens, Hq, Hkv, D, dtype, atol, causal=False, window=0, bias=None,
         seed=0):
    _banner(name)
    q, k, v = _inputs(q_lens, kv_lens, Hq, Hkv, D, dtype, seed)
    g = torch.Generator().manual_seed(seed + 1)
    dout = randn((sum(q_lens), Hq, D), dtype, g)
    cq, ck = cu_of(q_lens), cu_of(kv_lens)
    dev = "cuda"
    qm = q.to(dev).requires_grad_()
    km = k.to(dev).requires_grad_()
    vm = v.to(dev).requires_grad_()
    out = mt.varlen_attention(qm, km, vm, cq.to(dev), ck.to(dev), max(q_lens), causal=causal,
                              window=window, attn_bias=None if bias is None else bias.to(dev))
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    ro, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cq, ck, None, causal, window, bias)
    errs = {}
    for nm, a, b in (("out", out, ro), ("dQ", qm.grad, rq), ("dK", km.grad, rk), ("dV", vm.grad, rv)):
        assert torch.isfinite(a.float()).all(), f"{name}: non-finite {nm}"
        errs[nm] = (a.detach().cpu().float() - b).abs().max().item()
        if dtype != torch.float32:
            st = err_stats(a, b, dtype)
            errs[nm + "_rms_rel"] = st["rms_rel"]
    print("  " + " ".join(f"{k_}={v_:.3e}" for k_, v_ in errs.items()) + f" atol={atol}", flush=True)
    worst = max(errs["dQ"], errs["dK"], errs["dV"])
    assert worst < atol, f"{name}: grad err {errs}"
    if dtype != torch.float32:   # and the relative RMS criterion of tests/helpers.py
        for nm in ("out", "dQ", "dK", "dV"):
            assert errs[nm + "_rms_rel"] <= RMS_BOUND[dtype], f"{name}: {nm} rms_rel {errs[nm + '_rms_rel']:.3e}"
    return qm.grad, km.grad, vm.grad


# ---------------------------------------------------------------------------
# forward: dtype sweep, ragged, cross, packed (tests/test_correctness.py:316-319)
# ---------------------------------------------------------------------------
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
def test_self_ragged(mt, dtype):
    _fwd(mt, f"self[{dtype}] ragged", [5, 128, 33, 1000], [5, 128, 33, 1000], 12, 12, 128, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_cross(mt, dtype):
    _fwd(mt, f"cross[{dtype}]", [64, 7, 300], [128, 1, 900], 12, 12, 128, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_packed(mt, dtype):
    _banner(f"packed[{dtype}]")
    g = torch.Generator().manual_seed(1)
    lens = [37, 256, 1, 1023]
    M, H, D = sum(lens), 12, 128
    qkv = randn((M, 3, H, D), dtype, g)
    q, k, v = qkv.unbind(1)
    ref, _ = oracle.varlen_forward(q, k, v, cu_of(lens), cu_of(lens))
    out = mt.flash_attn_varlen_qkvpacked_func(qkv.cuda(), cu_of(lens, "cuda"), max(lens))
    e1 = (out.cpu().float() - ref).abs().max().item()
    q_lens, kv_lens = [64, 512], [300, 100]
    q2 = randn((sum(q_lens), H, D), dtype, g)
    kv = randn((sum(kv_lens), 2, H, D), dtype, g)
    k2, v2 = kv.unbind(1)
    ref2, _ = oracle.varlen_forward(q2, k2, v2, cu_of(q_lens), cu_of(kv_lens))
    out2 = mt.flash_attn_varlen_kvpacked_func(q2.cuda(), kv.cuda(), cu_of(q_lens, "cuda"),
                                              cu_of(kv_lens, "cuda"), max(q_lens), max(kv_lens))
    e2 = (out2.cpu().float() - ref2).abs().max().item()
    print(f"  qkv_err={e1:.3e} kv_err={e2:.3e}", flush=True)
    assert e1 < REF_ATOL[dtype] and e2 < REF_ATOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_backward(mt, dtype):
    """Gradients through both packed wrappers (tests/test_correctness.py:68-96
    checks their forward): q/k/v are row-strided unbind views (row stride
    3*H*D, and 2*Hkv*D for kv), which the backward kernels read in place
    (the reference makes them contiguous first, mtlattn/__init__.py:42-45).
    Checked against the oracle's gradients of the unbound tensors."""
    _banner(f"packed backward[{dtype}]")
    g = torch.Generator().manual_seed(11)
    lens = [37, 256, 1, 700]
    M, H, D = sum(lens), 8, 128
    qkv = randn((M, 3, H, D), dtype, g)
    dout = randn((M, H, D), dtype, g)
    qkv_d = qkv.cuda().requires_grad_()
    out = mt.flash_attn_varlen_qkvpacked_func(qkv_d, cu_of(lens, "cuda"), max(lens), causal=True)
    out.backward(dout.cuda())
    q, k, v = qkv.unbind(1)
    ro, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cu_of(lens), cu_of(lens), None, True)
    ref = torch.stack([rq, rk, rv], dim=1)
    for nm, a, r in (("out", out, ro), ("dqkv", qkv_d.grad, ref)):
        st = err_stats(a, r, dtype)
        print(f"  qkv {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e}", flush=True)
        assert st["ok_elem"], f"qkvpacked {nm}: {st}"
    # kv-packed, GQA 8/2, cross lengths, window
    q_lens, kv_lens = [64, 300, 5], [300, 1000, 77]
    q2 = randn((sum(q_lens), H, D), dtype, g)
    kv = randn((sum(kv_lens), 2, 2, D), dtype, g)
    do2 = randn((sum(q_lens), H, D), dtype, g)
    q2d, kvd = q2.cuda().requires_grad_(), kv.cuda().requires_grad_()
    out2 = mt.flash_attn_varlen_kvpacked_func(q2d, kvd, cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda"),
                                              max(q_lens), max(kv_lens), causal=True, window_size=(255, 0))
    out2.backward(do2.cuda())
    k2, v2 = kv.unbind(1)
    ro2, _, rq2, rk2, rv2 = oracle.varlen_forward_backward(q2, k2, v2, do2, cu_of(q_lens), cu_of(kv_lens), None,
                                                           True, 256)
    for nm, a, r in (("out", out2, ro2), ("dq", q2d.grad, rq2), ("dkv", kvd.grad, torch.stack([rk2, rv2], 1))):
        st = err_stats(a, r, dtype)
        print(f"  kv {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e}", flush=True)
        assert st["ok_elem"], f"kvpacked {nm}: {st}"


# odd head dims, tiny windows, single long sequence (tests/test_correctness.py:321-328)
def test_head_dims_small(mt):
    _fwd(mt, "self D=64", [100, 200], [100, 200], 16, 16, 64, torch.float16)
    _fwd(mt, "self D=80", [77, 13], [77, 13], 8, 8, 80, torch.float16)


def test_5000_windows(mt):
    g = torch.Generator().manual_seed(2)
    wlens = torch.randint(1, 65, (5000,), generator=g).tolist()
    _fwd(mt, "5000 windows", wlens, wlens, 12, 12, 128, torch.float16, check_lse=False)


def test_single_16384(mt):
    _banner("1x16384 (heads 0 and 11 checked)")
    q, k, v = _inputs([16384], [16384], 12, 12, 128, torch.float16)
    cu = cu_of([16384])
    out = mt.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), 16384).cpu()
    ref, _, _, _, _ = oracle.varlen_forward_backward_blocked(q, k, v, None, cu, cu, heads=[0, 11],
                                                             backward=False, q_block=2048)
    err = (out[:, [0, 11]].float() - ref[:, [0, 11]]).abs().max().item()
    print(f"  max_err={err:.3e}", flush=True)
    assert err < 5e-3


# head dims 64/80/88/96/128 (matrix-core kernels; tests/test_correctness.py:332-343)
def test_mfma_d64(mt):
    _fwd(mt, "D=64 full", [2048], [2048], 12, 12, 64, torch.float16)
    _fwd(mt, "D=64 causal", [4096], [4096], 12, 12, 64, torch.float16, causal=True)
    _fwd(mt, "D=64 bf16", [1500], [1500], 8, 8, 64, torch.bfloat16, causal=True)
    _fwd(mt, "D=64 SWA", [2048], [2048], 12, 12, 64, torch.float16, causal=True, window=128)


def test_mfma_d64_rising_scores(mt):
    """Logits that grow along the key axis (key norms ramp up x12), so later
    tiles outweigh the running max by far more than 2^12: the D=64 forward's
    deferred tile max must rescale. Also a bias that lifts the last keys."""
    for dtype, causal in ((torch.float16, False), (torch.bfloat16, True)):
        name = f"D=64 rising scores {dtype} causal={causal}"
        _banner(name)
        lens = [1500, 2600]
        q, k, v = _inputs(lens, lens, 8, 8, 64, dtype, seed=5)
        for s, n in zip(cu_of(lens)[:-1].tolist(), lens):
            ramp = 1.0 + 11.0 * torch.arange(n, dtype=torch.float32) / n
            k[s:s + n] = (k[s:s + n].float() * ramp[:, None, None]).to(dtype)
        cu = cu_of(lens)
        lse = torch.empty(sum(lens), 8, dtype=torch.float32, device="cuda")
        out = mt._C.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), max(lens),
                                     0.125, causal, 0, lse, None).cpu()
        ref, ref_lse = oracle.varlen_forward(q, k, v, cu, cu, 0.125, causal)
        err = (out.float() - ref).abs().max().item()
        lerr = (lse.cpu() - ref_lse).abs().max().item()
        print(f"  max_err={err:.3e} lse_err={lerr:.3e}", flush=True)
        assert torch.isfinite(out.float()).all()
        assert err < REF_ATOL[dtype] and lerr < LSE_TOL[dtype]
    bias = _make_bias(2048, 8, 2048, False)
    bias[:, :, 1900:] += 40.0
    _fwd(mt, "D=64 bias lifts the tail", [2048], [2048], 8, 8, 64, torch.float16, bias=bias)


def test_rising_logits_between_tiles(mt):
    """The forward rescales O only when a row's max grows by more than a
    slack (32 log2 units for bf16, 15 for fp16, whose P must stay below 65504).
    Logits that step up by 15 (natural units, 21.6 in log2) after the first
    key tile and again later leave the slack without a rescale in bf16 and
    force one in fp16: forward and backward stay finite and match the oracle
    at the head dims of the non-deferred softmax (80, 128, 160, 256), with a
    per-head and a head-broadcast (staged) bias."""
    for dt in (torch.float16, torch.bfloat16):
        for D, bc in ((80, False), (128, True), (160, True), (256, False)):
            L, H = 300, 8
            bias = torch.full((L, 1 if bc else H, L), -20.0)
            bias[:, :, 64:] = -5.0
            bias[:, :, 200:] = 10.0
            name = f"rising logits {dt} D={D} {'broadcast' if bc else 'per-head'} bias"
            _fwd(mt, name, [L], [L], H, 2 if bc else H, D, dt, bias=bias)
            _bwd(mt, "bwd " + name, [L], [L], H, 2 if bc else H, D, dt, 6e-3 if dt == torch.float16 else 4e-2,
                 bias=bias)


def test_generic_head_dims(mt):
    _fwd(mt, "D=96 causal", [2048], [2048], 12, 12, 96, torch.float16, causal=True)
    _fwd(mt, "D=96 bf16", [1500], [1500], 8, 8, 96, torch.bfloat16)
    _fwd(mt, "D=80", [2048], [2048], 8, 8, 80, torch.float16)
    _fwd(mt, "D=80 causal", [1500], [1500], 12, 12, 80, torch.float16, causal=True)
    _fwd(mt, "D=88", [2048], [2048], 8, 8, 88, torch.float16)
    _fwd(mt, "D=88 bf16 causal", [1500], [1500], 8, 8, 88, torch.bfloat16, causal=True)
    _fwd(mt, "D=80 ragged causal", [200, 700], [200, 700], 8, 8, 80, torch.float16, causal=True)


def test_mfma_padded_head_dims(mt):
    """Head dims 80/88/96 run the matrix-core kernels on the 128-wide tile
    (operand columns past D zero, output columns past D dropped)."""
    b, h = torch.bfloat16, torch.float16
    for D in (80, 88, 96):
        _fwd(mt, f"D={D} bf16 GQA causal ragged", [300, 77, 513], [300, 77, 513], 16, 4, D, b, causal=True)
        _fwd(mt, f"D={D} fp16 cross window", [64, 200], [333, 260], 8, 2, D, h, causal=True, window=100)
        _bwd(mt, f"bwd D={D} bf16 GQA ragged", [200, 91, 333], [200, 91, 333], 12, 4, D, b, 4e-2, causal=True)
        _bwd(mt, f"bwd D={D} fp16 window cross", [150], [410], 8, 8, D, h, 6e-3, causal=True, window=90)
        _bwd(mt, f"bwd D={D} fp16 per-head bias", [640], [640], 8, 4, D, h, 6e-3,
             bias=_make_bias(640, 8, 640, False))
        _bwd(mt, f"bwd D={D} bf16 broadcast bias causal", [512], [512], 8, 8, D, b, 4e-2, causal=True,
             bias=_make_bias(512, 8, 512, True))


def test_mpp_hooks_fp32_outputs(mt):
    """The reference's backward test entries _C.mpp_bwd_dq and _C.mpp_bwd_dkv
    (src/ext.mm:597-711) return fp32 dQ and (dK, dV) from the 16-bit kernels,
    given the forward's LSE and delta = rowsum(dO * O): checked against the
    oracle's gradients on the one-wave-per-SIMD dK/dV kernel (D = 128 causal
    GQA, D = 256 windowed) and the wave-pair kernel (a broadcast bias)."""
    cases = [("D=128 bf16 causal GQA 8/2 ragged", [300, 77, 513], 8, 2, 128, torch.bfloat16, True, 0, None, 4e-2),
             ("D=256 fp16 window 200", [400, 250], 4, 4, 256, torch.float16, True, 200, None, 6e-3),
             ("D=128 fp16 broadcast bias", [384], 8, 8, 128, torch.float16, False, 0,
              _make_bias(384, 8, 384, True), 6e-3)]
    for name, lens, Hq, Hkv, D, dt, causal, window, bias, atol in cases:
        _banner(f"mpp hooks {name}")
        q, k, v = _inputs(lens, lens, Hq, Hkv, D, dt, 0)
        dout = randn((sum(lens), Hq, D), dt, torch.Generator().manual_seed(1))
        cu = cu_of(lens)
        scale = 1.0 / math.sqrt(D)
        qd, kd, vd, dd, cud = (t.cuda() for t in (q, k, v, dout, cu))
        bd = None if bias is None else bias.cuda()
        lse = torch.empty(sum(lens), Hq, dtype=torch.float32, device="cuda")
        o = mt._C.varlen_attention(qd, kd, vd, cud, cud, max(lens), scale, causal, window, lse, bd)
        delta = (o.float() * dd.float()).sum(-1)
        dq = mt._C.mpp_bwd_dq(qd, kd, vd, dd, lse, delta, cud, cud, max(lens), scale, causal, window, bd)
        dk, dv = mt._C.mpp_bwd_dkv(qd, kd, vd, dd, lse, delta, cud, cud, max(lens), scale, causal, window, bd)
        torch.cuda.synchronize()
        _, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cu, cu, None, causal, window, bias)
        errs = {}
        for nm, a, b in (("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
            assert a.dtype == torch.float32 and torch.isfinite(a).all(), f"{name}: {nm}"
            errs[nm] = (a.cpu() - b).abs().max().item()
            errs[nm + "_rms_rel"] = err_stats(a, b, dt)["rms_rel"]
        print("  " + " ".join(f"{k_}={v_:.3e}" for k_, v_ in errs.items()) + f" atol={atol}", flush=True)
        for nm in ("dQ", "dK", "dV"):
            assert errs[nm] < atol, f"{name}: {nm} {errs}"
            assert errs[nm + "_rms_rel"] <= RMS_BOUND[dt], f"{name}: {nm} rms_rel {errs[nm + '_rms_rel']:.3e}"


def test_windowed_backward_walk(mt):
    """Under a sliding window each dK/dV workgroup walks its query tiles
    from the tile whose index is a multiple of the walk's length and wraps
    to the top (first_q_tile, bwd_common.h): several key blocks per
    sequence with different starting tiles, windows that are not multiples
    of the tile sizes, cross lengths, GQA, on the one-wave-per-SIMD kernel
    (D = 128, 256; single key blocks under a window) and the wave-pair
    kernel (with a bias)."""
    b, h = torch.bfloat16, torch.float16
    _bwd(mt, "bwd window 700 GQA 8/2 ragged D=128", [1500, 2300], [1500, 2300], 8, 2, 128, b, 4e-2,
         causal=True, window=700)
    _bwd(mt, "bwd window 333 cross D=128 fp16", [900, 400], [1300, 1000], 8, 8, 128, h, 6e-3, causal=True,
         window=333)
    _bwd(mt, "bwd window 500 D=256", [1200], [1200], 4, 2, 256, b, 4e-2, causal=True, window=500)
    _bwd(mt, "bwd window 600 broadcast bias D=128", [1100], [1100], 8, 2, 128, h, 6e-3, causal=True,
         window=600, bias=_make_bias(1100, 8, 1100, True))


def test_mfma_wide_head_dims(mt):
    """Head dims 160/256 run the matrix-core kernels on 256-wide tiles: one
    launch per kernel where the registers allow it (every forward except the
    biased D = 256 one, dQ, dK/dV at D = 160), else 128-column slices; dK/dV
    at D = 256 without a bias runs all 256 columns in one pass (one wave per
    SIMD, 32 keys per wave)."""
    b, h = torch.bfloat16, torch.float16
    _bwd(mt, "bwd D=256 fp16 non-causal ragged MHA", [129, 300, 31], [129, 300, 31], 8, 8, 256, h, 6e-3)
    for D in (160, 256):
        _fwd(mt, f"D={D} bf16 GQA causal ragged", [300, 77, 513], [300, 77, 513], 16, 4, D, b, atol=4e-2,
             causal=True)
        _fwd(mt, f"D={D} fp16 cross window", [64, 200], [333, 260], 8, 2, D, h, causal=True, window=100)
        _bwd(mt, f"bwd D={D} bf16 GQA ragged", [200, 91, 333], [200, 91, 333], 12, 4, D, b, 4e-2, causal=True)
        _bwd(mt, f"bwd D={D} fp16 window cross", [150], [410], 8, 8, D, h, 6e-3, causal=True, window=90)
        _bwd(mt, f"bwd D={D} fp16 per-head bias", [640], [640], 8, 4, D, h, 6e-3,
             bias=_make_bias(640, 8, 640, False))
        _bwd(mt, f"bwd D={D} bf16 broadcast bias causal", [512], [512], 8, 8, D, b, 4e-2, causal=True,
             bias=_make_bias(512, 8, 512, True))


def test_large_head_dims(mt):
    _fwd(mt, "D=160 full", [2048], [2048], 8, 8, 160, torch.float16)
    _fwd(mt, "D=160 causal", [1500], [1500], 12, 12, 160, torch.float16, causal=True)
    _fwd(mt, "D=256 full", [2048], [2048], 8, 8, 256, torch.float16)
    _fwd(mt, "D=256 causal", [1024], [1024], 12, 12, 256, torch.float16, causal=True)
    _fwd(mt, "D=256 bf16", [1500], [1500], 8, 8, 256, torch.bfloat16, atol=4e-2, causal=True)


# decode / split-KV (tests/test_correctness.py:347-353)
def test_decode_cases(mt):
    _fwd(mt, "decode B1 kv8192", [1], [8192], 12, 12, 128, torch.float16, causal=True)
    _fwd(mt, "decode B1 noncausal", [1], [8192], 8, 8, 128, torch.float16)
    _fwd(mt, "decode B4 ragged", [1, 1, 1, 1], [8192, 4000, 6000, 2048], 8, 8, 128, torch.float16,
         causal=True)
    _fwd(mt, "decode B1 D64", [1], [4096], 8, 8, 64, torch.float16, causal=True)
    _fwd(mt, "decode bf16", [1], [5000], 8, 8, 128, torch.bfloat16, causal=True)
    _fwd(mt, "decode GQA B1", [1], [8192], 8, 2, 128, torch.float16, causal=True)
    _fwd(mt, "decode few-q (spec)", [4], [8000], 8, 8, 128, torch.float16, causal=True)
    _fwd(mt, "decode GQA 64/8 few-q", [3, 2], [9000, 4100], 64, 8, 128, torch.bfloat16, causal=True)


def test_decode_small_chunks(mt, monkeypatch):
    """The automatic split-KV path with 256-key chunks: many chunks per
    sequence, a partial last chunk, KV lengths below one chunk, an empty
    sequence, and speculative (q_len > 1) rows, all against the oracle."""
    from mtlattn_amd import capi
    monkeypatch.setenv("MTLATTN_DECODE_CHUNK", "256")
    q_lens, kv_lens = [1, 1, 1, 1, 1], [2048, 300, 0, 4097, 5800]
    q, k, v = _inputs(q_lens, kv_lens, 8, 2, 128, torch.bfloat16, seed=11)
    p = capi.problem_for(q.cuda(), k.cuda(), cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda"), 1, 0.1, causal=True)
    assert capi.lib().mtlattn_decode_num_splits(p) == sum(kv_lens) // 256 + len(kv_lens) + 1   # routed, chunked
    _fwd(mt, "decode 256-key chunks, ragged + empty", q_lens, kv_lens, 8, 2, 128, torch.bfloat16, causal=True,
         seed=11)
    _fwd(mt, "decode 256-key chunks, q_len 1-3 GQA 16/2", [2, 3, 1], [3000, 2600, 4100], 16, 2, 128,
         torch.float16, causal=True, seed=12)
    _fwd(mt, "decode 256-key chunks, non-causal D=64", [1, 1], [2304, 2560], 8, 8, 64, torch.bfloat16, seed=13)


def _decode_routed(q_lens, kv_lens, Hq, Hkv, D, window=0, bias=None, causal=True):
    from mtlattn_amd import capi
    q = torch.empty((sum(q_lens), Hq, D), dtype=torch.bfloat16, device="cuda")
    k = torch.empty((sum(kv_lens), Hkv, D), dtype=torch.bfloat16, device="cuda")
    p = capi.problem_for(q, k, cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda"), max(q_lens), 0.1, causal=causal,
                         window=window, bias=None if bias is None else bias.cuda())
    return capi.lib().mtlattn_decode_num_splits(p)


def test_decode_window_bias(mt, monkeypatch):
    """Sliding window and additive bias on the split-KV decode path (the
    reference sends both to its flash forward, src/ext.mm:372-374): the
    window's equal splits cover only the band, rows' bands are masked per
    element, the bias is added per (row, key). Every case is checked to be
    routed to split-KV, then compared with the oracle (O and LSE)."""
    h, b = torch.float16, torch.bfloat16
    cases = [
        ("window 2500, ragged + empty, q_len 1-2", [1, 1, 2, 1], [9000, 5000, 3000, 0], 8, 2, 128, h, True, 2500, None),
        ("window wider than the KV", [1, 1], [4000, 2600], 8, 8, 128, b, True, 6000, None),
        ("window non-causal D=64", [1, 3], [7000, 5000], 8, 8, 64, b, False, 3000, None),
        ("bias per head", [1, 1], [8192, 4000], 8, 8, 128, h, True, 0, "head"),
        ("bias broadcast GQA 16/2, q_len 3", [3, 1], [6000, 5000], 16, 2, 128, b, True, 0, "bcast"),
        ("window + bias GQA", [2, 1], [9000, 4500], 8, 2, 128, h, True, 2100, "head"),
    ]
    for chunk in (None, "256"):
        if chunk:
            monkeypatch.setenv("MTLATTN_DECODE_CHUNK", chunk)
        for name, ql, kl, hq, hkv, d, dt, causal, w, bk in cases:
            bias = None
            if bk is not None:
                bias = _make_bias(sum(ql), 1 if bk == "bcast" else hq, max(kl), bk == "bcast", seed=len(name))
            assert _decode_routed(ql, kl, hq, hkv, d, w, bias, causal) > 0, f"{name}: not routed to split-KV"
            _fwd(mt, f"decode {name} (chunk {chunk or 'auto'})", ql, kl, hq, hkv, d, dt, causal=causal, window=w,
                 bias=bias, seed=len(name))


def test_decode_routed_training_step(mt):
    """A training call the forward routes to split-KV (q_len 1-4, long KV):
    the combine kernel's LSE feeds the prefill backward. The reference's
    gate ignores the LSE request and leaves it unwritten for such calls
    (src/ext.mm:372-390); here the forward's LSE, and every gradient, are
    checked against the oracle with the relative criterion (P ~ 1/kv_len
    makes absolute tolerances meaningless), GQA 64/8, bf16, with and without
    a window and a per-head bias."""
    b = torch.bfloat16
    q_lens, kv_lens = [1, 4, 2], [8192, 20000, 12000]
    cases = [("plain", 0, False), ("window 3000", 3000, False), ("bias", 0, True), ("window + bias", 2500, True)]
    for name, w, with_bias in cases:
        _banner(f"decode-routed training step, {name}")
        q, k, v = _inputs(q_lens, kv_lens, 64, 8, 128, b, seed=31 + w)
        g = torch.Generator().manual_seed(41 + w)
        dout = randn((sum(q_lens), 64, 128), b, g)
        bias = _make_bias(sum(q_lens), 64, max(kv_lens), False, seed=5) if with_bias else None
        assert _decode_routed(q_lens, kv_lens, 64, 8, 128, w, bias) > 0, f"{name}: not routed to split-KV"
        cq, ck = cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda")
        qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
        bd = None if bias is None else bias.cuda()
        out = mt.varlen_attention(qm, km, vm, cq, ck, max(q_lens), causal=True, window=w, attn_bias=bd)
        out.backward(dout.cuda())
        lse = torch.empty(sum(q_lens), 64, dtype=torch.float32, device="cuda")
        mt._C.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cq, ck, max(q_lens), 1 / math.sqrt(128), True, w,
                               lse, bd)
        torch.cuda.synchronize()
        ro, rl, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cu_of(q_lens), cu_of(kv_lens), None,
                                                            True, w, bias)
        lerr = (lse.cpu() - rl).abs().max().item()
        print(f"  lse_err={lerr:.3e}", flush=True)
        assert lerr < LSE_TOL[b], f"{name}: lse err {lerr}"
        # dK / dV of a key sum only the <= 4 x 8 (query, head) terms of its
        # group, P and dS rounded to bf16 (as the reference rounds them,
        # src/attn_mpp.metal:625-630); dS changes sign, so with so few terms
        # the roundings do not average out and the worst element sits at
        # 2-2.5x the output's own rounding floor (RMS error stays at the
        # suite's level). Those two are held to 3 x floor + 2e-2 instead of
        # 2 x floor + 2e-2; every tensor meets the RMS bound.
        for nm, a, r in (("out", out, ro), ("dQ", qm.grad, rq), ("dK", km.grad, rk), ("dV", vm.grad, rv)):
            st = err_stats(a, r, b)
            print(f"  {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e}", flush=True)
            if nm in ("dK", "dV"):
                assert st["rms_rel"] <= RMS_BOUND[b] and st["rel"] <= 3 * st["floor"] + 2e-2, f"{name}: {nm} {st}"
            else:
                assert st["ok_elem"], f"{name}: {nm} out of tolerance {st}"


# causal (tests/test_correctness.py:367-371)
def test_causal_cases(mt):
    _fwd(mt, "causal self D=128", [1024], [1024], 12, 12, 128, torch.float16, causal=True)
    _fwd(mt, "causal self bf16", [777], [777], 8, 8, 128, torch.bfloat16, causal=True)
    _fwd(mt, "causal ragged D=128", [33, 256, 1000], [33, 256, 1000], 12, 12, 128, torch.float16,
         causal=True)
    _fwd(mt, "causal cross (cached)", [64], [320], 8, 8, 128, torch.float16, causal=True)
    _fwd(mt, "causal self D=64", [200, 50], [200, 50], 16, 16, 64, torch.float16, causal=True)
    _fwd(mt, "causal q>kv (empty rows)", [300, 40], [100, 40], 8, 8, 128, torch.bfloat16, causal=True)


# GQA / MQA (tests/test_correctness.py:375-379)
def test_gqa_cases(mt):
    _fwd(mt, "GQA 12->4 D=128", [512], [512], 12, 4, 128, torch.float16)
    _fwd(mt, "MQA 8->1 D=128", [33, 300], [33, 300], 8, 1, 128, torch.float16)
    _fwd(mt, "GQA 8->2 causal", [400], [400], 8, 2, 128, torch.float16, causal=True)
    _fwd(mt, "MQA cross cached", [16], [512], 8, 1, 128, torch.float16, causal=True)
    _fwd(mt, "GQA 8->2 D=64", [200, 50], [200, 50], 8, 2, 64, torch.float16)
    _fwd(mt, "GQA 32->8 causal bf16", [700, 300], [700, 300], 32, 8, 128, torch.bfloat16, causal=True)


# sliding window (tests/test_correctness.py:383-387)
def test_window_cases(mt):
    _fwd(mt, "SWA causal w=128 D=128", [1024], [1024], 12, 12, 128, torch.float16, causal=True,
         window=128)
    _fwd(mt, "SWA causal ragged", [600, 50, 333], [600, 50, 333], 8, 8, 128, torch.float16,
         causal=True, window=64)
    _fwd(mt, "SWA w>=len (no-op)", [200], [200], 8, 8, 128, torch.float16, causal=True, window=512)
    _fwd(mt, "SWA non-causal band", [256], [256], 8, 8, 128, torch.float16, causal=False, window=48)
    _fwd(mt, "SWA D=64", [300, 40], [300, 40], 16, 16, 64, torch.float16, causal=True, window=80)
    _fwd(mt, "SWA GQA bf16", [900], [900], 32, 8, 128, torch.bfloat16, causal=True, window=300)


def test_window_cases_long(mt):
    """Windows of 1024 keys and more at the 128-wide head dims without a bias:
    the forward's 128-key tiles (shorter windows take 64-key ones), with the
    window's first tile rounded down to a tile boundary, ragged and cross
    (kv longer than q) sequences, and the non-causal band."""
    b, h = torch.bfloat16, torch.float16
    _fwd(mt, "SWA w=1500 GQA bf16 ragged", [3000, 1700], [3000, 1700], 16, 4, 128, b, causal=True,
         window=1500)
    _fwd(mt, "SWA w=1024 D=96 fp16", [2100], [2100], 8, 8, 96, h, causal=True, window=1024)
    _fwd(mt, "SWA w=1100 cross (kv longer)", [700, 300], [2500, 1300], 8, 2, 128, h, causal=True,
         window=1100)
    _fwd(mt, "SWA non-causal w=1200", [1800], [1800], 8, 2, 128, h, causal=False, window=1200)
    _bwd(mt, "bwd bf16 window 1500 GQA", [2000], [2000], 16, 4, 128, b, 4e-2, causal=True, window=1500)


# backward (tests/test_correctness.py:390-407)
def test_bwd_fp32(mt):
    f = torch.float32
    _bwd(mt, "bwd full fp32", [256], [256], 8, 8, 128, f, 1e-4)
    _bwd(mt, "bwd causal fp32", [256], [256], 8, 8, 128, f, 1e-4, causal=True)
    _bwd(mt, "bwd GQA+causal", [256], [256], 8, 2, 128, f, 1e-4, causal=True)
    _bwd(mt, "bwd window", [512], [512], 8, 8, 128, f, 1e-4, causal=True, window=64)
    _bwd(mt, "bwd varlen GQA", [128, 300], [128, 300], 12, 4, 128, f, 1e-4, causal=True)


def test_fp32_matrix_cores(mt, monkeypatch):
    """fp32 inputs at head dims up to 128 that are a multiple of 4 run the
    fp32 matrix-core kernels (v_mfma_f32_32x32x2_f32, columns padded to a
    multiple of 32): ragged GQA causal with a one-token sequence, cross
    lengths with a window, non-causal cross, per-head and broadcast bias,
    lengths around the 128-row workgroup and 32-row tile edges, forward and
    backward against the oracle; and both these kernels and the portable
    ones (MTLATTN_NO_MFMA) against the fp64 oracle with the fp32 criterion of
    tests/helpers.py (floor32 = the fp32 oracle's own error)."""
    f = torch.float32
    for D in (16, 36, 64, 100, 128):
        _fwd(mt, f"fp32 D={D} GQA causal ragged", [300, 77, 513, 1], [300, 77, 513, 1], 8, 2, D, f, causal=True)
        _bwd(mt, f"fp32 bwd D={D} GQA causal ragged", [200, 91, 333, 1], [200, 91, 333, 1], 8, 2, D, f, 1e-4,
             causal=True)
    _fwd(mt, "fp32 D=64 cross window", [64, 200], [333, 260], 8, 2, 64, f, causal=True, window=100)
    _bwd(mt, "fp32 bwd D=96 cross window", [150, 40], [410, 30], 4, 4, 96, f, 1e-4, causal=True, window=90)
    _bwd(mt, "fp32 bwd D=128 cross non-causal GQA", [100, 33], [250, 700], 8, 4, 128, f, 1e-4)
    _bwd(mt, "fp32 bwd D=64 tile edges", [1, 31, 32, 33, 127, 128, 129], [1, 31, 32, 33, 127, 128, 129], 4, 2, 64,
         f, 1e-4, causal=True)
    _bwd(mt, "fp32 bwd D=64 per-head bias", [640], [640], 8, 4, 64, f, 1e-4, bias=_make_bias(640, 8, 640, False))
    _bwd(mt, "fp32 bwd D=128 broadcast bias causal ragged", [300, 212], [300, 212], 8, 8, 128, f, 1e-4,
         causal=True, bias=_make_bias(512, 8, 300, True))
    _banner("fp32 matrix cores and portable kernels vs the fp64 oracle")
    lens = [700, 129]
    q, k, v = _inputs(lens, lens, 8, 2, 128, f, seed=4)
    dout = randn((sum(lens), 8, 128), f, torch.Generator().manual_seed(5))
    cu = cu_of(lens, "cuda")
    res = []
    for env in ("0", "1"):
        monkeypatch.setenv("MTLATTN_NO_MFMA", env)
        qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
        out = mt.varlen_attention(qm, km, vm, cu, cu, max(lens), causal=True, window=300)
        out.backward(dout.cuda())
        torch.cuda.synchronize()
        res.append([t.detach().cpu() for t in (out, qm.grad, km.grad, vm.grad)])
    monkeypatch.delenv("MTLATTN_NO_MFMA")
    args = (q, k, v, dout, cu_of(lens), cu_of(lens), None, True, 300, None)
    r64 = oracle.varlen_forward_backward(*args, dtype=torch.float64)
    r32 = oracle.varlen_forward_backward(*args, dtype=torch.float32)
    for i, (nm, j) in enumerate((("out", 0), ("dQ", 2), ("dK", 3), ("dV", 4))):
        floor32 = err_stats(r32[j], r64[j], f)["rel"]
        for path, r in zip(("matrix cores", "portable"), res):
            st = err_stats(r[i], r64[j], f, floor32)
            print(f"  {nm} {path}: rel={st['rel']:.3e} floor32={floor32:.3e}", flush=True)
            assert st["ok_elem"], f"{nm} {path}: {st}"


def test_bwd_fp16(mt):
    h = torch.float16
    _bwd(mt, "bwd fp16 causal", [256], [256], 8, 8, 128, h, 5e-3, causal=True)
    _bwd(mt, "bwd fp16 varlen", [128, 300, 64], [128, 300, 64], 8, 8, 128, h, 5e-3, causal=True)
    _bwd(mt, "bwd fp16 varlen GQA", [200, 50, 333], [200, 50, 333], 12, 4, 128, h, 6e-3, causal=True)
    _bwd(mt, "bwd fp16 window", [512], [512], 8, 8, 128, h, 5e-3, causal=True, window=64)
    _bwd(mt, "bwd fp16 D=64", [200, 50], [200, 50], 8, 8, 64, h, 5e-3, causal=True)
    _bwd(mt, "bwd fp16 D=96 GQA", [256], [256], 8, 2, 96, h, 6e-3, causal=True)
    _bwd(mt, "bwd fp16 D=80", [256], [256], 8, 8, 80, h, 6e-3, causal=True)
    _bwd(mt, "bwd fp16 D=88 GQA", [200, 56], [200, 56], 8, 2, 88, h, 6e-3, causal=True)
    _bwd(mt, "bwd fp16 D=160", [512], [512], 8, 8, 160, h, 6e-3, causal=True)
    _bwd(mt, "bwd fp16 D=256", [512], [512], 8, 8, 256, h, 6e-3, causal=True)


def test_bwd_d64_paths(mt):
    """Head dim 64 backward without a bias runs its own dK/dV kernel (every
    wave computing all four products for its keys, 4-wave workgroups) and
    4-wave dQ workgroups: window band, cross lengths (kv longer and shorter
    than q, causal end-aligned), GQA causal, tiny and odd lengths around the
    128-key workgroup and 64-query stage edges, fp16 and bf16."""
    h, b = torch.float16, torch.bfloat16
    _bwd(mt, "D=64 window", [700, 300], [700, 300], 8, 8, 64, b, 4e-2, causal=True, window=100)
    _bwd(mt, "D=64 window non-causal", [500], [500], 4, 4, 64, h, 5e-3, window=70)
    _bwd(mt, "D=64 cross non-causal GQA", [100, 33], [250, 700], 8, 4, 64, h, 5e-3)
    _bwd(mt, "D=64 cross causal", [100, 257, 300], [300, 257, 129], 8, 8, 64, b, 4e-2, causal=True)
    _bwd(mt, "D=64 GQA causal", [600, 130], [600, 130], 16, 4, 64, b, 4e-2, causal=True)
    _bwd(mt, "D=64 tiny and odd", [1, 17, 129, 128, 65], [1, 17, 129, 128, 65], 4, 4, 64, h, 5e-3)
    _bwd(mt, "D=64 tiny causal", [1, 2, 63, 64, 127], [1, 2, 63, 64, 127], 4, 2, 64, h, 5e-3, causal=True)


def test_bwd_bf16(mt):
    b = torch.bfloat16
    _bwd(mt, "bwd bf16 varlen", [180, 90], [180, 90], 8, 8, 128, b, 4e-2, causal=True)
    _bwd(mt, "bwd bf16 GQA 32/8 causal", [300, 200], [300, 200], 32, 8, 128, b, 4e-2, causal=True)
    _bwd(mt, "bwd bf16 non-causal cross", [100, 33], [250, 70], 8, 4, 128, b, 4e-2)
    _bwd(mt, "bwd bf16 window GQA", [700], [700], 16, 4, 128, b, 4e-2, causal=True, window=200)
    _bwd(mt, "bwd bf16 D=64 MHA", [400, 1000], [400, 1000], 4, 4, 64, b, 4e-2)


# additive bias (tests/test_correctness.py:412-427)
def test_bias_fwd(mt):
    h = torch.float16
    _fwd(mt, "bias fwd perhead D128", [1536], [1536], 8, 8, 128, h, bias=_make_bias(1536, 8, 1536, False))
    _fwd(mt, "bias fwd broadcast D128", [1536], [1536], 8, 8, 128, h, bias=_make_bias(1536, 8, 1536, True))
    _fwd(mt, "bias fwd causal D128", [1536], [1536], 12, 12, 128, h, causal=True,
         bias=_make_bias(1536, 12, 1536, False))
    _fwd(mt, "bias fwd ragged varlen", [200, 50, 1300], [200, 50, 1300], 8, 8, 128, h,
         bias=_make_bias(1550, 8, 1300, False))
    _fwd(mt, "bias fwd cross", [64], [900], 8, 8, 128, h, bias=_make_bias(64, 8, 900, False))
    _fwd(mt, "bias fwd SWA", [1536], [1536], 8, 8, 128, h, causal=True, window=128,
         bias=_make_bias(1536, 8, 1536, False))
    _fwd(mt, "bias fwd bf16", [1500], [1500], 8, 8, 128, torch.bfloat16, bias=_make_bias(1500, 8, 1500, True))
    _fwd(mt, "bias fwd D64", [2048], [2048], 12, 12, 64, h, bias=_make_bias(2048, 12, 2048, False))
    _fwd(mt, "bias fwd D96 causal", [2048], [2048], 8, 8, 96, h, causal=True,
         bias=_make_bias(2048, 8, 2048, False))
    _fwd(mt, "bias fwd D256", [1024], [1024], 8, 8, 256, h, atol=6e-3, bias=_make_bias(1024, 8, 1024, False))


def test_bias_bwd(mt):
    h = torch.float16
    _bwd(mt, "bias bwd perhead D128", [1280], [1280], 8, 8, 128, h, 5e-3, bias=_make_bias(1280, 8, 1280, False))
    _bwd(mt, "bias bwd broadcast D128", [1280], [1280], 8, 8, 128, h, 5e-3, bias=_make_bias(1280, 8, 1280, True))
    _bwd(mt, "bias bwd causal D128", [1280], [1280], 12, 12, 128, h, 5e-3, causal=True,
         bias=_make_bias(1280, 12, 1280, False))
    _bwd(mt, "bias bwd GQA causal", [1024], [1024], 8, 2, 128, h, 6e-3, causal=True,
         bias=_make_bias(1024, 8, 1024, False))
    _bwd(mt, "bias bwd ragged", [128, 700], [128, 700], 8, 8, 128, h, 5e-3, bias=_make_bias(828, 8, 700, False))
    _bwd(mt, "bias bwd D64 bf16", [1280], [1280], 8, 8, 64, torch.bfloat16, 4e-2,
         bias=_make_bias(1280, 8, 1280, False))


def _misaligned(t):
    """A copy of `t` whose storage starts 4 bytes past a 16-byte boundary: the
    kernels then take the per-row (register) bias path."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    m = buf[1:].view(t.shape)
    m.copy_(t)
    assert m.data_ptr() % 16 != 0
    return m


def test_bias_staged_broadcast(mt):
    """Head-broadcast bias with GQA groups of 4 or 8 heads (32 or 64 query rows
    per workgroup) is staged in LDS with the K/V tiles. Checked against the
    oracle and bitwise against the per-row path (the same bias at a misaligned
    address), including tiles that cross the bias width and a bias narrower
    than the keys (missing columns read as 0)."""
    cases = [
        # name, q_lens, kv_lens, Hq, Hkv, D, dtype, causal, window, bias cols
        ("g=4 D128 bf16 causal ragged", [300, 77, 513], [300, 77, 513], 32, 8, 128, torch.bfloat16, True, 0, 516),
        ("g=8 D128 fp16 causal window", [700], [700], 16, 2, 128, torch.float16, True, 200, 704),
        ("g=4 D64 fp16 non-causal ragged", [200, 650], [200, 650], 8, 2, 64, torch.float16, False, 0, 652),
        ("g=4 D96 bf16 cross", [64, 130], [900, 300], 8, 2, 96, torch.bfloat16, False, 0, 900),
        ("g=4 D128 fp16 bias narrower than keys", [400], [400], 8, 2, 128, torch.float16, True, 0, 260),
    ]
    for name, ql, kl, hq, hkv, d, dt, causal, window, cols in cases:
        g = torch.Generator().manual_seed(len(name))
        bias = torch.randn((sum(ql), 1, cols), generator=g)
        bias[:, :, ::7] -= 30.0
        full = torch.zeros((sum(ql), 1, max(max(kl), cols)))
        full[:, :, :cols] = bias                       # missing columns read as 0
        # the oracle takes the zero-padded bias; the kernels the narrow one
        _banner(f"staged bias: {name}")
        q, k, v = _inputs(ql, kl, hq, hkv, d, dt, seed=3)
        cq, ck = cu_of(ql), cu_of(kl)
        scale = 1.0 / math.sqrt(d)
        outs = []
        for b in (bias.cuda(), _misaligned(bias.cuda())):
            lse = torch.empty(sum(ql), hq, dtype=torch.float32, device="cuda")
            o = mt._C.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), max(ql), scale, causal,
                                       window, lse, b)
            outs.append((o.cpu(), lse.cpu()))
        torch.cuda.synchronize()
        assert torch.equal(outs[0][0], outs[1][0]), f"{name}: staged and per-row bias outputs differ"
        assert torch.equal(outs[0][1], outs[1][1]), f"{name}: staged and per-row bias LSE differ"
        ref, ref_lse = oracle.varlen_forward(q, k, v, cq, ck, scale, causal, window, full[:, :, :max(kl)])
        err = (outs[0][0].float() - ref).abs().max().item()
        fin = torch.isfinite(ref_lse)
        lerr = (outs[0][1][fin] - ref_lse[fin]).abs().max().item()
        print(f"  bitwise equal to the per-row path; max_err={err:.3e} lse_err={lerr:.3e}", flush=True)
        assert err < REF_ATOL[dt], f"{name}: max_err {err}"
        assert lerr < LSE_TOL[dt], f"{name}: lse err {lerr}"
        # backward: dQ reads the staged tile too (dK/dV the per-row path)
        dout = randn((sum(ql), hq, d), dt, torch.Generator().manual_seed(11))
        grads = []
        for b in (bias.cuda(), _misaligned(bias.cuda())):
            qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
            o = mt.varlen_attention(qm, km, vm, cq.cuda(), ck.cuda(), max(ql), causal=causal, window=window,
                                    attn_bias=b)
            o.backward(dout.cuda())
            grads.append([t.grad.cpu() for t in (qm, km, vm)])
        for nm, x, y in zip(("dQ", "dK", "dV"), grads[0], grads[1]):
            assert torch.equal(x, y), f"{name}: staged and per-row bias {nm} differ"
        _, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cq, ck, None, causal, window,
                                                          full[:, :, :max(kl)])
        gerr = max((x.float() - r).abs().max().item() for x, r in zip(grads[0], (rq, rk, rv)))
        gtol = 4e-2 if dt == torch.bfloat16 else 6e-3
        print(f"  grads bitwise equal to the per-row path; grad_err={gerr:.3e} (tol {gtol})", flush=True)
        assert gerr < gtol, f"{name}: grad err {gerr}"


def test_empty_sequences(mt):
    """Zero-length query and key sequences inside a batch (repeated
    cu_seqlens entries), queries with no keys (O = 0, LSE = -inf, zero
    gradients) and an empty batch, forward and backward on the matrix-core and
    portable kernels."""
    cases = [
        ("bf16 D128 GQA non-causal", [0, 300, 5, 129, 0], [50, 300, 0, 129, 0], 8, 2, 128, torch.bfloat16, False),
        ("fp16 D64 causal", [0, 200, 7, 64], [40, 200, 0, 64], 4, 4, 64, torch.float16, True),
        ("fp32 D64 non-causal (fp32 matrix cores)", [0, 30, 5, 12], [50, 30, 0, 12], 4, 2, 64, torch.float32,
         False),
        ("fp32 D66 causal (portable)", [0, 30, 5, 12], [50, 30, 0, 12], 4, 2, 66, torch.float32, True),
    ]
    for name, ql, kl, hq, hkv, d, dt, causal in cases:
        _banner(f"empty sequences: {name}")
        q, k, v = _inputs(ql, kl, hq, hkv, d, dt, seed=8)
        cq, ck = cu_of(ql), cu_of(kl)
        dout = randn((sum(ql), hq, d), dt, torch.Generator().manual_seed(13))
        qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
        lse = torch.empty(sum(ql), hq, dtype=torch.float32, device="cuda")
        o1 = mt._C.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), max(ql), 1 / math.sqrt(d),
                                    causal, 0, lse, None)
        out = mt.varlen_attention(qm, km, vm, cq.cuda(), ck.cuda(), max(ql), causal=causal)
        out.backward(dout.cuda())
        torch.cuda.synchronize()
        ro, rl, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cq, ck, None, causal, 0, None)
        assert torch.equal(torch.isfinite(lse.cpu()), torch.isfinite(rl)), f"{name}: LSE -inf pattern"
        for nm, a, r in (("out", out, ro), ("dQ", qm.grad, rq), ("dK", km.grad, rk), ("dV", vm.grad, rv)):
            st = err_stats(a, r, dt)
            print(f"  {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} max_abs={st['max_abs']:.3e}", flush=True)
            assert torch.isfinite(a.float()).all(), f"{name}: non-finite {nm}"
            assert st["ok_elem"] or st["max_abs"] < REF_ATOL[dt], f"{name}: {nm} {st}"
        assert torch.equal(o1.cpu(), out.detach().cpu()), f"{name}: _C and public API disagree"
        # keys no query sees (the empty-query sequence's 50 keys) get exactly zero gradient
        assert km.grad[:kl[0]].abs().max().item() == 0.0 and vm.grad[:kl[0]].abs().max().item() == 0.0
    _banner("empty sequences: empty batch")
    q = torch.zeros((0, 8, 128), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    k = torch.zeros((0, 2, 128), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    v = torch.zeros((0, 2, 128), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    cu = torch.zeros(3, dtype=torch.int32, device="cuda")
    out = mt.varlen_attention(q, k, v, cu, cu, 0, causal=True)
    out.backward(torch.zeros_like(out))
    torch.cuda.synchronize()
    assert out.shape == (0, 8, 128) and q.grad.shape == q.shape and k.grad.shape == k.shape


def test_scale_modes(mt):
    """Explicit scales (mtlattn/__init__.py:82-83 only defaults it): a custom
    positive scale takes the raw-max softmax (with a bias, the biased raw max;
    with a head-broadcast bias and GQA, the staged bias), zero and negative
    scales the explicitly scaled one, on the prefill kernels forward and
    backward and on the split-KV decode path."""
    cases = [
        # name, q_lens, kv_lens, Hq, Hkv, D, dtype, causal, scale, bias kind
        ("scale 0.3 GQA causal", [300, 129], [300, 129], 8, 2, 128, torch.bfloat16, True, 0.3, None),
        ("scale 0.3 broadcast bias (staged)", [300, 129], [300, 129], 8, 2, 128, torch.float16, True, 0.3, "bcast"),
        ("scale -0.07 per-head bias", [200, 77], [200, 77], 4, 4, 64, torch.float16, False, -0.07, "head"),
        ("scale -0.07 GQA causal", [250], [250], 8, 2, 128, torch.bfloat16, True, -0.07, None),
        ("scale 0 broadcast bias", [150, 90], [150, 90], 8, 2, 128, torch.float16, True, 0.0, "bcast"),
    ]
    for name, ql, kl, hq, hkv, d, dt, causal, scale, bk in cases:
        _banner(f"scale modes: {name}")
        q, k, v = _inputs(ql, kl, hq, hkv, d, dt, seed=5)
        cq, ck = cu_of(ql), cu_of(kl)
        bias = None
        if bk is not None:
            bias = _make_bias(sum(ql), hq, max(kl), bk == "bcast", seed=9)
        dout = randn((sum(ql), hq, d), dt, torch.Generator().manual_seed(12))
        qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
        out = mt.varlen_attention(qm, km, vm, cq.cuda(), ck.cuda(), max(ql), scale=scale, causal=causal,
                                  attn_bias=None if bias is None else bias.cuda())
        out.backward(dout.cuda())
        torch.cuda.synchronize()
        ro, _, rq, rk, rv = oracle.varlen_forward_backward(q, k, v, dout, cq, ck, scale, causal, 0, bias)
        # the relative criterion (max|err| and RMS(err) against RMS(ref)):
        # gradients grow with the scale, absolute tolerances do not
        for nm, a, r in (("out", out, ro), ("dQ", qm.grad, rq), ("dK", km.grad, rk), ("dV", vm.grad, rv)):
            st = err_stats(a, r, dt)
            print(f"  {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e} "
                  f"max_abs={st['max_abs']:.3e}", flush=True)
            assert st["ok_elem"], f"{name}: {nm} out of tolerance {st}"
    # split-KV decode with explicit scales (q_len 1, long KV: the split path)
    for scale in (0.3, -0.05, 0.0):
        _banner(f"scale modes: decode scale {scale}")
        ql, kl = [1, 1, 1], [6000, 9000, 4100]
        q, k, v = _inputs(ql, kl, 16, 2, 128, torch.bfloat16, seed=6)
        cq, ck = cu_of(ql), cu_of(kl)
        out = mt.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), 1, scale=scale,
                                  causal=True).cpu()
        ref, _ = oracle.varlen_forward(q, k, v, cq, ck, scale, True, 0, None)
        err = (out.float() - ref).abs().max().item()
        print(f"  max_err={err:.3e}", flush=True)
        assert err < REF_ATOL[torch.bfloat16], f"decode scale {scale}: err {err}"


# SDPA adapter, padding-mask packing, mask -> bias (tests/test_correctness.py:437-448)
def test_sdpa_adapter(mt):
    for (B, Hq, Hkv, N, causal) in [(2, 8, 8, 1024, False), (1, 8, 2, 2048, False), (2, 12, 12, 512, True)]:
        _banner(f"sdpa B{B} {Hq}/{Hkv} N{N} causal={causal}")
        g = torch.Generator().manual_seed(0)
        q = randn((B, Hq, N, 128), torch.float16, g)
        k = randn((B, Hkv, N, 128), torch.float16, g)
        v = randn((B, Hkv, N, 128), torch.float16, g)
        gg = Hq // Hkv
        ref = torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float().repeat_interleave(gg, 1), v.float().repeat_interleave(gg, 1),
            is_causal=causal)
        out = mt.sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=causal).cpu().float()
        err = (out - ref).abs().max().item()
        print(f"  max_err={err:.3e}", flush=True)
        assert err < 5e-3


def test_padding_mask(mt):
    import torch.nn.functional as F
    for (B, H, N, Ls, causal) in [(4, 8, 1024, [1024, 800, 500, 1024], False), (3, 12, 1024, [1024, 700, 400], True)]:
        _banner(f"pad mask B{B} causal={causal}")
        g = torch.Generator().manual_seed(0)
        q = randn((B, H, N, 128), torch.float16, g)
        k = randn((B, H, N, 128), torch.float16, g)
        v = randn((B, H, N, 128), torch.float16, g)
        pack = lambda x: torch.cat([x[b, :, :Ls[b], :].transpose(0, 1) for b in range(B)], 0)
        ref, _ = oracle.varlen_forward(pack(q), pack(k), pack(v), cu_of(Ls), cu_of(Ls), causal=causal)
        mask = torch.zeros(B, 1, 1, N, dtype=torch.bool)
        for b, Lb in enumerate(Ls):
            mask[b, 0, 0, :Lb] = True
        mt.replace_sdpa(min_seqlen=1)
        try:
            out = F.scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda(),
                                                 is_causal=causal).cpu().float()
        finally:
            mt.restore_sdpa()
        outp = torch.cat([out[b, :, :Ls[b], :].transpose(0, 1) for b in range(B)], 0)
        err = (outp - ref).abs().max().item()
        pad_zero = all(out[b, :, Ls[b]:, :].abs().max().item() == 0 for b in range(B) if Ls[b] < N)
        print(f"  max_err={err:.3e} padded_rows_zero={pad_zero}", flush=True)
        assert err < 5e-3 and pad_zero


def test_pack_unpack_padded(mt):
    """Device pack/unpack of the SDPA adapter: valid prefixes land at
    cu[b] + n, cu is the prefix sum, padded tokens fill the tail rows, and the
    unpack restores the dense layout with zeros for padding (bitwise)."""
    for dtype, (B, H, N, D), lens in [(torch.bfloat16, (4, 3, 40, 64), [40, 0, 17, 33]),
                                      (torch.float32, (3, 2, 9, 24), [5, 9, 1]),
                                      (torch.float16, (2, 4, 16, 20), [0, 0])]:
        _banner(f"pack/unpack {dtype} B{B} H{H} N{N} D{D} lens={lens}")
        g = torch.Generator().manual_seed(3)
        base = randn((B, N, H, D), dtype, g).cuda()
        x = base.permute(0, 2, 1, 3)                       # strided [B, H, N, D] view
        L = torch.tensor(lens, dtype=torch.int32, device="cuda")
        packed, cu = mt._C.pack_padded(x, L)
        torch.cuda.synchronize()
        ref_cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
        assert torch.equal(cu.cpu(), ref_cu)
        xc = x.cpu()
        want = torch.cat([xc[b, :, :lens[b], :].transpose(0, 1) for b in range(B)], 0)
        assert torch.equal(packed[:int(ref_cu[-1])].cpu(), want)
        pads = torch.cat([xc[b, :, lens[b]:, :].transpose(0, 1) for b in range(B)], 0)
        assert torch.equal(packed[int(ref_cu[-1]):].cpu(), pads)     # a permutation: nothing lost
        out = mt._C.unpack_padded(packed, cu, L, B, N).cpu()
        keep = (torch.arange(N)[None, :] < torch.tensor(lens)[:, None])[:, None, :, None]
        assert torch.equal(out, torch.where(keep, xc, torch.zeros((), dtype=dtype)))


def test_sdpa_mask(mt):
    import torch.nn.functional as F
    for (B, H, N, bool_mask, bh) in [(2, 8, 1024, False, False), (2, 8, 1024, False, True),
                                     (2, 8, 1024, True, False), (1, 12, 2048, True, True)]:
        _banner(f"sdpa mask B{B} bool={bool_mask} head_broadcast={bh}")
        g = torch.Generator().manual_seed(0)
        q = randn((B, H, N, 128), torch.float16, g)
        k = randn((B, H, N, 128), torch.float16, g)
        v = randn((B, H, N, 128), torch.float16, g)
        hb = 1 if bh else H
        if bool_mask:
            m = torch.rand((B, hb, N, N), generator=g) > 0.3
            m[..., 0] = True
        else:
            m = torch.randn((B, hb, N, N), generator=g)
        out = mt.sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=m.cuda()).cpu().float()
        ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=m)
        err = (out - ref).abs().max().item()
        print(f"  max_err={err:.3e}", flush=True)
        assert err < 5e-3


def test_replace_sdpa_float_masks(mt):
    """Through replace_sdpa(), a float additive mask on equal query and key
    lengths is an additive bias, not a key-padding mask: its values must reach
    the kernels (the reference's padding shortcut takes any float mask without
    -inf entries as keep-all and drops them). A float mask of 0 / -inf with a
    kept key prefix per batch still takes the packed padding path (its padded
    query rows come back zero). Against torch's SDPA in fp32 on the CPU."""
    import torch.nn.functional as F
    orig = F.scaled_dot_product_attention
    mt.replace_sdpa(min_seqlen=1)
    try:
        g = torch.Generator().manual_seed(5)
        B, H, N, D = 2, 4, 300, 64
        q, k, v = (randn((B, H, N, D), torch.bfloat16, g) for _ in range(3))
        lens = [300, 171]
        pad = torch.full((B, 1, 1, N), float("-inf"))
        for b, L in enumerate(lens):
            pad[b, 0, 0, :L] = 0.0
        for name, m in (("float [B,H,N,N]", torch.randn((B, H, N, N), generator=g)),
                        ("float [1,1,N,N]", torch.randn((1, 1, N, N), generator=g)),
                        ("float padding 0/-inf", pad)):
            _banner(f"replace_sdpa {name}")
            out = F.scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), attn_mask=m.cuda()).cpu().float()
            ref = orig(q.float(), k.float(), v.float(), attn_mask=m)
            if name.startswith("float padding"):
                for b, L in enumerate(lens):
                    assert not out[b, :, L:].any(), "padded query rows must be zero"
                    ref[b, :, L:] = 0.0
            err = (out - ref).abs().max().item()
            print(f"  max_err={err:.3e}", flush=True)
            assert err < REF_ATOL[torch.bfloat16], f"{name}: err {err}"
    finally:
        mt.restore_sdpa()


def test_bias_per_sequence_rows(mt):
    """A 4-D bias [B or 1, H or 1, Nq, max_kv] is indexed by (sequence,
    sequence-local row) in place; rows past Nq read row Nq - 1. It must give
    bitwise the results of the 3-D bias gathered from it, forward and
    backward, on the matrix-core, portable and decode kernels."""
    cases = [
        ("bf16 D128 ragged causal", [300, 77, 513], [300, 77, 513], 8, 2, 128, torch.bfloat16, True, (3, 8), 513),
        ("fp16 D64 broadcast batch+head", [200, 650], [200, 650], 4, 4, 64, torch.float16, False, (1, 1), 650),
        ("bf16 rows past Nq clamp", [100, 260], [100, 260], 8, 8, 128, torch.bfloat16, True, (2, 1), 200),
        ("fp32 matrix-core kernels", [40, 90], [40, 90], 4, 2, 64, torch.float32, True, (2, 4), 90),
        ("fp32 portable kernels", [40, 90], [40, 90], 4, 2, 66, torch.float32, True, (2, 4), 90),
        ("decode q_len 2", [2, 1], [3000, 2500], 8, 2, 128, torch.bfloat16, True, (2, 8), 2),
    ]
    for name, ql, kl, hq, hkv, d, dt, causal, (bb, bh), nq in cases:
        _banner(f"per-sequence bias rows: {name}")
        q, k, v = _inputs(ql, kl, hq, hkv, d, dt, seed=len(name))
        g = torch.Generator().manual_seed(len(name) + 1)
        b4 = torch.randn((bb, bh, nq, max(kl)), generator=g)
        b4[..., ::5] -= 20.0
        rows = []
        for s, L in enumerate(ql):
            idx = torch.clamp(torch.arange(L), max=nq - 1)
            rows.append(b4[s if bb > 1 else 0][:, idx, :].transpose(0, 1))
        b3 = torch.cat(rows).contiguous()                       # [total_q, bh, max_kv]
        cq, ck = cu_of(ql, "cuda"), cu_of(kl, "cuda")
        dout = randn((sum(ql), hq, d), dt, g).cuda()
        res = []
        for bias in (b4, b3):
            qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
            out = mt.varlen_attention(qm, km, vm, cq, ck, max(ql), causal=causal, attn_bias=bias.cuda())
            out.backward(dout)
            res.append([t.detach().cpu() for t in (out, qm.grad, km.grad, vm.grad)])
        for nm, a, b in zip(("out", "dQ", "dK", "dV"), res[0], res[1]):
            assert torch.equal(a, b), f"{name}: {nm} differs between 4-D and gathered 3-D bias"
        ref, _ = oracle.varlen_forward(q, k, v, cu_of(ql), cu_of(kl), 1 / math.sqrt(d), causal, 0, b3)
        err = (res[0][0].float() - ref).abs().max().item()
        print(f"  bitwise equal; max_err vs oracle={err:.3e}", flush=True)
        assert err < REF_ATOL[dt]


def test_outlier_channels(mt):
    """Outlier channels x300 (tests/test_correctness.py:449-465): finite output,
    loose tolerance."""
    _banner("outlier channels bf16")
    g = torch.Generator().manual_seed(3)
    q = randn((2048, 12, 128), torch.bfloat16, g)
    q[:, :, 5] *= 300
    k = randn((2048, 12, 128), torch.bfloat16, g)
    k[:, :, 5] *= 300
    v = randn((2048, 12, 128), torch.bfloat16, g)
    cu = cu_of([1024, 1024])
    out = mt.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), 1024).cpu()
    ref, _ = oracle.varlen_forward(q, k, v, cu, cu)
    err = (out.float() - ref).abs().max().item()
    print(f"  max_err={err:.3e}", flush=True)
    assert torch.isfinite(out.float()).all() and err < 1e-1


# ---------------------------------------------------------------------------
# bookkeeping invariants beyond the reference's suite
# ---------------------------------------------------------------------------
def test_split_kv_invariants(mt):
    """Any split count gives the unsplit answer; split 1 is a plain forward."""
    _banner("split-KV num_splits sweep")
    q_lens, kv_lens = [1, 1, 1], [5000, 2100, 9001]
    q, k, v = _inputs(q_lens, kv_lens, 16, 4, 128, torch.bfloat16)
    cq, ck = cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda")
    ref, _ = oracle.varlen_forward(q, k, v, cu_of(q_lens), cu_of(kv_lens), causal=True)
    outs = []
    for ns in (1, 2, 7, 32, 100):
        o = mt._C.attn_splitkv(q.cuda(), k.cuda(), v.cuda(), cq, ck, 1, 1 / math.sqrt(128), True, ns).cpu()
        err = (o.float() - ref).abs().max().item()
        print(f"  ns={ns} max_err={err:.3e}", flush=True)
        assert err < 3e-2
        outs.append(o.float())
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 2e-2


def test_split_kv_window_bias(mt):
    """Explicit split counts with a window (splits of the band only) and a
    per-head bias, through _C.attn_splitkv's window/attn_bias arguments."""
    _banner("split-KV num_splits sweep, window + bias")
    q_lens, kv_lens = [1, 2, 1], [5000, 2100, 9001]
    q, k, v = _inputs(q_lens, kv_lens, 8, 2, 128, torch.bfloat16, seed=3)
    bias = _make_bias(sum(q_lens), 8, max(kv_lens), False, seed=4)
    cq, ck = cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda")
    for w, b in ((1500, None), (0, bias), (3000, bias)):
        ref, _ = oracle.varlen_forward(q, k, v, cu_of(q_lens), cu_of(kv_lens), 1 / math.sqrt(128), True, w, b)
        for ns in (1, 3, 16):
            o = mt._C.attn_splitkv(q.cuda(), k.cuda(), v.cuda(), cq, ck, 2, 1 / math.sqrt(128), True, ns, window=w,
                                   attn_bias=None if b is None else b.cuda()).cpu()
            err = (o.float() - ref).abs().max().item()
            print(f"  window={w} bias={b is not None} ns={ns} max_err={err:.3e}", flush=True)
            assert err < 3e-2


def _paged(k, v, kv_lens, page_size, seed):
    """Scatter contiguous K/V rows into randomly permuted pages of a cache
    [num_pages, page_size, Hkv, D] (two spare pages); block_table rows past a
    sequence's pages hold -1."""
    g = torch.Generator().manual_seed(seed)
    n_pages = [-(-L // page_size) for L in kv_lens]
    total = sum(n_pages) + 2
    perm = torch.randperm(total, generator=g)
    kc = torch.randn((total, page_size) + tuple(k.shape[1:]), generator=g).to(k.dtype)
    vc = torch.randn((total, page_size) + tuple(v.shape[1:]), generator=g).to(v.dtype)
    bt = torch.full((len(kv_lens), max(max(n_pages), 1)), -1, dtype=torch.int32)
    off, used = 0, 0
    for s, L in enumerate(kv_lens):
        for j in range(n_pages[s]):
            pg = int(perm[used])
            used += 1
            bt[s, j] = pg
            n = min(page_size, L - j * page_size)
            kc[pg, :n] = k[off + j * page_size: off + j * page_size + n]
            vc[pg, :n] = v[off + j * page_size: off + j * page_size + n]
        off += L
    return kc, vc, bt


def test_paged_decode(mt, monkeypatch):
    """Decode over a paged KV cache (no reference counterpart): pages of 16,
    48, 64 and 256 tokens in permuted order, against the oracle on the
    contiguous K/V (O and LSE), with causal, window and bias; and, with the
    split length fixed, bitwise equal to the contiguous split-KV path with
    the same split count."""
    cases = [
        ("ps16 ragged GQA", [1, 1, 2], [3000, 700, 5001], 8, 2, 128, torch.bfloat16, 16, True, 0, False),
        ("ps48 D64 non-causal", [1, 3], [2500, 4100], 8, 8, 64, torch.float16, 48, False, 0, False),
        ("ps64 window", [1, 1], [6000, 2000], 16, 2, 128, torch.bfloat16, 64, True, 1500, False),
        ("ps256 bias", [2, 1], [4500, 3333], 8, 2, 128, torch.float16, 256, True, 0, True),
        ("ps16 empty sequence", [1, 1], [0, 1234], 8, 8, 128, torch.bfloat16, 16, True, 0, False),
    ]
    for name, ql, kl, hq, hkv, d, dt, ps, causal, w, with_bias in cases:
        _banner(f"paged decode {name}")
        q, k, v = _inputs(ql, kl, hq, hkv, d, dt, seed=len(name))
        kc, vc, bt = _paged(k, v, kl, ps, seed=len(name))
        bias = _make_bias(sum(ql), hq, max(kl), False, seed=3) if with_bias else None
        cq, ck = cu_of(ql), cu_of(kl)
        lse = torch.empty(sum(ql), hq, dtype=torch.float32, device="cuda")
        out = mt.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), cq.cuda(), ck.cuda(), bt.cuda(), max(ql), max(kl),
                              causal=causal, window=w, attn_bias=None if bias is None else bias.cuda(),
                              lse_out=lse).cpu()
        ref, ref_lse = oracle.varlen_forward(q, k, v, cq, ck, 1 / math.sqrt(d), causal, w, bias)
        err = (out.float() - ref).abs().max().item()
        fin = torch.isfinite(ref_lse)
        assert torch.equal(torch.isfinite(lse.cpu()), fin), f"{name}: LSE -inf pattern"
        lerr = (lse.cpu()[fin] - ref_lse[fin]).abs().max().item()
        print(f"  max_err={err:.3e} lse_err={lerr:.3e}", flush=True)
        assert err < REF_ATOL[dt] and lerr < LSE_TOL[dt], name
    # fixed 256-key chunks on both paths: the same work items, the same
    # arithmetic as the contiguous automatic decode path
    monkeypatch.setenv("MTLATTN_DECODE_CHUNK", "256")
    ql, kl = [1, 1, 1], [3000, 1111, 4444]
    q, k, v = _inputs(ql, kl, 8, 2, 128, torch.bfloat16, seed=21)
    kc, vc, bt = _paged(k, v, kl, 32, seed=21)
    cq, ck = cu_of(ql, "cuda"), cu_of(kl, "cuda")
    assert _decode_routed(ql, kl, 8, 2, 128) > 0
    out = mt.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), cq, ck, bt.cuda(), 1, max(kl), causal=True).cpu()
    ref = mt.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cq, ck, 1, causal=True).cpu()
    assert torch.equal(out, ref), "paged != contiguous split-KV with the same chunks"


def test_paged_decode_shared_pages(mt):
    """Sequences that share pages (prefix caching, beam search): the sum of
    the logical KV lengths exceeds the cache's capacity, and every sequence
    must still see all of its keys. Each sequence reads the same 12 pages of
    a 12-page cache (4 x 3072 logical keys over 3072 cached rows), against
    the oracle on the equivalent contiguous K/V."""
    _banner("paged decode, 4 sequences sharing one cache's pages")
    ps, n_pages, B, hq, hkv, d = 256, 12, 4, 16, 2, 128
    g = torch.Generator().manual_seed(9)
    kc = randn((n_pages, ps, hkv, d), torch.bfloat16, g)
    vc = randn((n_pages, ps, hkv, d), torch.bfloat16, g)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = perm.repeat(B, 1)                                   # every sequence: the same pages
    kv_lens = [3072, 3000, 2049, 3072]
    q_lens = [1, 2, 1, 1]
    q = randn((sum(q_lens), hq, d), torch.bfloat16, g)
    kflat = kc[perm.long()].reshape(n_pages * ps, hkv, d)
    vflat = vc[perm.long()].reshape(n_pages * ps, hkv, d)
    k = torch.cat([kflat[:L] for L in kv_lens])
    v = torch.cat([vflat[:L] for L in kv_lens])
    assert sum(kv_lens) > n_pages * ps
    lse = torch.empty(sum(q_lens), hq, dtype=torch.float32, device="cuda")
    out = mt.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda"), bt.cuda(),
                          max(q_lens), max(kv_lens), causal=True, lse_out=lse).cpu()
    ref, ref_lse = oracle.varlen_forward(q, k, v, cu_of(q_lens), cu_of(kv_lens), 1 / math.sqrt(d), True)
    err = (out.float() - ref).abs().max().item()
    lerr = (lse.cpu() - ref_lse).abs().max().item()
    print(f"  max_err={err:.3e} lse_err={lerr:.3e}", flush=True)
    assert err < REF_ATOL[torch.bfloat16] and lerr < LSE_TOL[torch.bfloat16]


def test_binding_validation(mt):
    """Argument checks of the torch binding that need GPU tensors (no kernel
    runs): a block table narrower than max_seqlen_kv, and lse / delta of the
    wrong shape in the backward test entries."""
    _banner("binding validation")
    dev = "cuda"
    q = torch.zeros(2, 8, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(4, 16, 2, 128, dtype=torch.bfloat16, device=dev)
    cq, ck = cu_of([1, 1], dev), cu_of([40, 30], dev)
    bt = torch.zeros(2, 2, dtype=torch.int32, device=dev)    # 2 pages of 16 = 32 keys per sequence
    with pytest.raises(RuntimeError, match="block_table has 2 pages"):
        mt._C.paged_decode(q, kc, kc, cq, ck, bt, 1, 40, 0.1, True)
    k = torch.zeros(2, 2, 128, dtype=torch.bfloat16, device=dev)
    cu = cu_of([2], dev)
    good = torch.zeros(2, 8, device=dev)
    bad = torch.zeros(2, 4, device=dev)
    with pytest.raises(RuntimeError, match="lse must be"):
        mt._C.mpp_bwd_dq(q, k, k, q, bad, good, cu, cu, 2, 0.1)
    with pytest.raises(RuntimeError, match="delta must be"):
        mt._C.mpp_bwd_dkv(q, k, k, q, good, bad[:1], cu, cu, 2, 0.1)


def test_ragged_equals_per_sequence(mt):
    """A ragged batch equals per-sequence calls, bitwise (varlen bookkeeping)."""
    _banner("ragged == per-sequence (bitwise)")
    lens = [1, 77, 300, 64, 1000]
    q, k, v = _inputs(lens, lens, 8, 2, 128, torch.bfloat16, seed=5)
    cu = cu_of(lens)
    full = mt.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), max(lens), causal=True).cpu()
    off = 0
    for L in lens:
        one = cu_of([L], "cuda")
        o = mt.varlen_attention(q[off:off + L].cuda(), k[off:off + L].cuda(), v[off:off + L].cuda(), one, one, L,
                                causal=True).cpu()
        assert torch.equal(o, full[off:off + L]), f"len {L} differs"
        off += L


def test_rows_outside_sequences(mt):
    """cu_seqlens that start after row 0 and end before the last row: the
    rows no sequence owns get zero dQ / dK / dV (all three cleared in one
    launch), the owned rows match the oracle on the owned slice."""
    _banner("rows outside [cu[0], cu[B]) get zero gradient")
    lens = [100, 250]
    q0, k0, tail = 3, 5, 7
    g = torch.Generator().manual_seed(9)
    Hq, Hkv, D, dt = 8, 2, 128, torch.bfloat16
    q = randn((q0 + sum(lens) + tail, Hq, D), dt, g)
    k = randn((k0 + sum(lens) + tail, Hkv, D), dt, g)
    v = randn((k0 + sum(lens) + tail, Hkv, D), dt, g)
    dout = randn((q.shape[0], Hq, D), dt, g)
    cq = cu_of(lens) + q0
    ck = cu_of(lens) + k0
    qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
    out = mt.varlen_attention(qm, km, vm, cq.cuda(), ck.cuda(), max(lens), causal=True)
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    for name, gr, lo in (("dQ", qm.grad, q0), ("dK", km.grad, k0), ("dV", vm.grad, k0)):
        gr = gr.cpu()
        hi = lo + sum(lens)
        assert torch.count_nonzero(gr[:lo]) == 0 and torch.count_nonzero(gr[hi:]) == 0, f"{name} outside rows"
    sl_q, sl_k = slice(q0, q0 + sum(lens)), slice(k0, k0 + sum(lens))
    _, _, rq, rk, rv = oracle.varlen_forward_backward(q[sl_q], k[sl_k], v[sl_k], dout[sl_q], cu_of(lens), cu_of(lens),
                                                      None, True)
    errs = [(qm.grad.cpu()[sl_q].float() - rq).abs().max().item(),
            (km.grad.cpu()[sl_k].float() - rk).abs().max().item(),
            (vm.grad.cpu()[sl_k].float() - rv).abs().max().item()]
    print(f"  dQ/dK/dV max_err={errs}", flush=True)
    assert max(errs) < 4e-2


def test_determinism(mt):
    """Forward and backward are bitwise run-to-run deterministic (no atomics)."""
    _banner("determinism fwd+bwd")
    lens = [513, 1024, 77]
    q, k, v = _inputs(lens, lens, 16, 4, 128, torch.bfloat16, seed=9)
    g = torch.Generator().manual_seed(10)
    dout = randn((sum(lens), 16, 128), torch.bfloat16, g).cuda()
    cu = cu_of(lens, "cuda")
    res = []
    for _ in range(2):
        qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
        o = mt.varlen_attention(qm, km, vm, cu, cu, max(lens), causal=True)
        o.backward(dout)
        res.append([o.detach().cpu(), qm.grad.cpu(), km.grad.cpu(), vm.grad.cpu()])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D", [128, 88, 256])
def test_mfma_matches_generic(mt, D):
    """The MFMA kernels and the portable kernels agree (both vs the oracle too)."""
    import subprocess
    import sys
    _banner(f"MFMA vs generic path D={D} (subprocess with MTLATTN_NO_MFMA=1)")
    code = (
        "import torch, mtlattn, math, sys\n"
        "sys.path.insert(0, '.')\n"
        "from tests.helpers import cu_of, randn\n"
        "g = torch.Generator().manual_seed(4)\n"
        "lens=[100,257,31]\n"
        f"q=randn((388,8,{D}),torch.float16,g).cuda(); k=randn((388,4,{D}),torch.float16,g).cuda(); v=randn((388,4,{D}),torch.float16,g).cuda()\n"
        "cu=cu_of(lens,'cuda')\n"
        "o=mtlattn.varlen_attention(q,k,v,cu,cu,257,causal=True,window=50)\n"
        "torch.save(o.cpu(), sys.argv[1])\n")
    outs = []
    for env in ({}, {"MTLATTN_NO_MFMA": "1"}):
        path = f"/tmp/mtl_path_{len(env)}.pt"
        e = dict(os.environ, **env)
        r = subprocess.run([sys.executable, "-c", code, path], env=e, timeout=300,
                           cwd=os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
        assert r.returncode == 0
        outs.append(torch.load(path, weights_only=True).float())
    err = (outs[0] - outs[1]).abs().max().item()
    print(f"  mfma_vs_generic={err:.3e}", flush=True)
    assert err < 5e-3


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.float32, 128), (torch.float32, 66),
                                     (torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float16, 80)])
def test_nan_inputs_propagate(mt, dtype, D):
    """A NaN in q or k gives NaN outputs and LSEs in exactly the rows that
    see it, as a softmax over a NaN logit does in the oracle; every other
    row stays finite. (A clamp through fmaxf once turned NaN logits into
    weights of 0 in the fp32 kernels, so a NaN row looked fully masked:
    O = 0, LSE = -inf.) fp32 at 64 / 128 runs on the fp32 matrix cores, at 66
    on the portable kernels; 16-bit on the flash forward."""
    _banner(f"NaN inputs {dtype} D={D}")
    lens = [40, 50]
    Hq, Hkv = 4, 2
    q, k, v = _inputs(lens, lens, Hq, Hkv, D, dtype, seed=11)
    q[45, 3, 3] = float("nan")   # sequence 1, query head 3 (kv head 1), one row
    k[20, 0, 5] = float("nan")   # sequence 0, kv head 0: query heads 0 and 1, every row
    cu = cu_of(lens, "cuda")
    lse = torch.empty(sum(lens), Hq, dtype=torch.float32, device="cuda")
    out = mt._C.varlen_attention(q.cuda(), k.cuda(), v.cuda(), cu, cu, max(lens), 1 / math.sqrt(D), False, 0, lse)
    torch.cuda.synchronize()
    expect = torch.zeros(sum(lens), Hq, dtype=torch.bool)
    expect[0:40, 0:2] = True
    expect[45, 3] = True
    ref, ref_lse = oracle.varlen_forward(q, k, v, cu.cpu(), cu.cpu(), 1 / math.sqrt(D), False, 0, None)
    assert torch.equal(ref_lse.isnan(), expect), "the oracle's NaN pattern"
    o_nan = out.float().cpu().isnan()
    l_nan = lse.cpu().isnan()
    print(f"  out rows NaN: {int(o_nan.all(-1).sum())} (expect {int(expect.sum())}); "
          f"LSE NaN: {int(l_nan.sum())}", flush=True)
    assert torch.equal(o_nan.all(-1), expect) and torch.equal(o_nan.any(-1), expect)
    assert torch.equal(l_nan, expect)
    assert torch.isfinite(out.float().cpu()[~expect]).all() and torch.isfinite(lse.cpu()[~expect]).all()


@pytest.mark.gpu
def test_nan_inputs_propagate_split_kv(mt):
    """The split-KV decode path keeps NaN rows NaN: a NaN in a query row makes
    every split's LSE of that row NaN, and the combine's max over the splits
    must not drop them (an fmaxf max would, and the row would come out as an
    empty one: O = 0). A NaN in one key makes only the split that holds it
    NaN; the combine's weights carry that into the row."""
    _banner("NaN inputs, split-KV decode")
    q_lens, kv_lens = [1, 1, 1], [5000, 2100, 9001]
    Hq, Hkv = 8, 2
    q, k, v = _inputs(q_lens, kv_lens, Hq, Hkv, 128, torch.bfloat16, seed=5)
    q[1, 5, 7] = float("nan")        # sequence 1, query head 5 only
    k[5000 + 2100 + 300, 0, 9] = float("nan")   # sequence 2, kv head 0: query heads 0-3
    cq, ck = cu_of(q_lens, "cuda"), cu_of(kv_lens, "cuda")
    expect = torch.zeros(3, Hq, dtype=torch.bool)
    expect[1, 5] = True
    expect[2, 0:4] = True
    for ns in (1, 4, 16):
        o = mt._C.attn_splitkv(q.cuda(), k.cuda(), v.cuda(), cq, ck, 1, 1 / math.sqrt(128), True, ns).cpu()
        nan_rows = o.float().isnan().all(-1)
        print(f"  ns={ns} NaN rows {int(nan_rows.sum())} (expect {int(expect.sum())})", flush=True)
        assert torch.equal(nan_rows, expect) and torch.equal(o.float().isnan().any(-1), expect)
        assert torch.isfinite(o.float()[~expect]).all()
