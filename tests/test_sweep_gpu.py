"""GPU parity sweep: a fixed, seeded list of mixed cases crossing what the
targeted tests cover one feature at a time. It varies dtype (bf16, fp16,
fp32), head dim (every matrix-core size, the fp32 matrix-core sizes, and
sizes only the portable kernels take), GQA ratio, ragged and cross lengths
(kv shorter and longer than q, one-token sequences), causal, window, bias
(none, head-broadcast, per-head, 4-D per-sequence) and scale; a second set
has few queries against long KV, which the forward routes to split-KV
decode; a third has longer rows, GQA groups up to 16 and explicit scales
(negative and zero among them). Each case runs
forward + backward through mtlattn.varlen_attention and is checked against
the fp64 oracle. Every case prints its parameters first.

Criteria:
  * fp32: tests/helpers.py's, max|err| / RMS(ref) <= 1e-5 + 2 * floor32, with
    floor32 the fp32 oracle's own deviation from fp64 on the same case, plus
    4 u32 max|ref| (u32 = 2^-24): on heavy-tailed cases (a few keys
    dominating, so max|ref| is ~100x the RMS) one ulp of the largest element
    alone exceeds 1e-5 RMS, and the fp32 oracle's own deviation there is
    whatever its rounding happened to be;
  * fp16 / bf16: RMS(err) / RMS(ref) <= RMS_BOUND (tests/helpers.py), and
    max|err| <= 4 u max|ref| + 2e-2 RMS(ref) with u the unit roundoff
    (2^-8 bf16, 2^-11 fp16: 8 and 11 significand bits, as tests/helpers.py). The 16-bit kernels round P (and dS) to the
    input type before the second products (u), write the output in it (u),
    and take the LSE from the sum of the rounded P, which can be off by 2u
    when a few keys dominate a row; this sweep's random shapes include such
    rows (one query against hundreds of keys), where the largest element
    carries all three, so the bound is stated in u at the largest element
    rather than in the rounding floor of tests/helpers.py. For dQ and dK it
    is 8 u max|ref|: dS = P (dP - delta) with delta = rowsum(dO * O) formed
    from the stored (rounded) O, as in the reference, so dS carries delta's
    rounding (u |dO . O|) however small dP - delta is; where the two nearly
    cancel at a few dominant keys, that error rides on the largest dQ / dK
    elements in addition to P's, dS's and the output's roundings;
  * the backward takes P = exp(x - LSE) with the forward's fp32 LSE, so
    each bound also allows 4 u32 |LSE|max max|ref| (the LSE's own rounding,
    relative to P; the oracle takes its softmax directly);
  * a tensor whose exact value is below 1e-6 everywhere (every sequence one
    token long, or one key dominating each row: dQ ~ 0) is the difference
    of terms that cancel, and its error is the fp32 rounding of those terms,
    not a fraction of its own size. It is held to
    max|err| <= 1e-2 max|ref| + 64 u32 C, with C the size of the cancelling
    terms: for dQ, |scale| max|delta| max|K| (dS = P (dP - delta) times K);
    for dK, |scale| max|delta| max|Q| Lq (up to Lq query rows add to a
    key); for out and dV, max|V| and max|dO| Lq."""

import math
import random

import pytest
import torch

import oracle
from tests.helpers import RMS_BOUND, TOL_RMS, cu_of, err_stats, randn

UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}

pytestmark = pytest.mark.gpu

D16 = [64, 80, 88, 96, 128, 160, 256, 48]      # 48: portable kernels
D32 = [16, 32, 64, 100, 128, 36, 66, 160]     # 66, 160: portable kernels


def _cases(n=40, seed=1234):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = [torch.bfloat16, torch.float16, torch.float32][i % 3]
        d = rng.choice(D32 if dt == torch.float32 else D16)
        hkv = rng.choice([1, 2])
        g = rng.choice([1, 2, 4, 8])
        b = rng.randint(1, 4)
        cap = 400 if d >= 160 else 700
        ql = [rng.choice([1, rng.randint(1, cap)]) for _ in range(b)]
        cross = rng.random() < 0.4
        kl = [max(1, rng.randint(1, cap)) if cross else x for x in ql]
        causal = rng.random() < 0.6
        window = rng.choice([0, 0, rng.randint(1, 300)])
        bias = rng.choice([None, "bcast", "head", "4d"])
        scale = rng.choice([None, None, 0.2])
        out.append((i, dt, d, g * hkv, hkv, ql, kl, causal, window, bias, scale))
    return out


def _decode_cases(n=16, seed=4321):
    """Few queries against long KV (average >= 2048 keys, q_len <= 16): the
    forward routes to split-KV decode + combine (with window and bias too),
    the backward runs the prefill kernels on the combine's LSE."""
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = [torch.bfloat16, torch.float16][i % 2]
        d = rng.choice([64, 128])
        hkv = rng.choice([1, 2, 4])
        g = rng.choice([1, 4, 8])
        b = rng.randint(1, 5)
        ql = [rng.randint(1, 16) for _ in range(b)]
        kl = [rng.randint(2048, 9000) for _ in range(b)]
        causal = rng.random() < 0.7
        window = rng.choice([0, rng.randint(64, 5000)])
        bias = rng.choice([None, "bcast", "head", "4d"])
        scale = rng.choice([None, 0.2])
        out.append((100 + i, dt, d, g * hkv, hkv, ql, kl, causal, window, bias, scale))
    return out


def _wide_cases(n=16, seed=77):
    """Longer rows (up to 2048 keys), GQA groups up to 16 heads, and
    explicit scales including negative and zero (the explicitly scaled
    softmax mode)."""
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = [torch.bfloat16, torch.float16, torch.float32][i % 3]
        d = rng.choice(D32 if dt == torch.float32 else D16)
        hkv = rng.choice([1, 2])
        g = rng.choice([1, 4, 16])
        b = rng.randint(1, 3)
        cap = 600 if d >= 160 else 2048
        ql = [rng.choice([1, rng.randint(1, cap)]) for _ in range(b)]
        cross = rng.random() < 0.3
        kl = [max(1, rng.randint(1, cap)) if cross else x for x in ql]
        causal = rng.random() < 0.6
        window = rng.choice([0, 0, rng.randint(1, 600)])
        bias = rng.choice([None, "bcast", "head", "4d"])
        scale = rng.choice([None, 0.2, -0.1, 0.0, 0.05])
        out.append((200 + i, dt, d, g * hkv, hkv, ql, kl, causal, window, bias, scale))
    return out


def _bias(kind, ql, kl, hq, gen):
    """(bias given to the kernels, the 3-D bias the oracle uses)."""
    if kind is None:
        return None, None
    if kind == "4d":
        nq = max(ql)
        b4 = torch.randn((len(ql), 1, nq, max(kl)), generator=gen)
        b4[..., ::5] -= 20.0
        rows = [b4[s][:, :L, :].transpose(0, 1) for s, L in enumerate(ql)]
        return b4, torch.cat(rows).contiguous()
    b = torch.randn((sum(ql), 1 if kind == "bcast" else hq, max(kl)), generator=gen)
    b[:, :, ::7] -= 30.0
    return b, b


@pytest.mark.parametrize("case", _cases() + _decode_cases() + _wide_cases(), ids=lambda c: f"case{c[0]}")
def test_sweep(case):
    import mtlattn
    i, dt, d, hq, hkv, ql, kl, causal, window, bias_kind, scale = case
    print(f"\n[case] sweep {i}: {dt} D={d} Hq={hq} Hkv={hkv} q={ql} kv={kl} causal={causal} "
          f"window={window} bias={bias_kind} scale={scale}", flush=True)
    gen = torch.Generator().manual_seed(100 + i)
    q = randn((sum(ql), hq, d), dt, gen)
    k = randn((sum(kl), hkv, d), dt, gen)
    v = randn((sum(kl), hkv, d), dt, gen)
    dout = randn((sum(ql), hq, d), dt, gen)
    bias_in, bias_ref = _bias(bias_kind, ql, kl, hq, gen)
    cq, ck = cu_of(ql), cu_of(kl)
    qm, km, vm = (t.cuda().requires_grad_() for t in (q, k, v))
    out = mtlattn.varlen_attention(qm, km, vm, cq.cuda(), ck.cuda(), max(ql), scale=scale, causal=causal,
                                   window=window, attn_bias=None if bias_in is None else bias_in.cuda())
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    args = (q, k, v, dout, cq, ck, sc, causal, window, bias_ref)
    r64 = oracle.varlen_forward_backward(*args, dtype=torch.float64)
    r32 = oracle.varlen_forward_backward(*args, dtype=torch.float32) if dt == torch.float32 else None
    lse_ref = r64[1][torch.isfinite(r64[1])]
    lse_term = 4 * 2.0 ** -24 * (lse_ref.abs().max().item() if lse_ref.numel() else 0.0)
    # size of the terms that cancel in a tensor whose exact value is ~0
    delta = (dout.double() * r64[0].double()).sum(-1).abs().max().item() if dout.numel() else 0.0
    amax = lambda t: t.double().abs().max().item() if t.numel() else 0.0
    lq = max(ql)
    cancel = {"out": amax(v), "dV": amax(dout) * lq, "dQ": abs(sc) * delta * amax(k),
              "dK": abs(sc) * delta * amax(q) * lq}
    for nm, a, j in (("out", out, 0), ("dQ", qm.grad, 2), ("dK", km.grad, 3), ("dV", vm.grad, 4)):
        assert torch.isfinite(a.float()).all(), f"case {i}: non-finite {nm}"
        ref = r64[j].float()
        got = a.detach().float().cpu()
        max_abs = (got - ref).abs().max().item() if ref.numel() else 0.0
        if ref.numel() == 0:
            continue
        if ref.abs().max().item() <= 1e-6:
            bound = 1e-2 * ref.abs().max().item() + 64 * 2.0 ** -24 * cancel[nm]
            print(f"  {nm}: near zero, max|ref|={ref.abs().max().item():.3e} max_abs={max_abs:.3e} "
                  f"bound={bound:.3e}", flush=True)
            assert max_abs <= bound, f"case {i}: {nm} max_abs {max_abs:.3e} > {bound:.3e}"
            continue
        if dt == torch.float32:
            f32 = err_stats(r32[j], r64[j], dt)["rel"]
            st = err_stats(a, ref, dt, f32)
            bound = (TOL_RMS[dt] + 2 * f32) * st["rms_ref"] + (4 * 2.0 ** -24 + lse_term) * ref.abs().max().item()
            print(f"  {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor32={f32:.3e} "
                  f"max_abs={max_abs:.3e} bound={bound:.3e}", flush=True)
            assert max_abs <= bound, f"case {i}: {nm} max_abs {max_abs:.3e} > {bound:.3e}"
        else:
            st = err_stats(a, ref, dt)
            rms = st["rms_ref"]
            ku = 8 if nm in ("dQ", "dK") else 4
            bound = (ku * UNIT_ROUNDOFF[dt] + lse_term) * ref.abs().max().item() + TOL_RMS[dt] * rms
            print(f"  {nm}: rel={st['rel']:.3e} rms_rel={st['rms_rel']:.3e} floor={st['floor']:.3e} "
                  f"max_abs={max_abs:.3e} bound={bound:.3e}", flush=True)
            assert st["rms_rel"] <= RMS_BOUND[dt], f"case {i}: {nm} rms_rel {st['rms_rel']:.3e}"
            assert max_abs <= bound, f"case {i}: {nm} max_abs {max_abs:.3e} > {bound:.3e}"
