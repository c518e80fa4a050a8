"""Pins the CPU oracle (oracle/reference.py) before it is trusted as the
checker: against the committed golden fixtures (element-by-element fp64
brute force), closed forms, autograd gradcheck, mutual agreement of its three
forms, and planted mistakes that the checks must catch."""

import math
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.helpers import cu_of

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_small.npz")


def _golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def _case(z, name):
    t = lambda k: torch.from_numpy(z[f"{name}/{k}"])
    Hq, Hkv, D, causal, window = (int(x) for x in z[f"{name}/meta"])
    bias = t("bias") if f"{name}/bias" in z.files else None
    return dict(q=t("q"), k=t("k"), v=t("v"), dout=t("dout"), cu_q=t("cu_q"), cu_kv=t("cu_kv"),
                causal=bool(causal), window=window, bias=bias, D=D,
                out=t("out"), lse=t("lse"), dq=t("dq"), dk=t("dk"), dv=t("dv"))


@pytest.mark.parametrize("name", _golden_cases()[1])
def test_oracle_matches_golden(name):
    z, _ = _golden_cases()
    c = _case(z, name)
    scale = 1.0 / math.sqrt(c["D"])
    out, lse, dq, dk, dv = oracle.varlen_forward_backward(
        c["q"], c["k"], c["v"], c["dout"], c["cu_q"], c["cu_kv"], scale, c["causal"], c["window"],
        c["bias"], dtype=torch.float64)
    torch.testing.assert_close(out, c["out"], rtol=1e-10, atol=1e-12)
    fin = torch.isfinite(c["lse"])
    assert torch.equal(torch.isfinite(lse), fin)
    torch.testing.assert_close(lse[fin], c["lse"][fin], rtol=1e-10, atol=1e-12)
    for a, b in ((dq, c["dq"]), (dk, c["dk"]), (dv, c["dv"])):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-11)
    # the blocked (memory-bounded) form agrees too, with a tiny query block
    bo, bl, bq, bk, bv = oracle.varlen_forward_backward_blocked(
        c["q"], c["k"], c["v"], c["dout"], c["cu_q"], c["cu_kv"], scale, c["causal"], c["window"],
        c["bias"], dtype=torch.float64, q_block=2)
    torch.testing.assert_close(bo, c["out"], rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(bl[fin], c["lse"][fin], rtol=1e-10, atol=1e-12)
    for a, b in ((bq, c["dq"]), (bk, c["dk"]), (bv, c["dv"])):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-11)


def _rand(lens_q, lens_k, Hq, Hkv, D, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sum(lens_q), Hq, D, generator=g, dtype=dtype)
    k = torch.randn(sum(lens_k), Hkv, D, generator=g, dtype=dtype)
    v = torch.randn(sum(lens_k), Hkv, D, generator=g, dtype=dtype)
    return q, k, v


def test_single_allowed_key_closed_form():
    # causal, q_len == kv_len: row 0 sees only key 0; window 1: row i sees only key i + coff
    lens_q, lens_k = [5, 3], [7, 3]
    q, k, v = _rand(lens_q, lens_k, 2, 2, 8)
    out, lse = oracle.varlen_forward(q, k, v, cu_of(lens_q), cu_of(lens_k), 0.3, causal=True, window=1,
                                     dtype=torch.float64)
    qo = ko = 0
    for ql, kl in zip(lens_q, lens_k):
        coff = kl - ql
        for i in range(ql):
            torch.testing.assert_close(out[qo + i], v[ko + i + coff], rtol=0, atol=1e-12)
            s = 0.3 * (q[qo + i] * k[ko + i + coff]).sum(-1)
            torch.testing.assert_close(lse[qo + i], s, rtol=1e-12, atol=1e-12)
        qo += ql
        ko += kl


def test_zero_logits_mean_closed_form():
    # Q = 0, no bias: O is the mean of V over the allowed keys, LSE = log(#allowed)
    lens = [6, 9]
    q, k, v = _rand(lens, lens, 4, 2, 8)
    q.zero_()
    for causal, window in ((False, 0), (True, 0), (True, 3), (False, 4)):
        out, lse = oracle.varlen_forward(q, k, v, cu_of(lens), cu_of(lens), 1.0, causal, window,
                                         dtype=torch.float64)
        off = 0
        for L in lens:
            m = oracle.allowed_mask(L, L, causal, window)
            for i in range(L):
                keys = m[i].nonzero().flatten() + off
                exp = v[keys].repeat_interleave(2, 1).mean(0)
                torch.testing.assert_close(out[off + i], exp, rtol=0, atol=1e-12)
                assert abs(lse[off + i, 0].item() - math.log(len(keys))) < 1e-12
            off += L


def test_row_constant_bias_shifts_lse_only():
    lens = [5, 4]
    q, k, v = _rand(lens, lens, 2, 2, 8)
    c = torch.randn(9, 2, 1, dtype=torch.float64)
    bias = c.expand(9, 2, 5).contiguous()
    o0, l0 = oracle.varlen_forward(q, k, v, cu_of(lens), cu_of(lens), 0.5, True, 0, dtype=torch.float64)
    o1, l1 = oracle.varlen_forward(q, k, v, cu_of(lens), cu_of(lens), 0.5, True, 0, bias, dtype=torch.float64)
    torch.testing.assert_close(o0, o1, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(l1 - l0, c[:, :, 0], rtol=1e-12, atol=1e-12)


def test_convex_combination_bound():
    # |O| <= max |V| over allowed keys (tests/test_mps_sdpa_bug.py:13-15)
    lens = [40, 17]
    q, k, v = _rand(lens, lens, 3, 1, 16, seed=4)
    out, _ = oracle.varlen_forward(q * 3, k, v, cu_of(lens), cu_of(lens), None, True, 0, dtype=torch.float64)
    assert out.abs().max() <= v.abs().max() + 1e-12


def test_empty_rows_zero_and_neg_inf():
    q, k, v = _rand([6], [2], 2, 2, 4)
    out, lse = oracle.varlen_forward(q, k, v, cu_of([6]), cu_of([2]), None, True, 0, dtype=torch.float64)
    # coff = -4: rows 0..3 see no key
    assert torch.equal(out[:4], torch.zeros_like(out[:4]))
    assert torch.isinf(lse[:4]).all() and (lse[:4] < 0).all()
    assert torch.isfinite(lse[4:]).all()


def test_nan_logit_rows_stay_nan():
    """Only rows with no allowed key are special-cased to O = 0 and
    LSE = -inf; a NaN logit gives NaN in its row, as a plain softmax does,
    in the graph form and the blocked form alike (a planted check: treating
    every non-finite LSE as empty turns these rows into zeros)."""
    q, k, v = _rand([5, 6], [5, 6], 2, 1, 4)
    q[7, 1, 0] = float("nan")          # sequence 1, head 1, one query row
    k[2, 0, 3] = float("nan")          # sequence 0: every row of both heads
    dout = torch.ones_like(q)
    cq = cu_of([5, 6])
    out, lse = oracle.varlen_forward(q, k, v, cq, cq, None, False, 0, dtype=torch.float64)
    ob, lb = oracle.varlen_forward_backward_blocked(q, k, v, dout, cq, cq, None, False, 0, backward=False,
                                                    dtype=torch.float64)[:2]
    expect = torch.zeros(11, 2, dtype=torch.bool)
    expect[0:5] = True
    expect[7, 1] = True
    for o, l in ((out, lse), (ob, lb)):
        assert torch.equal(l.isnan(), expect)
        assert torch.equal(o.isnan().all(-1), expect) and torch.equal(o.isnan().any(-1), expect)


def test_gqa_equals_expanded_mha():
    lens = [7, 5]
    q, k, v = _rand(lens, lens, 6, 2, 8, seed=2)
    g = torch.Generator().manual_seed(3)
    do = torch.randn(12, 6, 8, generator=g, dtype=torch.float64)
    a = oracle.varlen_forward_backward(q, k, v, do, cu_of(lens), cu_of(lens), None, True, 0, dtype=torch.float64)
    ke, ve = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    b = oracle.varlen_forward_backward(q, ke, ve, do, cu_of(lens), cu_of(lens), None, True, 0, dtype=torch.float64)
    torch.testing.assert_close(a[0], b[0])
    torch.testing.assert_close(a[2], b[2])
    torch.testing.assert_close(a[3], b[3].view(12, 2, 3, 8).sum(2))
    torch.testing.assert_close(a[4], b[4].view(12, 2, 3, 8).sum(2))


def test_gradcheck_fp64():
    lens_q, lens_k = [3, 2], [4, 2]
    q, k, v = _rand(lens_q, lens_k, 2, 1, 4, seed=8)
    cq, ck = cu_of(lens_q), cu_of(lens_k)

    def f(q_, k_, v_):
        return R._forward_graph(q_, k_, v_, R.seq_lens(cq), R.seq_lens(ck), 0.7, True, 3, None, 2)[0]

    assert torch.autograd.gradcheck(f, (q.requires_grad_(), k.requires_grad_(), v.requires_grad_()))


def test_delta_identity():
    # delta_i = sum_j P_ij dP_ij = rowsum(dO * O)
    lens = [9]
    q, k, v = _rand(lens, lens, 1, 1, 8, seed=11)
    g = torch.Generator().manual_seed(12)
    do = torch.randn(9, 1, 8, generator=g, dtype=torch.float64)
    out, lse = oracle.varlen_forward(q, k, v, cu_of(lens), cu_of(lens), 0.4, True, 0, dtype=torch.float64)
    s = 0.4 * q[:, 0] @ k[:, 0].T
    s = s.masked_fill(~oracle.allowed_mask(9, 9, True, 0), float("-inf"))
    p = torch.exp(s - lse[:, 0:1])
    dp = do[:, 0] @ v[:, 0].T
    torch.testing.assert_close((p * dp).sum(-1), (do[:, 0] * out[:, 0]).sum(-1))


def test_attended_pairs():
    # square self-attention matches the reference bench's closed forms (mtlattn/bench.py:25-32)
    for M in (1, 7, 100):
        assert oracle.attended_pairs([M], [M], causal=False) == M * M
        assert oracle.attended_pairs([M], [M], causal=True) == M * (M + 1) // 2
        for W in (1, 5, 300):
            assert oracle.attended_pairs([M], [M], causal=True, window=W) == sum(min(i + 1, W) for i in range(M))
    # general: equals the mask population
    for ql, kl, c, w in ((5, 9, True, 0), (9, 5, True, 3), (6, 6, False, 2), (4, 10, False, 0)):
        assert oracle.attended_pairs([ql], [kl], c, w) == int(oracle.allowed_mask(ql, kl, c, w).sum())
    # C3: 8 x 4096 causal
    assert oracle.attended_pairs([4096] * 8, [4096] * 8, True) == 67_125_248


# ---- planted mistakes: each must be caught by a check above ----------------
def _golden_forward_ok(forward_fn):
    z, names = _golden_cases()
    for name in names:
        c = _case(z, name)
        out, _ = forward_fn(c["q"], c["k"], c["v"], c["cu_q"], c["cu_kv"], 1.0 / math.sqrt(c["D"]),
                            c["causal"], c["window"], c["bias"], dtype=torch.float64)
        if not torch.allclose(out, c["out"], rtol=1e-8, atol=1e-10):
            return False
    return True


def test_planted_causal_offset_is_caught(monkeypatch):
    def no_offset(ql, kl, causal, window, q_rows=None, k_cols=None):   # drops coff = kl - ql
        i = torch.arange(ql)[:, None]
        j = torch.arange(kl)[None, :]
        m = torch.ones(ql, kl, dtype=torch.bool)
        if causal:
            m &= j <= i
        if window > 0:
            m &= j > i - window
        return m
    assert _golden_forward_ok(oracle.varlen_forward)
    monkeypatch.setattr(R, "allowed_mask", no_offset)
    assert not _golden_forward_ok(oracle.varlen_forward)


def test_planted_gqa_mapping_is_caught(monkeypatch):
    orig = torch.Tensor.repeat_interleave

    def tiled(self, repeats, dim=None, **kw):      # h % Hkv instead of h // g
        if dim == 1 and isinstance(repeats, int):
            return self.repeat(1, repeats, 1)
        return orig(self, repeats, dim, **kw)
    monkeypatch.setattr(torch.Tensor, "repeat_interleave", tiled)
    assert not _golden_forward_ok(oracle.varlen_forward)


def test_planted_transposed_operand_is_caught(monkeypatch):
    good = R._forward_graph

    def swapped(qf, kf, vf, *a):                    # k and v swapped
        return good(qf, vf, kf, *a)
    monkeypatch.setattr(R, "_forward_graph", swapped)
    assert not _golden_forward_ok(oracle.varlen_forward)
