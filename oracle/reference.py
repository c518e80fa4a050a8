"""fp32 / fp64 CPU restatement of mtlattn's varlen attention (forward, LSE, backward).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product path.

What it restates (reference = lastowl/mtlattn 0.4.0):

* ``varlen_forward``  -- ``ref_varlen`` (tests/test_correctness.py:12-40): a
  per-sequence loop over cu_seqlens, inputs upcast from their storage dtype,
  logits ``scale * q k^T (+ bias[qo:qo+ql, :, :kl])``, the end-aligned causal
  mask ``j <= i + (kl - ql)`` and the window bound ``j > i + (kl - ql) - W``
  (tests/test_correctness.py:26-36), softmax, ``@ v``. GQA follows
  ``repeat_interleave(g, 1)`` of K/V (tests/test_correctness.py:109-110).
  Also returns the natural-log LSE the kernels emit
  (src/attn_mpp.metal:313-315).
* ``varlen_forward_backward`` -- the differentiable reference
  (tests/test_correctness.py:169-211, 248-288): autograd through the same
  graph, GQA gradients folded with ``.view(Mk, Hkv, g, D).sum(2)``
  (tests/test_correctness.py:204-205), the bias held constant.
* ``varlen_forward_backward_blocked`` -- the same mathematics written out by
  hand (dS = P * (dP - delta), src/attention.metal:707-717), chunked over query
  blocks and restricted to each block's allowed key band so large configs fit
  in host memory. Pinned against the autograd form by tests.
* ``attended_pairs`` -- the FLOP convention of mtlattn/bench.py:25-32 (count
  only attended pairs), generalised to ragged batches, windows and cross shapes.
* ``brute_force`` -- pure-Python fp64 loops over single elements for tiny
  inputs; an independent statement used to pin the torch forms above.

Deliberate difference from the torch reference: a query row with no allowed
key yields O = 0 and LSE = -inf (the kernels' convention,
src/attention.metal:232,250; src/attn_mpp.metal:307,315) instead of the NaN a
softmax over an all -inf row gives.
"""

import math

import torch

__all__ = [
    "allowed_mask",
    "attended_pairs",
    "brute_force",
    "seq_lens",
    "varlen_forward",
    "varlen_forward_backward",
    "varlen_forward_backward_blocked",
]


def seq_lens(cu):
    """cu_seqlens (tensor or list, [B+1]) -> python list of B lengths."""
    c = cu.tolist() if torch.is_tensor(cu) else list(cu)
    return [int(c[i + 1]) - int(c[i]) for i in range(len(c) - 1)]


def allowed_mask(ql, kl, causal, window, q_rows=None, k_cols=None):
    """Bool [ql, kl] (or the sub-block given by q_rows/k_cols ranges) of allowed
    (query i, key j) pairs: causal => j <= i + coff; window W > 0 => j > i + coff - W,
    coff = kl - ql (tests/test_correctness.py:26-36). Non-causal with a window is a
    lower bound only (tests/test_correctness.py:386)."""
    i = (torch.arange(ql) if q_rows is None else torch.arange(*q_rows))[:, None]
    j = (torch.arange(kl) if k_cols is None else torch.arange(*k_cols))[None, :]
    coff = kl - ql
    m = torch.ones(i.shape[0], j.shape[1], dtype=torch.bool)
    if causal:
        m &= j <= i + coff
    if window > 0:
        m &= j > i + coff - window
    return m


def attended_pairs(q_lens, kv_lens, causal=False, window=0):
    """Exact number of allowed (query, key) pairs per head, summed over sequences.
    Generalises mtlattn/bench.py:25-32 (square self-attention) to ragged/cross
    shapes; closed form per row, no L x L materialisation."""
    total = 0
    for ql, kl in zip(q_lens, kv_lens):
        coff = kl - ql
        for i in range(ql):
            hi = min(kl - 1, i + coff) if causal else kl - 1
            lo = max(0, i + coff - window + 1) if window > 0 else 0
            if hi >= lo:
                total += hi - lo + 1
    return total


def _bias_block(bias, qo, ql, kl, Hq):
    """bias[qo:qo+ql, :, :kl] as [H or 1, ql, kl] fp (tests/test_correctness.py:24-25)."""
    b = bias[qo:qo + ql, :, :kl].permute(1, 0, 2)
    if b.shape[0] not in (1, Hq):
        raise ValueError("bias dim1 must be 1 or Hq")
    return b


def _masked_softmax(a, mask):
    """Softmax over the last dim restricted to `mask`; rows with no allowed key
    give P = 0 and LSE = -inf (differentiable). Only those rows are special:
    a row with a NaN logit keeps the NaN a plain softmax gives it."""
    a = a.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(a, dim=-1)
    valid = lse != float("-inf")
    a_safe = torch.where(valid[..., None], a, torch.zeros_like(a))
    p = torch.softmax(a_safe, dim=-1) * valid[..., None].to(a.dtype)
    return p, lse


def _forward_graph(qf, kf, vf, q_lens, kv_lens, scale, causal, window, bias, g):
    """Shared forward used by the autograd oracle. qf: [Mq, Hq, D], kf/vf: [Mk, Hkv, D]
    in the compute dtype. Returns (out [Mq,Hq,D], lse [Mq,Hq])."""
    Hq = qf.shape[1]
    ke = kf.repeat_interleave(g, 1)   # tests/test_correctness.py:109-110
    ve = vf.repeat_interleave(g, 1)
    outs, lses = [], []
    qo = ko = 0
    for ql, kl in zip(q_lens, kv_lens):
        qi = qf[qo:qo + ql].permute(1, 0, 2)     # [H, ql, D]
        ki = ke[ko:ko + kl].permute(1, 0, 2)
        vi = ve[ko:ko + kl].permute(1, 0, 2)
        a = (qi @ ki.transpose(-1, -2)) * scale
        if bias is not None:
            a = a + _bias_block(bias, qo, ql, kl, Hq).to(a.dtype)
        p, lse = _masked_softmax(a, allowed_mask(ql, kl, causal, window))
        outs.append((p @ vi).permute(1, 0, 2))
        lses.append(lse.permute(1, 0))
        qo += ql
        ko += kl
    D = qf.shape[2]
    if not outs:
        return qf.new_zeros(0, Hq, D), qf.new_zeros(0, Hq)
    return torch.cat(outs, 0), torch.cat(lses, 0)


def varlen_forward(q, k, v, cu_q, cu_kv, scale=None, causal=False, window=0, bias=None,
                   dtype=torch.float32):
    """Oracle forward: (out, lse) in `dtype` (fp32 default, fp64 for pinning).
    q: [Mq, Hq, D], k/v: [Mk, Hkv, D] (any float dtype, any device -> CPU),
    cu_*: [B+1] int, bias: optional [Mq, Hq or 1, >= max_kv] additive."""
    q_lens, kv_lens = seq_lens(cu_q), seq_lens(cu_kv)
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    g = q.shape[1] // k.shape[1]
    qf = q.detach().cpu().to(dtype)
    kf = k.detach().cpu().to(dtype)
    vf = v.detach().cpu().to(dtype)
    bf = None if bias is None else bias.detach().cpu().to(dtype)
    with torch.no_grad():
        return _forward_graph(qf, kf, vf, q_lens, kv_lens, scale, causal, window, bf, g)


def varlen_forward_backward(q, k, v, dout, cu_q, cu_kv, scale=None, causal=False, window=0,
                            bias=None, dtype=torch.float32):
    """Oracle forward + autograd backward (tests/test_correctness.py:169-211):
    returns (out, lse, dq, dk, dv), GQA grads folded over the g query heads of
    each kv head (tests/test_correctness.py:204-205)."""
    q_lens, kv_lens = seq_lens(cu_q), seq_lens(cu_kv)
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    Hkv = k.shape[1]
    g = q.shape[1] // Hkv
    qf = q.detach().cpu().to(dtype).requires_grad_()
    kf = k.detach().cpu().to(dtype).requires_grad_()
    vf = v.detach().cpu().to(dtype).requires_grad_()
    bf = None if bias is None else bias.detach().cpu().to(dtype)
    with torch.enable_grad():
        out, lse = _forward_graph(qf, kf, vf, q_lens, kv_lens, scale, causal, window, bf, g)
        out.backward(dout.detach().cpu().to(dtype))
    return out.detach(), lse.detach(), qf.grad, kf.grad, vf.grad


def _key_band(q_first, q_last, ql, kl, causal, window):
    """Smallest key range [lo, hi) containing every allowed key of query rows
    q_first..q_last (seq-local)."""
    coff = kl - ql
    hi = min(kl, q_last + coff + 1) if causal else kl
    lo = max(0, q_first + coff - window + 1) if window > 0 else 0
    return lo, max(lo, hi)


def varlen_forward_backward_blocked(q, k, v, dout, cu_q, cu_kv, scale=None, causal=False,
                                    window=0, bias=None, dtype=torch.float32, q_block=512,
                                    heads=None, seqs=None, backward=True):
    """Memory-bounded oracle: explicit forward and backward formulas
    (P = exp(logit - lse); delta = rowsum(dO * O); dS = P * (dP - delta);
    dQ = scale dS K; dK = scale dS^T Q; dV = P^T dO; src/attention.metal:707-717),
    per sequence, per query block of `q_block` rows, over that block's key band.

    `heads` (iterable of kv-head indices) and `seqs` (iterable of sequence
    indices) restrict the work to a sample; rows/keys outside the sample are
    left at zero in the returned tensors. Returns (out, lse, dq, dk, dv);
    gradients are None when backward=False."""
    q_lens, kv_lens = seq_lens(cu_q), seq_lens(cu_kv)
    Mq, Hq, D = q.shape
    Mk, Hkv = k.shape[0], k.shape[1]
    g = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    heads = list(range(Hkv)) if heads is None else list(heads)
    seqs = list(range(len(q_lens))) if seqs is None else list(seqs)
    qc = q.detach().cpu()
    kc = k.detach().cpu()
    vc = v.detach().cpu()
    dc = None if dout is None else dout.detach().cpu()
    out = torch.zeros(Mq, Hq, D, dtype=dtype)
    lse = torch.full((Mq, Hq), float("-inf"), dtype=dtype)
    dq = torch.zeros(Mq, Hq, D, dtype=dtype) if backward else None
    dk = torch.zeros(Mk, Hkv, D, dtype=dtype) if backward else None
    dv = torch.zeros(Mk, Hkv, D, dtype=dtype) if backward else None
    qoffs = [0]
    koffs = [0]
    for ql, kl in zip(q_lens, kv_lens):
        qoffs.append(qoffs[-1] + ql)
        koffs.append(koffs[-1] + kl)
    hsel = torch.tensor([hk * g + j for hk in heads for j in range(g)], dtype=torch.long)
    hk_sel = torch.tensor(heads, dtype=torch.long)
    for s in seqs:
        ql, kl = q_lens[s], kv_lens[s]
        qo, ko = qoffs[s], koffs[s]
        if ql == 0:
            continue
        kseq = kc[ko:ko + kl].index_select(1, hk_sel).to(dtype).permute(1, 0, 2)  # [nh, kl, D]
        vseq = vc[ko:ko + kl].index_select(1, hk_sel).to(dtype).permute(1, 0, 2)
        dks = torch.zeros_like(kseq) if backward else None
        dvs = torch.zeros_like(vseq) if backward else None
        for b0 in range(0, ql, q_block):
            b1 = min(ql, b0 + q_block)
            lo, hi = _key_band(b0, b1 - 1, ql, kl, causal, window)
            qb = qc[qo + b0:qo + b1].index_select(1, hsel).to(dtype).permute(1, 0, 2)
            qb = qb.reshape(len(heads), g, b1 - b0, D)                         # [nh, g, nq, D]
            if hi <= lo:
                continue
            kb, vb = kseq[:, lo:hi], vseq[:, lo:hi]                             # [nh, nk, D]
            a = torch.matmul(qb, kb.transpose(-1, -2).unsqueeze(1)) * scale     # [nh, g, nq, nk]
            if bias is not None:
                bb = bias[qo + b0:qo + b1, :, lo:hi].detach().cpu().to(dtype).permute(1, 0, 2)
                if bb.shape[0] == 1:
                    a = a + bb.unsqueeze(0)
                else:
                    a = a + bb.index_select(0, hsel).reshape(len(heads), g, b1 - b0, hi - lo)
            m = allowed_mask(ql, kl, causal, window, q_rows=(b0, b1), k_cols=(lo, hi))
            a = a.masked_fill(~m, float("-inf"))
            l_b = torch.logsumexp(a, dim=-1)                                    # [nh, g, nq]
            valid = l_b != float("-inf")      # rows with no allowed key (NaN rows stay NaN)
            p = torch.exp(a - torch.where(valid, l_b, torch.zeros_like(l_b))[..., None])
            p = p * valid[..., None].to(dtype)
            o_b = torch.matmul(p, vb.unsqueeze(1))                              # [nh, g, nq, D]
            rows = slice(qo + b0, qo + b1)
            out[rows, hsel] = o_b.reshape(len(heads) * g, b1 - b0, D).permute(1, 0, 2)
            lse[rows, hsel] = l_b.reshape(len(heads) * g, b1 - b0).permute(1, 0)
            if not backward:
                continue
            do_b = dc[qo + b0:qo + b1].index_select(1, hsel).to(dtype).permute(1, 0, 2)
            do_b = do_b.reshape(len(heads), g, b1 - b0, D)
            delta = (do_b * o_b).sum(-1)                                        # [nh, g, nq]
            dp = torch.matmul(do_b, vb.transpose(-1, -2).unsqueeze(1))         # [nh, g, nq, nk]
            ds = p * (dp - delta[..., None])
            dq_b = torch.matmul(ds, kb.unsqueeze(1)) * scale                    # [nh, g, nq, D]
            dq[rows, hsel] = dq_b.reshape(len(heads) * g, b1 - b0, D).permute(1, 0, 2)
            dks[:, lo:hi] += torch.matmul(ds.transpose(-1, -2), qb).sum(1) * scale
            dvs[:, lo:hi] += torch.matmul(p.transpose(-1, -2), do_b).sum(1)
        if backward:
            dk[ko:ko + kl, hk_sel] = dks.permute(1, 0, 2)
            dv[ko:ko + kl, hk_sel] = dvs.permute(1, 0, 2)
    return out, lse, dq, dk, dv


def brute_force(q, k, v, dout, cu_q, cu_kv, scale, causal=False, window=0, bias=None):
    """Element-by-element fp64 statement in plain Python (tiny inputs only).
    Written independently of the torch forms: explicit loops for the logits,
    a two-pass max/sum softmax, and the textbook gradient formulas. Returns
    python nested lists (out, lse, dq, dk, dv) with dq/dk/dv None if dout is None."""
    q_lens, kv_lens = seq_lens(cu_q), seq_lens(cu_kv)
    Q = q.double().tolist()
    K = k.double().tolist()
    V = v.double().tolist()
    dO = None if dout is None else dout.double().tolist()
    B = None if bias is None else bias.double().tolist()
    Mq, Hq, D = len(Q), len(Q[0]) if Q else 0, q.shape[-1]
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = [[[0.0] * D for _ in range(Hq)] for _ in range(Mq)]
    lse = [[float("-inf")] * Hq for _ in range(Mq)]
    dq = [[[0.0] * D for _ in range(Hq)] for _ in range(Mq)]
    dk = [[[0.0] * D for _ in range(Hkv)] for _ in range(k.shape[0])]
    dv = [[[0.0] * D for _ in range(Hkv)] for _ in range(k.shape[0])]
    qo = ko = 0
    for ql, kl in zip(q_lens, kv_lens):
        coff = kl - ql
        for h in range(Hq):
            hk = h // g
            hb = 0 if (B is not None and len(B[0]) == 1) else h
            for i in range(ql):
                keys = []
                for j in range(kl):
                    if causal and not (j <= i + coff):
                        continue
                    if window > 0 and not (j > i + coff - window):
                        continue
                    keys.append(j)
                if not keys:
                    continue
                logit = {}
                for j in keys:
                    s = 0.0
                    for d in range(D):
                        s += Q[qo + i][h][d] * K[ko + j][hk][d]
                    s *= scale
                    if B is not None:
                        s += B[qo + i][hb][j]
                    logit[j] = s
                mx = max(logit.values())
                tot = sum(math.exp(logit[j] - mx) for j in keys)
                lse[qo + i][h] = mx + math.log(tot)
                P = {j: math.exp(logit[j] - mx) / tot for j in keys}
                for d in range(D):
                    out[qo + i][h][d] = sum(P[j] * V[ko + j][hk][d] for j in keys)
                if dO is None:
                    continue
                dP = {j: sum(dO[qo + i][h][d] * V[ko + j][hk][d] for d in range(D)) for j in keys}
                delta = sum(P[j] * dP[j] for j in keys)
                for j in keys:
                    ds = P[j] * (dP[j] - delta)
                    for d in range(D):
                        dq[qo + i][h][d] += scale * ds * K[ko + j][hk][d]
                        dk[ko + j][hk][d] += scale * ds * Q[qo + i][h][d]
                        dv[ko + j][hk][d] += P[j] * dO[qo + i][h][d]
        qo += ql
        ko += kl
    if dO is None:
        return out, lse, None, None, None
    return out, lse, dq, dk, dv
