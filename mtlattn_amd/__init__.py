"""mtlattn for AMD Instinct MI355X (gfx950): fused variable-length attention.

Drop-in for the reference package's public API (mtlattn/__init__.py:15-22 of
lastowl/mtlattn 0.4.0): ``varlen_attention``, the flash_attn-style packed
wrappers, a dense ``sdpa`` adapter and ``replace_sdpa``/``restore_sdpa``.
Tensors live on PyTorch-ROCm's ``cuda`` device; the work runs in hand-written
gfx950 HIP kernels behind the C ABI in ``include/mtlattn_capi.h`` (the
``_C`` torch binding next to this file wraps it).

Conventions shared with the reference:
  * q/k/v are packed ``[total_tokens, heads, D]`` (row-strided views allowed,
    head stride must be D), ``cu_seqlens`` are int32 ``[B+1]`` offsets;
  * causal is end-aligned: query i sees key j iff j <= i + (kv_len - q_len);
  * ``window=W > 0`` additionally requires j > i + (kv_len - q_len) - W;
  * GQA: query head h reads kv head h // (Hq // Hkv);
  * ``attn_bias`` is an additive fp32 ``[total_q, Hq or 1, max_kv]`` mask,
    indexed by global query row, head and sequence-local key, applied in the
    forward and backward but not differentiated.
"""

import math
import weakref

import torch

try:
    from . import _C
except ImportError as exc:  # the product path has no fallback: fail loudly
    raise ImportError(
        "mtlattn_amd: the native extension (_C + libmtlattn_hip.so) is not built; "
        "run `python -m mtlattn_amd.build` (or __graft_entry__.build())") from exc

__version__ = "0.4.0+mi355x"

__all__ = [
    "varlen_attention",
    "flash_attn_varlen_qkvpacked_func",
    "flash_attn_varlen_kvpacked_func",
    "sdpa",
    "replace_sdpa",
    "restore_sdpa",
]


class _VarlenAttnFn(torch.autograd.Function):
    """Autograd node for varlen attention (reference: mtlattn/__init__.py:25-46).

    Forward asks the kernel for the natural-log LSE and keeps it for the
    backward, which recomputes P from it. The additive bias is a constant: it
    enters both passes and receives no gradient."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_kv, max_q, scale, causal, window, bias):
        lse = torch.empty((q.shape[0], q.shape[1]), dtype=torch.float32, device=q.device)
        out = _C.varlen_attention(q, k, v, cu_q, cu_kv, max_q, scale, causal, window, lse, bias)
        ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_kv)
        ctx.scale = scale
        ctx.causal = causal
        ctx.window = window
        ctx.bias = bias
        ctx.max_q = max_q
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, cu_q, cu_kv = ctx.saved_tensors
        grads = _C.varlen_attention_bwd(
            q, k, v, out, dout.contiguous(), lse, cu_q, cu_kv,
            ctx.scale, ctx.causal, ctx.window, ctx.bias)
        return (*grads, None, None, None, None, None, None, None)


def _prep_bias(attn_bias):
    """Bring an additive mask to the kernel contract (reference:
    mtlattn/__init__.py:49-63): fp32, 3-D, unit stride on the key dim. A 4-D
    mask [B or 1, H or 1, Nq, max_kv], indexed by sequence and
    sequence-local row (no counterpart in the reference), is passed as it is
    when its key dim has unit stride. A mask that requires grad is rejected
    -- it would be applied but never receive a gradient."""
    if attn_bias is None:
        return None
    if attn_bias.requires_grad:
        raise NotImplementedError(
            "mtlattn: a differentiable attn_bias (requires_grad=True) is not supported; "
            "detach it or treat the mask as constant")
    b = attn_bias if attn_bias.dtype == torch.float32 else attn_bias.float()
    if b.dim() not in (3, 4) or b.stride(-1) != 1:
        b = b.contiguous()
    return b


def varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_kv, max_seqlen_q, scale=None,
                     causal=False, window=0, attn_bias=None):
    """Variable-length attention over packed sequences (reference:
    mtlattn/__init__.py:66-92).

    q: [Mq, Hq, D]; k, v: [Mk, Hkv, D] GPU tensors (fp32/fp16/bf16).
    cu_seqlens_q / cu_seqlens_kv: int [B+1] offsets into the packed rows.
    max_seqlen_q: upper bound on query lengths (routes few-query calls to
        split-KV decode). scale defaults to 1/sqrt(D).
    causal / window / attn_bias: see the module docstring.
    Returns [Mq, Hq, D] in q's dtype. Differentiable in q, k and v."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    cu_q = cu_seqlens_q.int()
    cu_kv = cu_seqlens_kv.int()
    bias = _prep_bias(attn_bias)
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
    if needs_grad:
        return _VarlenAttnFn.apply(q, k, v, cu_q, cu_kv, int(max_seqlen_q), float(scale),
                                   bool(causal), int(window), bias)
    return _C.varlen_attention(q, k, v, cu_q, cu_kv, int(max_seqlen_q), float(scale),
                               bool(causal), int(window), None, bias)


def _window_from_kwargs(window, kwargs):
    """flash_attn's ``window_size=(left, right)`` -> ``window = left + 1``
    (reference: mtlattn/__init__.py:95-101); ``right`` is not used."""
    ws = kwargs.get("window_size")
    if ws is not None and ws[0] is not None and ws[0] >= 0:
        return int(ws[0]) + 1
    return window


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, softmax_scale=None,
                                     causal=False, window=0, **kwargs):
    """flash_attn-style entry, qkv: [M, 3, H, D] (reference:
    mtlattn/__init__.py:104-110). Differentiable; q/k/v are row-strided views."""
    q, k, v = qkv.unbind(dim=1)
    return varlen_attention(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, softmax_scale,
                            causal=causal, window=_window_from_kwargs(window, kwargs))


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                    max_seqlen_k, softmax_scale=None, causal=False, window=0,
                                    **kwargs):
    """flash_attn-style entry, q: [Mq, H, D], kv: [Mkv, 2, Hkv, D] (reference:
    mtlattn/__init__.py:113-120). Differentiable."""
    k, v = kv.unbind(dim=1)
    return varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, softmax_scale,
                            causal=causal, window=_window_from_kwargs(window, kwargs))


def paged_decode(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_kv, block_table, max_seqlen_q,
                 max_seqlen_kv, scale=None, causal=False, window=0, attn_bias=None, lse_out=None):
    """Decode (max_seqlen_q <= 16 query rows per sequence) over a paged KV
    cache; the reference has no paged KV, the layout is FlashAttention's
    varlen call with a block table.

    q: [Mq, Hq, D]; k_cache, v_cache: [num_pages, page_size, Hkv, D] with
    page_size a multiple of 16; block_table: int [B, max_pages], logical key
    j of sequence s in page block_table[s, j // page_size]; cu_seqlens_kv:
    int [B+1] prefix sums of the logical KV lengths; max_seqlen_kv bounds
    them. causal / window / attn_bias as in varlen_attention; lse_out: an
    optional fp32 [Mq, Hq] tensor receiving the natural-log LSE. Forward
    only (fp16/bf16, D in {64, 128}). Returns [Mq, Hq, D]."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _C.paged_decode(q, k_cache, v_cache, cu_seqlens_q.int(), cu_seqlens_kv.int(), block_table.int(),
                           int(max_seqlen_q), int(max_seqlen_kv), float(scale), bool(causal), int(window),
                           lse_out, _prep_bias(attn_bias))


# ---- dense scaled_dot_product_attention adapter ----

_ORIG_SDPA = None
# Query length from which replace_sdpa() intercepts (reference default,
# mtlattn/__init__.py:129).
_SDPA_MIN_SEQLEN = 1024


def _sdpa_mask_to_bias(attn_mask, B, Hq, Nq, Nkv):
    """Dense SDPA mask -> additive fp32 bias [b, h, Nq, Nkv], b in {1, B}, h in
    {1, Hq}, which the kernels index by (sequence, sequence-local row) in
    place (reference: mtlattn/__init__.py:132-159, which copies it to
    [B*Nq, h, Nkv]). Bool masks keep True (0) and drop False (-inf); float
    masks are already additive and are not copied when fp32 with a unit-stride
    key dim (broadcast dims stay stride 0). Shapes: [Nq, Nkv] or
    [b in {1, B}, h in {1, Hq}, Nq, Nkv]. Anything else raises
    NotImplementedError."""
    m = attn_mask
    if m.dim() == 2:
        m = m.reshape(1, 1, Nq, Nkv)
    elif m.dim() != 4:
        raise NotImplementedError("mtlattn: attn_mask must be 2D or 4D")
    elif m.shape[2] != Nq or m.shape[3] != Nkv:
        raise NotImplementedError("mtlattn: attn_mask query/key dims must match")
    if m.dtype == torch.bool:
        m = torch.where(m, torch.zeros((), dtype=torch.float32, device=m.device),
                        torch.full((), float("-inf"), dtype=torch.float32, device=m.device))
    else:
        m = m.float()
    b, h = m.shape[0], m.shape[1]
    if b not in (1, B):
        raise NotImplementedError("mtlattn: attn_mask batch dim must be 1 or B")
    if h not in (1, Hq):
        raise NotImplementedError("mtlattn: attn_mask head dim must be 1 or num_heads")
    if m.stride(-1) != 1 and Nkv > 1:
        m = m.contiguous()
    return m


def sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None):
    """Dense [B, H, N, D] attention through the varlen kernel (reference:
    mtlattn/__init__.py:162-181): equal-length batches become trivial
    cu_seqlens; GQA when key/value have fewer heads; an attn_mask becomes an
    additive bias. Forward only; dropout is not supported."""
    B, Hq, Nq, D = query.shape
    Hkv, Nkv = key.shape[1], key.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q = query.transpose(1, 2).contiguous().view(B * Nq, Hq, D)
    k = key.transpose(1, 2).contiguous().view(B * Nkv, Hkv, D)
    v = value.transpose(1, 2).contiguous().view(B * Nkv, Hkv, D)
    dev = query.device
    cu_q = torch.arange(0, (B + 1) * Nq, Nq, dtype=torch.int32, device=dev)
    cu_kv = torch.arange(0, (B + 1) * Nkv, Nkv, dtype=torch.int32, device=dev)
    bias = None if attn_mask is None else _sdpa_mask_to_bias(attn_mask, B, Hq, Nq, Nkv)
    out = varlen_attention(q, k, v, cu_q, cu_kv, Nq, scale, causal=is_causal, attn_bias=bias)
    return out.view(B, Nq, Hq, D).transpose(1, 2).contiguous()


def _basic_ok(query, key, value, dropout_p, min_seqlen):
    """Whether replace_sdpa() may take a call (reference:
    mtlattn/__init__.py:184-199): 4-D GPU tensors, no dropout, fp32/fp16/bf16,
    D <= 128, GQA-divisible heads, no autograd, and long enough queries."""
    if query.device.type != "cuda" or query.dim() != 4:
        return False
    if dropout_p != 0.0:
        return False
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if query.shape[-1] > 128 or key.shape[-1] > 128:
        return False
    if key.shape[1] == 0 or query.shape[1] % key.shape[1] != 0:
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        return False
    return query.shape[2] >= min_seqlen


# The padding path's one host decision -- a device reduction read back to the
# host -- is made once per mask tensor and reused while that tensor is alive
# and unmodified (same object, version counter, storage, shape and strides):
# a model passes the same mask to every layer's attention call, so a forward
# pass waits on the device once for it, not once per layer. Entries go when
# their mask is freed.
_PAD_DECISIONS = {}


def _padding_decision(attn_mask, B, Hq, Nq, Nkv):
    """(ok, lens) for a self-attention mask over [B, Hq, Nq, Nkv]: ok when it
    depends only on (batch, key) with the kept keys a prefix (and, for a float
    mask, adds exactly 0 to them); lens = kept keys per batch (int32, on the
    mask's device), or None when the mask does not broadcast to that shape.
    Cached per mask tensor (see _PAD_DECISIONS)."""
    sig = (attn_mask._version, attn_mask.data_ptr(), tuple(attn_mask.shape), tuple(attn_mask.stride()),
           B, Hq, Nq, Nkv)
    hit = _PAD_DECISIONS.get(id(attn_mask))
    if hit is not None and hit[0]() is attn_mask and hit[1] == sig:
        return hit[2], hit[3]
    keep0 = attn_mask if attn_mask.dtype == torch.bool else attn_mask > -1e30
    try:
        keep = keep0.expand(B, Hq, Nq, Nkv)
    except RuntimeError:
        return False, None
    kv_keep = keep[:, 0, 0, :]
    lens = kv_keep.sum(dim=1, dtype=torch.int32)
    idx = torch.arange(Nkv, device=attn_mask.device)
    # both tests in one device reduction, compared at the mask's own
    # broadcast shape, not the expanded [B, H, N, N]
    ok = torch.logical_and((keep0 == kv_keep[:, None, None, :]).all(),
                           (kv_keep == (idx[None, :] < lens[:, None])).all())
    if attn_mask.dtype != torch.bool:
        # a float mask is a padding mask only if it adds nothing to the keys
        # it keeps (else its values are an additive bias)
        ok = torch.logical_and(ok, (attn_mask.masked_fill(~keep0, 0) == 0).all())
    ok = bool(ok)
    k = id(attn_mask)
    _PAD_DECISIONS[k] = (weakref.ref(attn_mask, lambda _r, k=k: _PAD_DECISIONS.pop(k, None)), sig, ok, lens)
    return ok, lens


def _try_padding_varlen(query, key, value, attn_mask, is_causal, scale):
    """Self-attention key-padding mask -> packed varlen call (reference:
    mtlattn/__init__.py:202-249). Applies when the mask depends only on
    (batch, key) and keeps a contiguous key prefix per batch, and a float mask
    adds exactly 0 to the keys it keeps; returns the dense [B, H, N, D] result
    with padded query rows zeroed, or None when the mask is not of that form.
    (The reference takes any float mask without -inf entries as keep-all and
    drops its values; here such a mask is left to the additive-bias path.)"""
    B, Hq, Nq, D = query.shape
    Hkv, Nkv = key.shape[1], key.shape[2]
    if Nq != Nkv:
        return None
    # the one host decision, made once per mask tensor (_padding_decision)
    ok, lens = _padding_decision(attn_mask, B, Hq, Nq, Nkv)
    if not ok:
        return None
    # pack, attend, unpack on the device: no lengths on the host, no
    # per-batch copies (rows past cu[B] belong to no sequence)
    qp, cu = _C.pack_padded(query, lens)
    kp, _ = _C.pack_padded(key, lens)
    vp, _ = _C.pack_padded(value, lens)
    op = varlen_attention(qp, kp, vp, cu, cu, Nq, scale, causal=is_causal)
    return _C.unpack_padded(op, cu, lens, B, Nq)


def replace_sdpa(min_seqlen=_SDPA_MIN_SEQLEN):
    """Monkey-patch torch.nn.functional.scaled_dot_product_attention so calls
    this library handles well (long queries, padding masks, additive masks,
    forward only) run here and all others go to the original (reference:
    mtlattn/__init__.py:252-287). Idempotent; undo with restore_sdpa()."""
    global _ORIG_SDPA
    if _ORIG_SDPA is None:
        _ORIG_SDPA = torch.nn.functional.scaled_dot_product_attention
    orig = _ORIG_SDPA

    def patched(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                scale=None, **kwargs):
        if _basic_ok(query, key, value, dropout_p, min_seqlen):
            sc = scale if scale is not None else 1.0 / math.sqrt(query.shape[-1])
            if attn_mask is None:
                # end-aligned causal differs from SDPA's top-left convention
                # unless the query and key lengths agree
                if not (is_causal and query.shape[2] != key.shape[2]):
                    return sdpa(query, key, value, None, dropout_p, is_causal, scale)
            else:
                r = _try_padding_varlen(query, key, value, attn_mask, is_causal, sc)
                if r is not None:
                    return r
                try:
                    return sdpa(query, key, value, attn_mask, dropout_p, is_causal, scale)
                except (NotImplementedError, RuntimeError):
                    pass
        return orig(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                    is_causal=is_causal, scale=scale, **kwargs)

    torch.nn.functional.scaled_dot_product_attention = patched


def restore_sdpa():
    """Undo replace_sdpa() (reference: mtlattn/__init__.py:290-295)."""
    global _ORIG_SDPA
    if _ORIG_SDPA is not None:
        torch.nn.functional.scaled_dot_product_attention = _ORIG_SDPA
        _ORIG_SDPA = None
