"""Host-side logic of the Python API (mtlattn_amd/__init__.py) that needs no
GPU: window mapping, bias preparation, SDPA mask -> bias layout, the
replace_sdpa gate and fallbacks, and the binding's argument checks."""

import pytest
import torch
import torch.nn.functional as F

import mtlattn
import mtlattn_amd as M


def test_import_name_is_the_same_module():
    assert mtlattn.varlen_attention is M.varlen_attention
    assert mtlattn._C is M._C
    assert set(mtlattn.__all__) == {"varlen_attention", "flash_attn_varlen_qkvpacked_func",
                                    "flash_attn_varlen_kvpacked_func", "sdpa", "replace_sdpa", "restore_sdpa"}
    # paged-KV decode has no reference counterpart: reachable, not in __all__
    assert mtlattn.paged_decode is M.paged_decode and hasattr(M._C, "paged_decode")


def test_binding_exports_reference_names():
    for n in ("varlen_attention", "varlen_attention_bwd", "attn_splitkv", "mpp_bwd_dq", "mpp_bwd_dkv",
              "mpp_available", "gpu_core_count"):
        assert hasattr(M._C, n), n
    assert M._C.mpp_available() is True


def test_window_from_kwargs():
    # flash_attn window_size=(left, right) -> window = left + 1 (mtlattn/__init__.py:95-101)
    assert M._window_from_kwargs(0, {"window_size": (127, 0)}) == 128
    assert M._window_from_kwargs(5, {"window_size": (-1, -1)}) == 5
    assert M._window_from_kwargs(7, {}) == 7
    assert M._window_from_kwargs(7, {"window_size": (None, 0)}) == 7


def test_prep_bias():
    assert M._prep_bias(None) is None
    b = torch.randn(4, 1, 6, dtype=torch.float64)
    out = M._prep_bias(b)
    assert out.dtype == torch.float32 and out.stride(-1) == 1
    nc = torch.randn(4, 6, 2).transpose(1, 2)          # last dim not contiguous
    assert M._prep_bias(nc).is_contiguous()
    with pytest.raises(NotImplementedError, match="differentiable attn_bias"):
        M._prep_bias(torch.randn(2, 1, 3, requires_grad=True))


def test_sdpa_mask_to_bias_bool_and_float():
    """Dense masks become [b, h, Nq, Nkv] fp32 additive biases that the kernels
    index by (sequence, local row): bool -> 0 / -inf, fp32 float masks used in
    place (no copy), broadcast dims kept at size 1."""
    B, H, Nq, Nkv = 2, 3, 4, 5
    m = torch.rand(B, H, Nq, Nkv) > 0.5
    b = M._sdpa_mask_to_bias(m, B, H, Nq, Nkv)
    assert b.shape == (B, H, Nq, Nkv) and b.dtype == torch.float32
    assert torch.equal(b, torch.where(m, 0.0, float("-inf")))
    f = torch.randn(1, 1, Nq, Nkv)
    bf = M._sdpa_mask_to_bias(f, B, H, Nq, Nkv)
    assert bf.shape == (1, 1, Nq, Nkv) and bf.data_ptr() == f.data_ptr()   # in place
    two_d = M._sdpa_mask_to_bias(f[0, 0], B, H, Nq, Nkv)
    assert two_d.shape == (1, 1, Nq, Nkv) and two_d.data_ptr() == f.data_ptr()
    full = torch.randn(B, H, Nq, Nkv)
    assert M._sdpa_mask_to_bias(full, B, H, Nq, Nkv).data_ptr() == full.data_ptr()
    # a strided key dim is made contiguous; half precision is cast to fp32
    t = torch.randn(B, H, Nkv, Nq).transpose(2, 3)
    assert M._sdpa_mask_to_bias(t, B, H, Nq, Nkv).stride(-1) == 1
    assert M._sdpa_mask_to_bias(full.half(), B, H, Nq, Nkv).dtype == torch.float32
    # _prep_bias keeps a 4-D mask with a unit-stride key dim as it is
    assert M._prep_bias(full).data_ptr() == full.data_ptr()


@pytest.mark.parametrize("shape,msg", [
    ((2, 3, 5), "2D or 4D"),
    ((2, 3, 4, 6), "query/key dims"),
    ((3, 1, 4, 5), "batch dim"),
    ((2, 2, 4, 5), "head dim"),
])
def test_sdpa_mask_rejects(shape, msg):
    with pytest.raises(NotImplementedError, match=msg):
        M._sdpa_mask_to_bias(torch.zeros(shape), 2, 3, 4, 5)


def test_basic_ok_gate_on_cpu():
    q = torch.randn(1, 8, 2048, 64)
    assert not M._basic_ok(q, q, q, 0.0, 1024)            # not a GPU tensor

    class FakeDev:
        type = "cuda"

    class T:
        def __init__(self, shape, dtype=torch.float16, rg=False):
            self.shape, self.dtype, self.requires_grad, self.device = shape, dtype, rg, FakeDev()

        def dim(self):
            return len(self.shape)

    ok = T((1, 8, 2048, 64))
    assert M._basic_ok(ok, T((1, 2, 2048, 64)), ok, 0.0, 1024)
    assert not M._basic_ok(ok, ok, ok, 0.1, 1024)                         # dropout
    assert not M._basic_ok(T((1, 8, 2048, 64), torch.float64), ok, ok, 0.0, 1024)
    assert not M._basic_ok(T((1, 8, 2048, 160)), ok, ok, 0.0, 1024)      # D > 128
    assert not M._basic_ok(ok, T((1, 3, 2048, 64)), ok, 0.0, 1024)        # GQA divisibility
    assert not M._basic_ok(T((1, 8, 512, 64)), ok, ok, 0.0, 1024)         # below min_seqlen
    with torch.enable_grad():
        assert not M._basic_ok(T((1, 8, 2048, 64), rg=True), ok, ok, 0.0, 1024)


def test_replace_restore_idempotent_and_fallback():
    orig = F.scaled_dot_product_attention
    M.replace_sdpa()
    patched = F.scaled_dot_product_attention
    M.replace_sdpa()                                        # idempotent: still wraps the original
    try:
        assert F.scaled_dot_product_attention is not orig
        q = torch.randn(1, 2, 8, 16)
        # CPU tensors are never intercepted: identical to native SDPA
        assert torch.equal(F.scaled_dot_product_attention(q, q, q, is_causal=True),
                           orig(q, q, q, is_causal=True))
    finally:
        M.restore_sdpa()
    assert F.scaled_dot_product_attention is orig
    M.restore_sdpa()                                        # no-op
    assert F.scaled_dot_product_attention is orig
    del patched


def test_padding_mask_detection_rejects_non_padding():
    q = torch.randn(2, 2, 6, 8)
    # query-dependent mask: not a key-padding mask
    m = torch.ones(2, 1, 6, 6, dtype=torch.bool).tril()
    assert M._try_padding_varlen(q, q, q, m, False, 0.3) is None
    # non-prefix keep pattern
    m2 = torch.ones(2, 1, 1, 6, dtype=torch.bool)
    m2[:, :, :, 1] = False
    assert M._try_padding_varlen(q, q, q, m2, False, 0.3) is None
    # cross-attention shapes are not token padding
    assert M._try_padding_varlen(q, torch.randn(2, 2, 7, 8), torch.randn(2, 2, 7, 8),
                                 torch.ones(2, 1, 1, 7, dtype=torch.bool), False, 0.3) is None


def test_padding_decision_cached_per_mask():
    """The padding path's host decision is made once per mask tensor: a second
    call with the same, unmodified mask reuses it (the same lens tensor, no
    new device reduction); an in-place change, another shape or another mask
    decides again; the entry goes when the mask is freed."""
    import gc
    B, H, N = 3, 2, 8
    m = torch.zeros(B, 1, 1, N, dtype=torch.bool)
    for b, n in enumerate((5, 8, 1)):
        m[b, :, :, :n] = True
    ok, lens = M._padding_decision(m, B, H, N, N)
    assert ok and lens.tolist() == [5, 8, 1]
    ok2, lens2 = M._padding_decision(m, B, H, N, N)
    assert ok2 and lens2 is lens
    assert id(m) in M._PAD_DECISIONS
    # another broadcast shape of the same mask is decided afresh
    ok3, lens3 = M._padding_decision(m, B, 4, N, N)
    assert ok3 and lens3 is not lens
    # a change through another view of the same storage (views share the
    # version counter): batch 2 keeps keys 0-1, still a prefix, new lengths
    m.view(B, N)[2, 1] = True
    ok5, lens5 = M._padding_decision(m, B, H, N, N)
    assert ok5 and lens5.tolist() == [5, 8, 2]
    # in place: key 6 of batch 0 kept -> no longer a prefix
    m[0, 0, 0, 6] = True
    ok4, _ = M._padding_decision(m, B, H, N, N)
    assert not ok4
    # a float mask with a nonzero value on a kept key is a bias, not padding
    f = torch.zeros(B, 1, 1, N)
    f[:, :, :, 6:] = float("-inf")
    assert M._padding_decision(f, B, H, N, N)[0]
    f2 = f.clone()
    f2[1, 0, 0, 0] = 0.5
    assert not M._padding_decision(f2, B, H, N, N)[0]
    # a query-dependent mask
    assert not M._padding_decision(torch.ones(B, 1, N, N, dtype=torch.bool).tril(), B, H, N, N)[0]
    k = id(m)
    del m
    gc.collect()
    assert k not in M._PAD_DECISIONS


def test_binding_rejects_cpu_tensors():
    q = torch.randn(4, 2, 8)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        M._C.varlen_attention(q, q, q, cu, cu, 4, 0.3, False, 0, None, None)
    with pytest.raises(RuntimeError, match="GPU"):
        M.varlen_attention(q, q, q, cu, cu, 4)
