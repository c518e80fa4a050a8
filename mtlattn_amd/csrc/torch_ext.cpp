// mtlattn._C for PyTorch-ROCm: the thin torch binding over the C ABI of
// libmtlattn_hip.so. Replaces the reference's pybind11 module
// (src/ext.mm:784-811) with the same function names, argument names and
// defaults. Tensor checks mirror src/ext.mm:306-365 (TORCH_CHECK ->
// RuntimeError); outputs and scratch are allocated through torch's caching
// allocator; work is enqueued on the current HIP stream of the input's device
// with no host synchronisation.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <tuple>

#include "../../include/mtlattn_capi.h"

namespace {

int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return MTLATTN_DTYPE_F32;
        case at::kHalf: return MTLATTN_DTYPE_F16;
        case at::kBFloat16: return MTLATTN_DTYPE_BF16;
        default: TORCH_CHECK(false, "mtlattn: unsupported dtype ", t);
    }
    return -1;
}

void check_rc(int rc) { TORCH_CHECK(rc == MTLATTN_OK, mtlattn_last_error()); }

void* current_stream(const at::Tensor& t) {
    return (void*)at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

bool defined(const c10::optional<at::Tensor>& t) { return t.has_value() && t->defined() && t->numel() > 0; }

// q/k/v layout checks of src/ext.mm:306-331.
void check_qkv(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "mtlattn: q/k/v must be GPU (HIP) tensors");
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "mtlattn: q/k/v must be [M, H, D]");
    const auto H = q.size(1), H_kv = k.size(1), D = q.size(2);
    TORCH_CHECK(D >= 1 && D <= 256, "mtlattn: head_dim ", D, " unsupported (expected 1..256)");
    TORCH_CHECK(v.size(1) == H_kv && k.size(2) == D && v.size(2) == D, "mtlattn: k/v head/dim shape mismatch");
    TORCH_CHECK(k.size(0) == v.size(0), "mtlattn: k/v token count mismatch");
    TORCH_CHECK(H_kv > 0 && H % H_kv == 0, "mtlattn: query heads (", H, ") must be a multiple of kv heads (", H_kv,
                ")");
    TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(), "mtlattn: dtype mismatch");
    dtype_code(q.scalar_type());
    for (const auto& t : {q, k, v}) {
        TORCH_CHECK((t.size(2) == 1 || t.stride(2) == 1) && (t.size(1) == 1 || t.stride(1) == D),
                    "mtlattn: inner dims must be contiguous ([M, H, D] with row-only striding)");
        TORCH_CHECK(t.get_device() == q.get_device(), "mtlattn: q/k/v must be on the same device");
    }
}

void check_cu(const at::Tensor& cu_q, const at::Tensor& cu_kv, const at::Tensor& q) {
    TORCH_CHECK(cu_q.is_cuda() && cu_kv.is_cuda(), "mtlattn: cu_seqlens must be on the GPU");
    TORCH_CHECK(cu_q.get_device() == q.get_device() && cu_kv.get_device() == q.get_device(),
                "mtlattn: cu_seqlens must be on the device of q");
    TORCH_CHECK(cu_q.scalar_type() == at::kInt && cu_kv.scalar_type() == at::kInt, "mtlattn: cu_seqlens must be int32");
    TORCH_CHECK(cu_q.dim() == 1 && cu_kv.dim() == 1 && cu_q.numel() == cu_kv.numel() && cu_q.numel() >= 2,
                "mtlattn: cu_seqlens_q/kv must both be [B+1]");
}

// lse / delta of the backward test entries: [total_q, Hq] on q's device.
void check_rowhead(const at::Tensor& t, const at::Tensor& q, const char* name) {
    TORCH_CHECK(t.is_cuda() && t.get_device() == q.get_device() && t.dim() == 2 && t.size(0) == q.size(0) &&
                    t.size(1) == q.size(1),
                "mtlattn: ", name, " must be a [total_q, H] GPU tensor");
}

int64_t row_stride(const at::Tensor& t) { return t.size(0) > 1 ? t.stride(0) : t.size(1) * t.size(2); }

// Bias checks of src/ext.mm:348-365, plus the key-dim extent for bounds.
// Also accepted (no counterpart in the reference): a 4-D mask [B or 1,
// H or 1, Nq, max_kv] indexed by (sequence, sequence-local row), used in
// place (the SDPA adapter's dense masks).
void fill_bias(mtlattn_problem& p, const c10::optional<at::Tensor>& attn_bias, const at::Tensor& q,
               at::Tensor& keep) {
    p.bias = nullptr;
    p.bias_q_stride = p.bias_h_stride = p.bias_kv_cols = 0;
    p.bias_seq_local = 0;
    p.bias_seq_stride = p.bias_seq_rows = 0;
    if (!defined(attn_bias)) return;
    keep = *attn_bias;
    TORCH_CHECK(keep.is_cuda() && keep.get_device() == q.get_device(), "mtlattn: attn_mask must be a GPU tensor");
    TORCH_CHECK(keep.scalar_type() == at::kFloat, "mtlattn: attn_mask must be float32");
    if (keep.dim() == 4) {
        TORCH_CHECK(keep.size(0) == p.num_seqs || keep.size(0) == 1,
                    "mtlattn: a 4-D attn_mask's dim0 must be the number of sequences or 1");
        TORCH_CHECK(keep.size(1) == q.size(1) || keep.size(1) == 1, "mtlattn: attn_mask dim1 must be num_heads (",
                    q.size(1), ") or 1 (broadcast)");
        TORCH_CHECK(keep.size(2) >= 1, "mtlattn: a 4-D attn_mask needs at least one query row");
        TORCH_CHECK(keep.size(3) <= 1 || keep.stride(3) == 1, "mtlattn: attn_mask last dim must be contiguous");
        TORCH_CHECK(keep.stride(0) >= 0 && keep.stride(1) >= 0 && keep.stride(2) >= 0,
                    "mtlattn: attn_mask strides must be non-negative");
        p.bias = keep.data_ptr<float>();
        p.bias_seq_local = 1;
        p.bias_seq_stride = keep.size(0) == 1 ? 0 : keep.stride(0);
        p.bias_seq_rows = keep.size(2);
        p.bias_q_stride = keep.stride(2);
        p.bias_h_stride = keep.size(1) == 1 ? 0 : keep.stride(1);
        p.bias_kv_cols = keep.size(3);
        return;
    }
    TORCH_CHECK(keep.dim() == 3, "mtlattn: attn_mask must be [total_q, H or 1, max_kv]");
    TORCH_CHECK(keep.size(0) == q.size(0), "mtlattn: attn_mask dim0 (", keep.size(0), ") must equal total_q (",
                q.size(0), ")");
    TORCH_CHECK(keep.size(1) == q.size(1) || keep.size(1) == 1, "mtlattn: attn_mask dim1 must be num_heads (",
                q.size(1), ") or 1 (broadcast)");
    TORCH_CHECK(keep.size(2) <= 1 || keep.stride(2) == 1, "mtlattn: attn_mask last dim must be contiguous");
    p.bias = keep.data_ptr<float>();
    p.bias_q_stride = keep.stride(0);
    p.bias_h_stride = keep.size(1) == 1 ? 0 : keep.stride(1);
    p.bias_kv_cols = keep.size(2);
}

mtlattn_problem make_problem(const at::Tensor& q, const at::Tensor& k, const at::Tensor& cu_q,
                             const at::Tensor& cu_kv, int64_t max_seqlen_q, double scale, bool causal,
                             int64_t window) {
    mtlattn_problem p;
    std::memset(&p, 0, sizeof(p));
    p.dtype = dtype_code(q.scalar_type());
    p.num_seqs = (int32_t)(cu_q.numel() - 1);
    p.total_q = q.size(0);
    p.total_kv = k.size(0);
    p.num_heads_q = (int32_t)q.size(1);
    p.num_heads_kv = (int32_t)k.size(1);
    p.head_dim = (int32_t)q.size(2);
    p.max_seqlen_q = (int32_t)std::min<int64_t>(max_seqlen_q, 0x7fffffff);
    p.scale = (float)scale;
    p.causal = causal ? 1 : 0;
    p.window = window > 0 ? (int32_t)std::min<int64_t>(window, 0x7fffffff) : 0;
    p.cu_seqlens_q = cu_q.data_ptr<int32_t>();
    p.cu_seqlens_kv = cu_kv.data_ptr<int32_t>();
    return p;
}

at::Tensor workspace(int64_t bytes, const at::Tensor& like) {
    return at::empty({std::max<int64_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// _C.varlen_attention (src/ext.mm:293-489).
at::Tensor varlen_attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                            const at::Tensor& cu_seqlens_q, const at::Tensor& cu_seqlens_kv, int64_t max_seqlen_q,
                            double scale, bool causal, int64_t window, c10::optional<at::Tensor> lse_out,
                            c10::optional<at::Tensor> attn_bias) {
    check_qkv(q, k, v);
    check_cu(cu_seqlens_q, cu_seqlens_kv, q);
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_seqlens_q.contiguous(), cu_kv = cu_seqlens_kv.contiguous();
    auto out = at::empty({q.size(0), q.size(1), q.size(2)}, q.options());
    float* lse = nullptr;
    if (defined(lse_out)) {
        const at::Tensor& l = *lse_out;
        TORCH_CHECK(l.is_cuda() && l.scalar_type() == at::kFloat && l.is_contiguous() && l.dim() == 2 &&
                        l.size(0) == q.size(0) && l.size(1) == q.size(1),
                    "mtlattn: lse_out must be a contiguous fp32 [total_q, H] GPU tensor");
        lse = l.data_ptr<float>();
    }
    if (q.size(0) == 0) return out;
    mtlattn_problem p = make_problem(q, k, cu_q, cu_kv, max_seqlen_q, scale, causal, window);
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    const size_t ws_bytes = mtlattn_varlen_fwd_workspace_size(&p);
    at::Tensor ws = workspace((int64_t)ws_bytes, q);
    check_rc(mtlattn_varlen_fwd(&p, q.data_ptr(), row_stride(q), k.data_ptr(), row_stride(k), v.data_ptr(),
                                row_stride(v), out.data_ptr(), lse, ws.data_ptr(), ws_bytes, current_stream(q)));
    return out;
}

// _C.varlen_attention_bwd (src/ext.mm:502-594).
std::tuple<at::Tensor, at::Tensor, at::Tensor> varlen_attention_bwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& o, const at::Tensor& dout,
    const at::Tensor& lse, const at::Tensor& cu_seqlens_q, const at::Tensor& cu_seqlens_kv, double scale,
    bool causal, int64_t window, c10::optional<at::Tensor> attn_bias) {
    check_qkv(q, k, v);
    check_cu(cu_seqlens_q, cu_seqlens_kv, q);
    TORCH_CHECK(o.sizes() == q.sizes() && dout.sizes() == q.sizes(), "mtlattn: o/dout must match q's shape");
    TORCH_CHECK(o.scalar_type() == q.scalar_type() && dout.scalar_type() == q.scalar_type(),
                "mtlattn: o/dout dtype mismatch");
    check_qkv(o, dout, dout);
    TORCH_CHECK(lse.is_cuda() && lse.scalar_type() == at::kFloat && lse.is_contiguous() && lse.dim() == 2 &&
                    lse.size(0) == q.size(0) && lse.size(1) == q.size(1),
                "mtlattn: lse must be a contiguous fp32 [total_q, H] GPU tensor");
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_seqlens_q.contiguous(), cu_kv = cu_seqlens_kv.contiguous();
    auto dQ = at::empty({q.size(0), q.size(1), q.size(2)}, q.options());
    auto dK = at::empty({k.size(0), k.size(1), k.size(2)}, k.options());
    auto dV = at::empty({v.size(0), v.size(1), v.size(2)}, v.options());
    mtlattn_problem p = make_problem(q, k, cu_q, cu_kv, q.size(0), scale, causal, window);
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    const size_t ws_bytes = mtlattn_varlen_bwd_workspace_size(&p);
    at::Tensor ws = workspace((int64_t)ws_bytes, q);
    check_rc(mtlattn_varlen_bwd(&p, q.data_ptr(), row_stride(q), k.data_ptr(), row_stride(k), v.data_ptr(),
                                row_stride(v), o.data_ptr(), row_stride(o), dout.data_ptr(), row_stride(dout),
                                lse.data_ptr<float>(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(), ws.data_ptr(),
                                ws_bytes, current_stream(q)));
    return {dQ, dK, dV};
}

// _C.attn_splitkv (src/ext.mm:716-773). `window` and `attn_bias` (after the
// reference's arguments) have no counterpart there: its split path takes
// neither.
at::Tensor attn_splitkv(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& cu_q_in,
                        const at::Tensor& cu_kv_in, int64_t max_seqlen_q, double scale, bool causal,
                        int64_t num_splits, int64_t window, c10::optional<at::Tensor> attn_bias) {
    check_qkv(q, k, v);
    check_cu(cu_q_in, cu_kv_in, q);
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_q_in.contiguous(), cu_kv = cu_kv_in.contiguous();
    auto out = at::empty({q.size(0), q.size(1), q.size(2)}, q.options());
    mtlattn_problem p = make_problem(q, k, cu_q, cu_kv, max_seqlen_q, scale, causal, window);
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    const size_t ws_bytes = mtlattn_attn_splitkv_workspace_size(&p, (int32_t)num_splits);
    at::Tensor ws = workspace((int64_t)ws_bytes, q);
    check_rc(mtlattn_attn_splitkv(&p, q.data_ptr(), row_stride(q), k.data_ptr(), row_stride(k), v.data_ptr(),
                                  row_stride(v), out.data_ptr(), nullptr, (int32_t)num_splits, ws.data_ptr(), ws_bytes,
                                  current_stream(q)));
    return out;
}

// _C.paged_decode: decode over a paged KV cache (no reference counterpart).
// k_cache / v_cache [num_pages, page_size, Hkv, D] (token rows may be
// strided; pages are page_size consecutive token rows), block_table int32
// [B, max_pages], cu_seqlens_kv the logical KV lengths.
at::Tensor paged_decode(const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                        const at::Tensor& cu_seqlens_q, const at::Tensor& cu_seqlens_kv, const at::Tensor& block_table,
                        int64_t max_seqlen_q, int64_t max_seqlen_kv, double scale, bool causal, int64_t window,
                        c10::optional<at::Tensor> lse_out, c10::optional<at::Tensor> attn_bias) {
    TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda(), "mtlattn: q/k_cache/v_cache must be GPU tensors");
    TORCH_CHECK(q.dim() == 3, "mtlattn: q must be [M, H, D]");
    TORCH_CHECK(k_cache.dim() == 4 && v_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes(),
                "mtlattn: k_cache/v_cache must both be [num_pages, page_size, Hkv, D]");
    const int64_t D = q.size(2), Hkv = k_cache.size(2), page_size = k_cache.size(1);
    TORCH_CHECK(k_cache.size(3) == D, "mtlattn: k_cache head dim must match q");
    TORCH_CHECK(Hkv > 0 && q.size(1) % Hkv == 0, "mtlattn: query heads must be a multiple of kv heads");
    TORCH_CHECK(q.scalar_type() == k_cache.scalar_type() && q.scalar_type() == v_cache.scalar_type(),
                "mtlattn: dtype mismatch");
    dtype_code(q.scalar_type());
    TORCH_CHECK((q.size(2) == 1 || q.stride(2) == 1) && (q.size(1) == 1 || q.stride(1) == D),
                "mtlattn: q inner dims must be contiguous");
    for (const auto& c : {k_cache, v_cache}) {
        TORCH_CHECK(c.stride(3) == 1 && (Hkv == 1 || c.stride(2) == D),
                    "mtlattn: cache inner dims [Hkv, D] must be contiguous");
        TORCH_CHECK(c.size(0) <= 1 || c.stride(0) == page_size * c.stride(1),
                    "mtlattn: cache pages must be page_size consecutive token rows");
        TORCH_CHECK(c.get_device() == q.get_device(), "mtlattn: q and the caches must be on the same device");
    }
    check_cu(cu_seqlens_q, cu_seqlens_kv, q);
    TORCH_CHECK(block_table.is_cuda() && block_table.get_device() == q.get_device() &&
                    block_table.scalar_type() == at::kInt && block_table.dim() == 2 &&
                    block_table.size(0) == cu_seqlens_q.numel() - 1,
                "mtlattn: block_table must be an int32 [B, max_pages] GPU tensor");
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_seqlens_q.contiguous(), cu_kv = cu_seqlens_kv.contiguous();
    TORCH_CHECK(max_seqlen_kv >= 0 && block_table.size(1) * page_size >= max_seqlen_kv,
                "mtlattn: block_table has ", block_table.size(1), " pages of ", page_size,
                " tokens per sequence, fewer than max_seqlen_kv (", max_seqlen_kv, ")");
    // one row of block_table.size(1) entries per sequence (the kernel clamps
    // its column reads to the row stride, so the rows must be dense)
    auto bt = block_table.contiguous();
    auto out = at::empty({q.size(0), q.size(1), q.size(2)}, q.options());
    float* lse = nullptr;
    if (defined(lse_out)) {
        const at::Tensor& l = *lse_out;
        TORCH_CHECK(l.is_cuda() && l.scalar_type() == at::kFloat && l.is_contiguous() && l.dim() == 2 &&
                        l.size(0) == q.size(0) && l.size(1) == q.size(1),
                    "mtlattn: lse_out must be a contiguous fp32 [total_q, H] GPU tensor");
        lse = l.data_ptr<float>();
    }
    if (q.size(0) == 0) return out;
    mtlattn_problem p;
    std::memset(&p, 0, sizeof(p));
    p.dtype = dtype_code(q.scalar_type());
    p.num_seqs = (int32_t)(cu_q.numel() - 1);
    p.total_q = q.size(0);
    // an upper bound on the logical KV total (cu_seqlens_kv[B]) from the
    // logical lengths alone: sequences may share pages (prefix caching, beam
    // search), so the sum can exceed the cache's capacity
    p.total_kv = std::min<int64_t>((int64_t)p.num_seqs * std::max<int64_t>(max_seqlen_kv, 0), 0x7fffffff);
    p.num_heads_q = (int32_t)q.size(1);
    p.num_heads_kv = (int32_t)Hkv;
    p.head_dim = (int32_t)D;
    p.max_seqlen_q = (int32_t)std::min<int64_t>(max_seqlen_q, 0x7fffffff);
    p.scale = (float)scale;
    p.causal = causal ? 1 : 0;
    p.window = window > 0 ? (int32_t)std::min<int64_t>(window, 0x7fffffff) : 0;
    p.cu_seqlens_q = cu_q.data_ptr<int32_t>();
    p.cu_seqlens_kv = cu_kv.data_ptr<int32_t>();
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    const size_t ws_bytes = mtlattn_paged_decode_workspace_size(&p, max_seqlen_kv);
    at::Tensor ws = workspace((int64_t)ws_bytes, q);
    const int64_t krs = k_cache.size(1) > 1 ? k_cache.stride(1) : Hkv * D;
    const int64_t vrs = v_cache.size(1) > 1 ? v_cache.stride(1) : Hkv * D;
    check_rc(mtlattn_paged_decode(&p, q.data_ptr(), row_stride(q), k_cache.data_ptr(), krs, v_cache.data_ptr(), vrs,
                                  (int32_t)page_size, k_cache.size(0), bt.data_ptr<int32_t>(), bt.stride(0),
                                  max_seqlen_kv, out.data_ptr(), lse, ws.data_ptr(), ws_bytes, current_stream(q)));
    return out;
}

// _C.mpp_bwd_dq (src/ext.mm:656-711): fp32 dQ.
at::Tensor mpp_bwd_dq(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& dO,
                      const at::Tensor& lse, const at::Tensor& delta, const at::Tensor& cu_q_in,
                      const at::Tensor& cu_kv_in, int64_t max_seqlen_q, double scale, bool causal, int64_t window,
                      c10::optional<at::Tensor> attn_bias) {
    check_qkv(q, k, v);
    check_cu(cu_q_in, cu_kv_in, q);
    TORCH_CHECK(dO.sizes() == q.sizes() && dO.scalar_type() == q.scalar_type(), "mtlattn: dO must match q");
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_q_in.contiguous(), cu_kv = cu_kv_in.contiguous();
    auto dOc = dO.contiguous();
    check_rowhead(lse, q, "lse");
    check_rowhead(delta, q, "delta");
    auto lsec = lse.to(at::kFloat).contiguous(), deltac = delta.to(at::kFloat).contiguous();
    auto dQ = at::zeros({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat));
    mtlattn_problem p = make_problem(q, k, cu_q, cu_kv, max_seqlen_q, scale, causal, window);
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    check_rc(mtlattn_bwd_dq(&p, q.data_ptr(), row_stride(q), k.data_ptr(), row_stride(k), v.data_ptr(),
                            row_stride(v), dOc.data_ptr(), row_stride(dOc), lsec.data_ptr<float>(),
                            deltac.data_ptr<float>(), dQ.data_ptr(), MTLATTN_DTYPE_F32, current_stream(q)));
    return dQ;
}

// _C.mpp_bwd_dkv (src/ext.mm:597-653): fp32 (dK, dV).
std::tuple<at::Tensor, at::Tensor> mpp_bwd_dkv(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                               const at::Tensor& dO, const at::Tensor& lse, const at::Tensor& delta,
                                               const at::Tensor& cu_q_in, const at::Tensor& cu_kv_in,
                                               int64_t max_seqlen_kv, double scale, bool causal, int64_t window,
                                               c10::optional<at::Tensor> attn_bias) {
    (void)max_seqlen_kv;   // grids are sized from tensor shapes; no host sync needed
    check_qkv(q, k, v);
    check_cu(cu_q_in, cu_kv_in, q);
    TORCH_CHECK(dO.sizes() == q.sizes() && dO.scalar_type() == q.scalar_type(), "mtlattn: dO must match q");
    const c10::OptionalDeviceGuard guard(q.device());
    auto cu_q = cu_q_in.contiguous(), cu_kv = cu_kv_in.contiguous();
    auto dOc = dO.contiguous();
    check_rowhead(lse, q, "lse");
    check_rowhead(delta, q, "delta");
    auto lsec = lse.to(at::kFloat).contiguous(), deltac = delta.to(at::kFloat).contiguous();
    auto dK = at::zeros({k.size(0), k.size(1), k.size(2)}, k.options().dtype(at::kFloat));
    auto dV = at::zeros_like(dK);
    mtlattn_problem p = make_problem(q, k, cu_q, cu_kv, q.size(0), scale, causal, window);
    at::Tensor bias_keep;
    fill_bias(p, attn_bias, q, bias_keep);
    check_rc(mtlattn_bwd_dkv(&p, q.data_ptr(), row_stride(q), k.data_ptr(), row_stride(k), v.data_ptr(),
                             row_stride(v), dOc.data_ptr(), row_stride(dOc), lsec.data_ptr<float>(),
                             deltac.data_ptr<float>(), dK.data_ptr(), dV.data_ptr(), MTLATTN_DTYPE_F32,
                             current_stream(q)));
    return {dK, dV};
}

// The reference's "is the fast path usable here" probe (src/ext.mm:780-782):
// the MFMA kernels are compiled into this build for gfx950.
// SDPA key-padding adapter on the device (see mtlattn_pack_padded): x is
// dense [B, H, N, D] with D contiguous, lens int32 [B] on x's device. Returns
// the packed rows [B * N, H, D] and cu_seqlens [B + 1].
std::tuple<at::Tensor, at::Tensor> pack_padded(const at::Tensor& x_in, const at::Tensor& lens) {
    TORCH_CHECK(x_in.is_cuda() && x_in.dim() == 4, "mtlattn: pack_padded expects a [B, H, N, D] GPU tensor");
    const at::Tensor x = (x_in.size(3) == 1 || x_in.stride(3) == 1) ? x_in : x_in.contiguous();
    TORCH_CHECK(lens.is_cuda() && lens.scalar_type() == at::kInt && lens.dim() == 1 && lens.size(0) == x.size(0) &&
                    lens.get_device() == x.get_device(),
                "mtlattn: lens must be int32 [B] on the device of x");
    const c10::DeviceGuard guard(x.device());
    const auto B = x.size(0), H = x.size(1), N = x.size(2), D = x.size(3);
    auto lc = lens.contiguous();
    auto packed = at::empty({B * N, H, D}, x.options());
    auto cu = at::empty({B + 1}, lens.options());
    check_rc(mtlattn_pack_padded(dtype_code(x.scalar_type()), (int32_t)B, (int32_t)N, (int32_t)H, (int32_t)D,
                                 x.data_ptr(), x.stride(0), x.stride(1), x.stride(2), lc.data_ptr<int32_t>(),
                                 cu.data_ptr<int32_t>(), packed.data_ptr(), current_stream(x)));
    return {packed, cu};
}

// Inverse of pack_padded: packed rows [B * N, H, D] -> dense contiguous
// [B, H, N, D], zeros for padded tokens.
at::Tensor unpack_padded(const at::Tensor& packed, const at::Tensor& cu, const at::Tensor& lens, int64_t B,
                         int64_t N) {
    TORCH_CHECK(packed.is_cuda() && packed.dim() == 3 && packed.size(0) == B * N,
                "mtlattn: unpack_padded expects packed rows [B * N, H, D]");
    TORCH_CHECK(cu.scalar_type() == at::kInt && cu.numel() == B + 1 && lens.scalar_type() == at::kInt &&
                    lens.numel() == B && cu.is_cuda() && lens.is_cuda(),
                "mtlattn: cu_seqlens [B + 1] and lens [B] must be int32 GPU tensors");
    const c10::DeviceGuard guard(packed.device());
    auto pc = packed.contiguous();
    const auto H = pc.size(1), D = pc.size(2);
    auto out = at::empty({B, H, N, D}, pc.options());
    auto lc = lens.contiguous();
    auto cc = cu.contiguous();
    check_rc(mtlattn_unpack_padded(dtype_code(pc.scalar_type()), (int32_t)B, (int32_t)N, (int32_t)H, (int32_t)D,
                                   pc.data_ptr(), lc.data_ptr<int32_t>(), cc.data_ptr<int32_t>(), out.data_ptr(),
                                   out.stride(0), out.stride(1), out.stride(2), current_stream(pc)));
    return out;
}

bool mpp_available() { return true; }

int64_t gpu_core_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    return mtlattn_gpu_core_count(dev);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("mpp_available", &mpp_available, "True: the MFMA fast path is compiled in for gfx950");
    m.def("pack_padded", &pack_padded, "SDPA key-padding adapter: dense [B,H,N,D] -> packed rows + cu_seqlens",
          py::arg("x"), py::arg("lens"));
    m.def("unpack_padded", &unpack_padded, "Inverse of pack_padded (zeros for padded tokens)", py::arg("packed"),
          py::arg("cu_seqlens"), py::arg("lens"), py::arg("B"), py::arg("N"));
    m.def("gpu_core_count", &gpu_core_count, "Compute-unit count of the current device (0 if unknown)");
    m.def("abi_version", [] { return mtlattn_abi_version(); }, "C ABI version of libmtlattn_hip.so");
    m.def("attn_splitkv", &attn_splitkv, "split-KV decode with an explicit split count (test entry)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("cu_q"), py::arg("cu_kv"), py::arg("max_seqlen_q"), py::arg("scale"),
          py::arg("causal"), py::arg("num_splits"), py::arg("window") = 0, py::arg("attn_bias") = c10::nullopt);
    m.def("paged_decode", &paged_decode, "decode (max_seqlen_q <= 16) over a paged KV cache", py::arg("q"),
          py::arg("k_cache"), py::arg("v_cache"), py::arg("cu_seqlens_q"), py::arg("cu_seqlens_kv"),
          py::arg("block_table"), py::arg("max_seqlen_q"), py::arg("max_seqlen_kv"), py::arg("scale"),
          py::arg("causal") = false, py::arg("window") = 0, py::arg("lse_out") = c10::nullopt,
          py::arg("attn_bias") = c10::nullopt);
    m.def("mpp_bwd_dkv", &mpp_bwd_dkv, "dK/dV backward kernel, fp32 outputs (test entry)", py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("dO"), py::arg("lse"), py::arg("delta"), py::arg("cu_q"), py::arg("cu_kv"),
          py::arg("max_seqlen_kv"), py::arg("scale"), py::arg("causal") = false, py::arg("window") = 0,
          py::arg("attn_bias") = c10::nullopt);
    m.def("mpp_bwd_dq", &mpp_bwd_dq, "dQ backward kernel, fp32 output (test entry)", py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("dO"), py::arg("lse"), py::arg("delta"), py::arg("cu_q"), py::arg("cu_kv"),
          py::arg("max_seqlen_q"), py::arg("scale"), py::arg("causal") = false, py::arg("window") = 0,
          py::arg("attn_bias") = c10::nullopt);
    m.def("varlen_attention", &varlen_attention, "Fused varlen attention forward (MI355X)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("cu_seqlens_q"), py::arg("cu_seqlens_kv"), py::arg("max_seqlen_q"),
          py::arg("scale"), py::arg("causal") = false, py::arg("window") = 0, py::arg("lse_out") = c10::nullopt,
          py::arg("attn_bias") = c10::nullopt);
    m.def("varlen_attention_bwd", &varlen_attention_bwd, "Varlen attention backward (dQ, dK, dV)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("o"), py::arg("dout"), py::arg("lse"), py::arg("cu_seqlens_q"),
          py::arg("cu_seqlens_kv"), py::arg("scale"), py::arg("causal") = false, py::arg("window") = 0,
          py::arg("attn_bias") = c10::nullopt);
}
