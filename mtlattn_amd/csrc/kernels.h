// Kernel parameter blocks and host-side launchers of the gfx950 kernels.
// Included by the kernel sources and by the C ABI (capi.hip); not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtlattn {

// Tensor geometry shared by every kernel (the scalar block of the reference's
// Params, src/ext.mm:44-57, with 64-bit row strides).
struct Geometry {
    const int* cu_q;
    const int* cu_kv;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, d;
    float scale;
    int causal, window;
    const float* bias;            // nullptr = no bias
    int64_t bias_qs, bias_hs, bias_cols;
    int64_t bias_ss = -1;         // >= 0: bias rows per sequence (bias_row_offset)
    int64_t bias_rows = 0;        // rows per sequence block when bias_ss >= 0
};

struct FwdArgs {
    Geometry geo;
    const void* q; int64_t q_rs;
    const void* k; int64_t k_rs;
    const void* v; int64_t v_rs;
    void* o;                      // contiguous [total_q, hq, d]
    float* lse;                   // nullable [total_q, hq]
    // fp32 matrix-core forward only: f32_splits > 1 splits each workgroup's
    // key tiles over that many workgroups, with normalised fp32 partials and
    // their LSEs in f32_part (f32_fwd_part_floats floats), then merged
    float* f32_part = nullptr;
    int f32_splits = 1;
};

struct BwdArgs {
    Geometry geo;
    const void* q; int64_t q_rs;
    const void* k; int64_t k_rs;
    const void* v; int64_t v_rs;
    const void* dout; int64_t do_rs;
    const float* lse;             // [total_q, hq]
    const float* delta;           // [total_q, hq]
    void* dq;                     // contiguous [total_q, hq, d]
    void* dk;                     // contiguous [total_kv, hkv, d]
    void* dv;
    int out_f32;                  // 1: dq/dk/dv are fp32, 0: input dtype
    // dQ only: with delta_out set, the dQ kernel computes delta = rowsum(dO * O)
    // itself from o (the forward's output) and writes it to delta_out for the
    // dK/dV kernel, in place of the separate preprocess (head dims 64 and 128)
    const void* o = nullptr; int64_t o_rs = 0;
    float* delta_out = nullptr;
    // fp32 matrix-core dQ and dK/dV only: f32_splits > 1 splits each
    // workgroup's work over that many workgroups, with fp32 partials in
    // f32_part (f32_dq_part_floats / f32_dkv_part_floats floats) summed in a
    // fixed order afterwards; dQ also takes o / delta_out (delta in-kernel)
    float* f32_part = nullptr;
    int f32_splits = 1;
};

struct DecodeArgs {
    Geometry geo;
    const void* q; int64_t q_rs;
    const void* k; int64_t k_rs;
    const void* v; int64_t v_rs;
    void* o;                      // contiguous [total_q, hq, d]
    float* lse;                   // nullable
    float* o_part;                // [hkv * head groups * slots * 16, d] (decode_workspace_rows)
    float* lse_part;              // [hkv * head groups * slots * 16]
    int num_splits;               // equal splits per sequence (used when chunk == 0)
    int chunk;                    // > 0: fixed KV chunk length (multiple of 32)
    int max_q;                    // bound on q lengths; heads_per_group * max_q <= 16
    // paged KV: k / v are caches [num_pages, page_size, hkv, d] (row strides
    // k_rs / v_rs per token), logical key j of sequence s in page
    // block_table[s * bt_stride + j / page_size]; block_table == nullptr:
    // contiguous K/V by cu_seqlens_kv
    const int* block_table = nullptr;
    int64_t bt_stride = 0;
    int page_size = 0, num_pages = 0;
};

// Launchers return hipSuccess or the launch error. `dtype` is MTLATTN_DTYPE_*.
hipError_t launch_fwd_mfma(int dtype, const FwdArgs& a, hipStream_t st);
hipError_t launch_fwd_generic(int dtype, const FwdArgs& a, hipStream_t st);
hipError_t launch_bwd_preprocess(int dtype, const Geometry& geo, const void* o, int64_t o_rs,
                                 const void* dout, int64_t do_rs, float* delta, hipStream_t st);
hipError_t launch_bwd_dq_mfma(int dtype, const BwdArgs& a, hipStream_t st);
hipError_t launch_bwd_dkv_mfma(int dtype, const BwdArgs& a, hipStream_t st);
// dK/dV without a bias at head dims 80-128, one wave per SIMD (bwd_wide.hip);
// hipErrorNotSupported when the problem is not for it. type_code: BF16::code / F16::code.
hipError_t launch_bwd_dkv_wide(int type_code, const BwdArgs& a, hipStream_t st);
hipError_t launch_bwd_dq_generic(int dtype, const BwdArgs& a, hipStream_t st);
hipError_t launch_bwd_dkv_generic(int dtype, const BwdArgs& a, hipStream_t st);
// fp32 inputs on the fp32 matrix cores (f32_mfma_head_dim, 16-byte aligned
// rows and outputs); dq / dk / dv are written as fp32
hipError_t launch_fwd_f32mfma(const FwdArgs& a, hipStream_t st);
hipError_t launch_bwd_dq_f32mfma(const BwdArgs& a, hipStream_t st);
hipError_t launch_bwd_dkv_f32mfma(const BwdArgs& a, hipStream_t st);
// Rows of a [total_rows, row_bytes] tensor outside [cu[0], cu[num_seqs]).
struct ZeroFill {
    void* ptr;
    int64_t row_bytes, total_rows;
    const int* cu;
};
// Zeroes those rows of up to three tensors in one launch.
hipError_t launch_zero_outside(const ZeroFill* fills, int n, int num_seqs, hipStream_t st);
hipError_t launch_decode(int dtype, const DecodeArgs& a, hipStream_t st);
hipError_t launch_pad_pack(int esize, int B, int N, int H, int D, const void* src, int64_t sb, int64_t sh,
                           int64_t sn, const int* lens, int* cu, void* dst, hipStream_t st);
hipError_t launch_pad_unpack(int esize, int B, int N, int H, int D, const void* src, const int* lens, const int* cu,
                             void* dst, int64_t sb, int64_t sh, int64_t sn, hipStream_t st);

// Partial rows of the split-KV workspace (fp32 O rows of D values plus one
// LSE each): kv heads x head groups x work-item slots x 16.
inline int64_t decode_workspace_rows(int64_t total_kv, int num_seqs, int hkv, int n_hg, int chunk, int ns) {
    const int64_t slots = chunk > 0 ? total_kv / chunk + num_seqs + 1 : (int64_t)num_seqs * ns;
    return (int64_t)hkv * n_hg * slots * 16;
}

// Which head dims have MFMA kernels.
// head dims of the matrix-core flash kernels (fp16/bf16): 64 and 128 native,
// 80, 88, 96 on the 128-wide tile with the spare columns unused, 160 and 256
// on 256-wide tiles with the output columns produced in slices
inline bool mfma_head_dim(int d) {
    return d == 64 || d == 80 || d == 88 || d == 96 || d == 128 || d == 160 || d == 256;
}
// head dims of the fp32 matrix-core kernels (columns padded to a multiple
// of 32 with zeros)
inline bool f32_mfma_head_dim(int d) { return d > 0 && d <= 128 && d % 4 == 0; }
// grid x of the fp32 matrix-core kernels: 128-row tiles over every sequence
inline int64_t f32_row_tiles(int64_t total_rows, int num_seqs) { return total_rows / 128 + num_seqs + 1; }
inline int64_t f32_fwd_part_floats(int splits, int64_t total_q, int hq, int d) {
    return splits > 1 ? (int64_t)splits * total_q * hq * (d + 1) : 0;
}
inline int64_t f32_dq_part_floats(int splits, int64_t total_q, int hq, int d) {
    return splits > 1 ? (int64_t)splits * total_q * hq * d : 0;
}
inline int64_t f32_dkv_part_floats(int splits, int64_t total_kv, int hkv, int d) {
    return splits > 1 ? (int64_t)splits * 2 * total_kv * hkv * d : 0;
}
// head dims of the split-KV decode kernels
inline bool decode_head_dim(int d) { return d == 64 || d == 128; }

}  // namespace mtlattn
