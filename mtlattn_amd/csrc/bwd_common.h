// Kernel parameters and small helpers shared by the 16-bit backward kernels
// (bwd.hip, bwd_wide.hip).
#pragma once

#include "common.h"
#include "kernels.h"

namespace mtlattn {
namespace {

struct BwdKParams {
    const uint16_t* q; const uint16_t* k; const uint16_t* v; const uint16_t* dout;
    const float* lse; const float* delta;
    void* dq; void* dk; void* dv;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs, do_rs;
    int64_t bias_qs, bias_hs, bias_cols, bias_ss, bias_rows;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, hpw, n_tiles, n_hg;
    float scale, scale_log2;
    int causal, window;
    int bias_v4;      // bias rows 16-byte aligned (pointer and strides)
    int bias_b32;     // 64 bias rows plus a row's columns span < 2^32 bytes (32-bit buffer offsets)
    const uint16_t* o; int64_t o_rs;   // forward output (dQ with delta_w)
    float* delta_w;   // non-null: the dQ kernel computes delta and writes it here
};

// Sum of the 8 products of one 16-byte chunk of O and dO. The preprocess and
// the dQ kernel's fused delta both use it and combine chunks in the same tree,
// so the two give bitwise equal deltas.
template <typename T>
__device__ inline float dot8(const u32x4_t a, const u32x4_t b) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc += lo16<T>(a[e]) * lo16<T>(b[e]) + hi16<T>(a[e]) * hi16<T>(b[e]);
    return acc;
}

template <typename T, bool OUT_F32>
__device__ inline void store4(void* base, int64_t off, float a, float b, float c, float d) {
    if (OUT_F32) {
        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(base) + off) = f32x4_t{a, b, c, d};
    } else {
        st8(reinterpret_cast<uint16_t*>(base) + off, u32x2_t{T::pack2(a, b), T::pack2(c, d)});
    }
}

// Staged lse / delta columns as the dK/dV products use them: lse (which = 0)
// becomes -lse log2(e), with rows of no allowed key (lse = -inf) giving -inf
// so that every P of theirs is exp2(-inf) = 0; delta (which = 1) becomes -delta.
// First query tile (its first row) of a dK/dV workgroup's walk over the
// n tiles q_lo, q_lo + qtl, ... of its query range. The walk descends from
// there and, reaching q_lo, wraps to the top tile. Without a window it starts
// at the top tile: every workgroup of a sequence then reads the same (tile,
// head) at the same time from the top, and the L2 serves the repeats. Under
// a sliding window the ranges of neighbouring key blocks are shifted copies
// of equal length, so the walk starts at the tile whose index is a multiple
// of n: each tile X then comes at step (start - X) mod n in every workgroup
// whose range holds it, and co-resident workgroups again read it together.
__device__ inline int first_q_tile(int q_lo, int n, int qtl, bool cyclic) {
    if (!cyclic || n <= 0) return q_lo + (n - 1) * qtl;
    const int lo_t = q_lo / qtl;
    return q_lo + (n - lo_t % n) % n * qtl;
}

__device__ inline float neg_lse2(float v) { return v == kNegInf ? kNegInf : -v * kLog2e; }
__device__ inline void neg_col(float* x, int which) {
    const float v = *x;
    *x = which ? -v : neg_lse2(v);
}

BwdKParams make_params(const BwdArgs& a) {
    const Geometry& g = a.geo;
    BwdKParams p;
    p.q = (const uint16_t*)a.q; p.k = (const uint16_t*)a.k; p.v = (const uint16_t*)a.v;
    p.dout = (const uint16_t*)a.dout;
    p.lse = a.lse; p.delta = a.delta;
    p.dq = a.dq; p.dk = a.dk; p.dv = a.dv;
    p.cu_q = g.cu_q; p.cu_kv = g.cu_kv; p.bias = g.bias;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs; p.do_rs = a.do_rs;
    p.bias_qs = g.bias_qs; p.bias_hs = g.bias_hs; p.bias_cols = g.bias_cols;
    p.bias_ss = g.bias_ss; p.bias_rows = g.bias_rows;
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.hkv = g.hkv; p.g = g.g;
    p.hpw = 1;
    p.n_tiles = 0; p.n_hg = 0;
    p.scale = g.scale; p.scale_log2 = g.scale * kLog2e;
    p.causal = g.causal; p.window = g.window > 0 ? g.window : 0;
    p.bias_b32 = g.bias != nullptr && (64 * g.bias_qs + g.bias_cols) * 4 < ((int64_t)1 << 32);
    p.bias_v4 = g.bias != nullptr && ((uintptr_t)g.bias % 16 == 0) && g.bias_qs % 4 == 0 && g.bias_hs % 4 == 0 &&
                (g.bias_ss < 0 || g.bias_ss % 4 == 0);
    p.o = (const uint16_t*)a.o; p.o_rs = a.o_rs;
    p.delta_w = a.delta_out;
    return p;
}

}  // namespace
}  // namespace mtlattn
