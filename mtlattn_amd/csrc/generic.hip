// Portable VALU kernels for every dtype and head dim up to 256: the fp32 path
// (the reference runs fp32 on its simdgroup kernels, src/attention.metal:334,
// 863) and head dims without an MFMA kernel. fp32 throughout, no reduced
// precision for fp32 inputs.
//
//   forward  : one wave per (query row, head). Keys in chunks of 64, lane =
//              key for q.k (q row staged in LDS), online softmax with wave
//              reductions, then lane = d for the P.V accumulation
//              (src/attention.metal:44-289 states the same mathematics).
//   dQ       : one wave per (query row, head) (src/attention.metal:741-784).
//   dK / dV  : one wave per (key row, kv head), looping over the g query heads
//              of the group and the query rows that can see the key
//              (src/attention.metal:788-835), plus window bounds.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

constexpr int kGenWaves = 4;
constexpr int kMaxD = 256;

struct GenParams {
    const void* q; const void* k; const void* v; const void* dout;
    void* o; float* lse;
    const float* lse_in; const float* delta;
    void* dq; void* dk; void* dv;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs, do_rs;
    int64_t bias_qs, bias_hs, bias_cols, bias_ss, bias_rows;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, d;
    float scale;
    int causal, window;
    int out_f32;
};

// Sequence containing packed row `row` (largest s with cu[s] <= row), or -1.
__device__ inline int seq_of_row(const int* __restrict__ cu, int num_seqs, int64_t total, int64_t row) {
    int lo = 0, hi = num_seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (seq_range(cu, mid, total).start <= row) lo = mid; else hi = mid - 1;
    }
    const SeqRange r = seq_range(cu, lo, total);
    return (row >= r.start && row < r.end) ? lo : -1;
}

// exp for the softmax: exp_fp32 for fp32 inputs (the accuracy of the fp32
// path), the hardware exponential for 16-bit ones
template <typename T>
__device__ inline float sexp(float a) {
    if constexpr (std::is_same<T, F32>::value) return exp_fp32(a);
    else return __expf(a);
}

template <typename T>
__device__ inline float ldf(const void* base, int64_t idx) {
    return T::to_float(reinterpret_cast<const typename T::raw*>(base)[idx]);
}

template <typename T>
__device__ inline void stf(void* base, int64_t idx, float x) {
    reinterpret_cast<typename T::raw*>(base)[idx] = T::from_float(x);
}

// dot(row of LDS floats, global row of T) over d elements
template <typename T>
__device__ inline float dot_row(const float* __restrict__ a, const void* base, int64_t off, int d) {
    const typename T::raw* b = reinterpret_cast<const typename T::raw*>(base) + off;
    float acc = 0.f;
    for (int i = 0; i < d; ++i) acc = fmaf(a[i], T::to_float(b[i]), acc);
    return acc;
}

template <typename T>
__global__ __launch_bounds__(kGenWaves * 64) void gen_fwd_kernel(GenParams p) {
    __shared__ float qs[kGenWaves][kMaxD];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * kGenWaves + w;
    if (pair >= p.total_q * p.hq) return;
    const int64_t row = pair / p.hq;
    const int head = (int)(pair - row * p.hq);
    const int s = seq_of_row(p.cu_q, p.num_seqs, p.total_q, row);
    if (s < 0) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int i = (int)(row - qr.start);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int coff = kv_len - q_len;
    const int hk = head / p.g;
    for (int c = lane; c < p.d; c += 64) qs[w][c] = ldf<T>(p.q, row * p.q_rs + (int64_t)head * p.d + c);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    const int hi = p.causal ? min(kv_len, i + coff + 1) : kv_len;
    const int lo = p.window > 0 ? max(0, i + coff - p.window + 1) : 0;
    const float* brow =
        p.bias ? p.bias + bias_row_offset(row, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) + (int64_t)head * p.bias_hs
               : nullptr;
    float m = kNegInf, l = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int kt = lo; kt < hi; kt += 64) {
        const int j = kt + lane;
        float x = kNegInf;
        if (j < hi) {
            x = dot_row<T>(qs[w], p.k, (int64_t)(kr.start + j) * p.k_rs + (int64_t)hk * p.d, p.d) * p.scale;
            if (brow != nullptr && j < p.bias_cols) x += brow[j];
        }
        const float mt = wave_max(x);
        const float mn = fmaxf(m, mt);
        const float mu = mn == kNegInf ? 0.f : mn;
        const float corr = sexp<T>(m - mu);
        const float pj = x == kNegInf ? 0.f : sexp<T>(x - mu);
        l = l * corr + wave_sum(pj);
        m = mn;
        // the chunk's P.V from zero, folded in with the rescale (one rounding
        // of the running sum per 64 keys instead of one per key)
        float part[4] = {0.f, 0.f, 0.f, 0.f};
        const int n = min(64, hi - kt);
        for (int jj = 0; jj < n; ++jj) {
            const float pw = __shfl(pj, jj);
            if (pw == 0.f) continue;
            const int64_t vo = (int64_t)(kr.start + kt + jj) * p.v_rs + (int64_t)hk * p.d;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int dd = lane + 64 * c;
                if (dd < p.d) part[c] = fmaf(pw, ldf<T>(p.v, vo + dd), part[c]);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fmaf(acc[c], corr, part[c]);
    }
    const float inv = !(l <= 0.f) ? 1.f / l : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int dd = lane + 64 * c;
        if (dd < p.d) stf<T>(p.o, (row * p.hq + head) * p.d + dd, acc[c] * inv);
    }
    if (p.lse != nullptr && lane == 0) p.lse[row * p.hq + head] = !(l <= 0.f) ? m + logf(l) : kNegInf;
}

template <typename T>
__global__ __launch_bounds__(kGenWaves * 64) void gen_dq_kernel(GenParams p) {
    __shared__ float qs[kGenWaves][kMaxD];
    __shared__ float ds_[kGenWaves][kMaxD];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * kGenWaves + w;
    if (pair >= p.total_q * p.hq) return;
    const int64_t row = pair / p.hq;
    const int head = (int)(pair - row * p.hq);
    const int s = seq_of_row(p.cu_q, p.num_seqs, p.total_q, row);
    if (s < 0) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int i = (int)(row - qr.start);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int coff = kv_len - q_len;
    const int hk = head / p.g;
    for (int c = lane; c < p.d; c += 64) {
        qs[w][c] = ldf<T>(p.q, row * p.q_rs + (int64_t)head * p.d + c);
        ds_[w][c] = ldf<T>(p.dout, row * p.do_rs + (int64_t)head * p.d + c);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    const float lse = p.lse_in[row * p.hq + head];
    const float dlt = p.delta[row * p.hq + head];
    const int hi = p.causal ? min(kv_len, i + coff + 1) : kv_len;
    const int lo = p.window > 0 ? max(0, i + coff - p.window + 1) : 0;
    const float* brow =
        p.bias ? p.bias + bias_row_offset(row, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) + (int64_t)head * p.bias_hs
               : nullptr;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (lse != kNegInf) {
        for (int kt = lo; kt < hi; kt += 64) {
            const int j = kt + lane;
            float dsj = 0.f;
            if (j < hi) {
                const int64_t ko = (int64_t)(kr.start + j) * p.k_rs + (int64_t)hk * p.d;
                const int64_t vo = (int64_t)(kr.start + j) * p.v_rs + (int64_t)hk * p.d;
                float x = dot_row<T>(qs[w], p.k, ko, p.d) * p.scale;
                if (brow != nullptr && j < p.bias_cols) x += brow[j];
                const float pj = sexp<T>(x - lse);
                const float dp = dot_row<T>(ds_[w], p.v, vo, p.d);
                dsj = pj * (dp - dlt);
            }
            const int n = min(64, hi - kt);
            float part[4] = {0.f, 0.f, 0.f, 0.f};   // this chunk's dS.K, added once per 64 keys
            for (int jj = 0; jj < n; ++jj) {
                const float sw = __shfl(dsj, jj);
                if (sw == 0.f) continue;
                const int64_t ko = (int64_t)(kr.start + kt + jj) * p.k_rs + (int64_t)hk * p.d;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int dd = lane + 64 * c;
                    if (dd < p.d) part[c] = fmaf(sw, ldf<T>(p.k, ko + dd), part[c]);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] += part[c];
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int dd = lane + 64 * c;
        if (dd >= p.d) continue;
        const int64_t o = (row * p.hq + head) * p.d + dd;
        if (p.out_f32) reinterpret_cast<float*>(p.dq)[o] = acc[c] * p.scale;
        else stf<T>(p.dq, o, acc[c] * p.scale);
    }
}

template <typename T>
__global__ __launch_bounds__(kGenWaves * 64) void gen_dkv_kernel(GenParams p) {
    __shared__ float ks_[kGenWaves][kMaxD];
    __shared__ float vs_[kGenWaves][kMaxD];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * kGenWaves + w;
    if (pair >= p.total_kv * p.hkv) return;
    const int64_t krow = pair / p.hkv;
    const int hk = (int)(pair - krow * p.hkv);
    const int s = seq_of_row(p.cu_kv, p.num_seqs, p.total_kv, krow);
    if (s < 0) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int j = (int)(krow - kr.start);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int coff = kv_len - q_len;
    for (int c = lane; c < p.d; c += 64) {
        ks_[w][c] = ldf<T>(p.k, krow * p.k_rs + (int64_t)hk * p.d + c);
        vs_[w][c] = ldf<T>(p.v, krow * p.v_rs + (int64_t)hk * p.d + c);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // queries i that see key j: causal i >= j - coff; window i <= j - coff + W - 1
    const int lo = p.causal ? max(0, j - coff) : 0;
    const int hi = p.window > 0 ? min(q_len, j - coff + p.window) : q_len;
    float dka[4] = {0.f, 0.f, 0.f, 0.f}, dva[4] = {0.f, 0.f, 0.f, 0.f};
    for (int hh = 0; hh < p.g; ++hh) {
        const int head = hk * p.g + hh;
        for (int qt = lo; qt < hi; qt += 64) {
            const int i = qt + lane;
            float pi = 0.f, dsi = 0.f;
            if (i < hi) {
                const int64_t row = qr.start + i;
                const float lse = p.lse_in[row * p.hq + head];
                if (lse != kNegInf) {
                    float x = dot_row<T>(ks_[w], p.q, row * p.q_rs + (int64_t)head * p.d, p.d) * p.scale;
                    if (p.bias != nullptr && j < p.bias_cols)
                        x += p.bias[bias_row_offset(row, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) +
                                    (int64_t)head * p.bias_hs + j];
                    pi = sexp<T>(x - lse);
                    const float dp = dot_row<T>(vs_[w], p.dout, row * p.do_rs + (int64_t)head * p.d, p.d);
                    dsi = pi * (dp - p.delta[row * p.hq + head]);
                }
            }
            const int n = min(64, hi - qt);
            // this chunk's P^T.dO and dS^T.Q, added once per 64 queries
            float pk[4] = {0.f, 0.f, 0.f, 0.f}, pv[4] = {0.f, 0.f, 0.f, 0.f};
            for (int ii = 0; ii < n; ++ii) {
                const float pw = __shfl(pi, ii), sw = __shfl(dsi, ii);
                if (pw == 0.f && sw == 0.f) continue;
                const int64_t row = qr.start + qt + ii;
                const int64_t qo = row * p.q_rs + (int64_t)head * p.d;
                const int64_t oo = row * p.do_rs + (int64_t)head * p.d;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int dd = lane + 64 * c;
                    if (dd < p.d) {
                        pv[c] = fmaf(pw, ldf<T>(p.dout, oo + dd), pv[c]);
                        pk[c] = fmaf(sw, ldf<T>(p.q, qo + dd), pk[c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dva[c] += pv[c];
                dka[c] += pk[c];
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int dd = lane + 64 * c;
        if (dd >= p.d) continue;
        const int64_t o = (krow * p.hkv + hk) * p.d + dd;
        if (p.out_f32) {
            reinterpret_cast<float*>(p.dk)[o] = dka[c] * p.scale;
            reinterpret_cast<float*>(p.dv)[o] = dva[c];
        } else {
            stf<T>(p.dk, o, dka[c] * p.scale);
            stf<T>(p.dv, o, dva[c]);
        }
    }
}

GenParams make_gen(const Geometry& g) {
    GenParams p{};
    p.cu_q = g.cu_q; p.cu_kv = g.cu_kv; p.bias = g.bias;
    p.bias_qs = g.bias_qs; p.bias_hs = g.bias_hs; p.bias_cols = g.bias_cols;
    p.bias_ss = g.bias_ss; p.bias_rows = g.bias_rows;
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.hkv = g.hkv; p.g = g.g; p.d = g.d;
    p.scale = g.scale; p.causal = g.causal; p.window = g.window > 0 ? g.window : 0;
    return p;
}

using GenKernel = void (*)(GenParams);

hipError_t dispatch(int dtype, const GenParams& p, int64_t pairs, hipStream_t st, GenKernel kbf16,
                    GenKernel kf16, GenKernel kf32) {
    if (pairs <= 0) return hipSuccess;
    const int64_t blocks = (pairs + kGenWaves - 1) / kGenWaves;
    if (blocks > 0x7fffffff || p.d > kMaxD) return hipErrorInvalidValue;
    const GenKernel k = dtype == MTLATTN_DTYPE_BF16 ? kbf16 : dtype == MTLATTN_DTYPE_F16 ? kf16 : kf32;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(kGenWaves * 64), 0, st, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_generic(int dtype, const FwdArgs& a, hipStream_t st) {
    GenParams p = make_gen(a.geo);
    p.q = a.q; p.k = a.k; p.v = a.v; p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs;
    p.o = a.o; p.lse = a.lse;
    return dispatch(dtype, p, a.geo.total_q * a.geo.hq, st, gen_fwd_kernel<BF16>, gen_fwd_kernel<F16>,
                    gen_fwd_kernel<F32>);
}

hipError_t launch_bwd_dq_generic(int dtype, const BwdArgs& a, hipStream_t st) {
    GenParams p = make_gen(a.geo);
    p.q = a.q; p.k = a.k; p.v = a.v; p.dout = a.dout;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs; p.do_rs = a.do_rs;
    p.lse_in = a.lse; p.delta = a.delta; p.dq = a.dq; p.out_f32 = a.out_f32;
    return dispatch(dtype, p, a.geo.total_q * a.geo.hq, st, gen_dq_kernel<BF16>, gen_dq_kernel<F16>,
                    gen_dq_kernel<F32>);
}

hipError_t launch_bwd_dkv_generic(int dtype, const BwdArgs& a, hipStream_t st) {
    GenParams p = make_gen(a.geo);
    p.q = a.q; p.k = a.k; p.v = a.v; p.dout = a.dout;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs; p.do_rs = a.do_rs;
    p.lse_in = a.lse; p.delta = a.delta; p.dk = a.dk; p.dv = a.dv; p.out_f32 = a.out_f32;
    return dispatch(dtype, p, a.geo.total_kv * a.geo.hkv, st, gen_dkv_kernel<BF16>, gen_dkv_kernel<F16>,
                    gen_dkv_kernel<F32>);
}

}  // namespace mtlattn
