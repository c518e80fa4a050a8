// Backward for fp16/bf16 on gfx950 MFMA: the delta preprocess, a dQ kernel
// and a dK/dV kernel (counterparts of the reference's bwd_dq_mpp /
// bwd_dkv_mpp, src/attn_mpp.metal:546-799, and the delta reduction at
// src/ext.mm:518). No atomics anywhere: every output element is written by
// exactly one lane, so results are bitwise run-to-run deterministic.
//
// Shared mathematics (src/attention.metal:707-717):
//   P = exp(scale q.k + bias - lse), dP = dO.v, dS = P (dP - delta),
//   dQ = scale dS K, dK = scale dS^T Q (summed over the GQA group), dV = P^T dO.
// P and dS are rounded to the input type before the second products, as the
// forward rounds P before P.V.
//
// dQ kernel: workgroup of 8 waves, 32 query rows x 1 head per wave, GQA heads
//   packed like the forward. Per 64-key tile staged in LDS (K row-major, V
//   row-major, K^T): S^T = K Q^T and dP^T = V dO^T (C layout: lane = query),
//   dS^T in registers, dQ^T += K^T dS^T.
// dK/dV kernel: workgroup of 8 waves, 32 keys per wave (256 keys of one kv
//   head). Loops over the g query heads of the group and over 64-query tiles
//   staged in LDS (Q, Q^T, dO, dO^T, lse, delta): S = Q K^T and dP = dO V^T
//   (C layout: lane = key), dV^T += dO^T P, dK^T += Q^T dS. Causal and window
//   bands skip whole query tiles (the reference skips causal only,
//   src/attn_mpp.metal:591).
#include "common.h"
#include "kernels.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kKT = 64;   // dQ: keys per tile
constexpr int kQT = 64;   // dK/dV: queries per tile
constexpr int kKW = 32;   // dK/dV: keys per wave

struct BwdKParams {
    const uint16_t* q; const uint16_t* k; const uint16_t* v; const uint16_t* dout;
    const float* lse; const float* delta;
    void* dq; void* dk; void* dv;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs, do_rs;
    int64_t bias_qs, bias_hs, bias_cols;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, hpw, n_tiles, n_hg;
    float scale, scale_log2;
    int causal, window;
};

__device__ inline bool allowed(int qrow, int key, int coff, int kv_len, int causal, int window) {
    bool ok = key < kv_len;
    if (causal) ok = ok && key <= qrow + coff;
    if (window > 0) ok = ok && key > qrow + coff - window;
    return ok;
}

template <typename T, bool OUT_F32>
__device__ inline void store4(void* base, int64_t off, float a, float b, float c, float d) {
    if (OUT_F32) {
        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(base) + off) = f32x4_t{a, b, c, d};
    } else {
        st8(reinterpret_cast<uint16_t*>(base) + off, u32x2_t{T::pack2(a, b), T::pack2(c, d)});
    }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
// 8 waves at D = 64; 4 waves (one per SIMD, 512-register budget) at D = 128.
template <int D> struct DqCfg { static constexpr int NW = D >= 128 ? 4 : 8; };

template <typename T, int D, bool BIAS, bool OUT_F32>
__global__ __launch_bounds__(DqCfg<D>::NW * 64, 1) void bwd_dq_kernel(BwdKParams p) {
    constexpr int NW = DqCfg<D>::NW;
    constexpr int HALF = NW * 32;             // loader threads per role
    constexpr int DC = D / 16, DB = D / 32;
    constexpr int TILE_BYTES = kKT * D * 2;
    constexpr int STAGE = 3 * TILE_BYTES;     // K, V (row-major), K^T
    constexpr int KUNITS = 2 * D;             // (4 keys x 8 d) units
    constexpr int KUPT = (KUNITS + HALF - 1) / HALF;   // K units per loader thread
    constexpr int VCH = kKT * D / 8 / HALF;   // 16-byte V chunks per loader thread
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const int QT = 32 * (NW / p.hpw);
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.n_hg);
    const int hg = L / p.n_tiles;
    const int t = p.n_tiles - 1 - (L - hg * p.n_tiles);
    const int s = find_seq_for_tile(p.cu_q, p.num_seqs, QT, t, p.total_q);
    const int tb = tile_base(p.cu_q, s, QT, p.total_q);
    if (t < tb) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int q0 = (t - tb) * QT;
    if (q0 >= q_len) return;

    const int wph = NW / p.hpw;
    const int head = hg * p.hpw + w / wph;
    const int hk = head / p.g;
    const int qa = q0 + 32 * (w % wph);
    const int coff = kv_len - q_len;
    const bool wave_active = qa < q_len;
    const int wq_last = min(q_len, qa + 32) - 1;
    const int qrow = qa + l32;
    const bool row_ok = qrow < q_len;
    // rows past the sequence end read its last row (finite, never stored)
    const int64_t grow = qr.start + min(qrow, q_len - 1);

    // B operands: Q^T and dO^T fragments (lane = query, d = 16 kc + 8 hi + j).
    u32x4_t qf[DC], df[DC];
    {
        const uint16_t* qp = p.q + grow * p.q_rs + (int64_t)head * D + 8 * hi;
        const uint16_t* dp = p.dout + grow * p.do_rs + (int64_t)head * D + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc) {
            qf[kc] = ld16(qp + 16 * kc);
            df[kc] = ld16(dp + 16 * kc);
        }
    }
    float lse2 = kPosInf, dlt = 0.f;
    if (row_ok) {
        const float l = p.lse[grow * p.hq + head];
        lse2 = l == kNegInf ? kPosInf : l * kLog2e;   // empty rows: P = 0
        dlt = p.delta[grow * p.hq + head];
    }
    const float* brow = nullptr;
    if (BIAS && row_ok) brow = p.bias + grow * p.bias_qs + (int64_t)head * p.bias_hs;

    const int q_last_wg = min(q_len, q0 + QT) - 1;
    const int kv_hi = p.causal ? min(kv_len, q_last_wg + coff + 1) : kv_len;
    int kv_lo = 0;
    if (p.window > 0) {
        kv_lo = max(0, q0 + coff - p.window + 1);
        kv_lo = (kv_lo / kKT) * kKT;
    }
    const int n_kv_tiles = kv_hi > kv_lo ? (kv_hi - kv_lo + kKT - 1) / kKT : 0;
    const uint16_t* kbase = p.k + (int64_t)kr.start * p.k_rs + (int64_t)hk * D;
    const uint16_t* vbase = p.v + (int64_t)kr.start * p.v_rs + (int64_t)hk * D;

    // Loader roles: the first half of the threads stage K (row-major and
    // transposed), the second half V (row-major).
    const bool role_k = w < NW / 2;               // wave-uniform roles
    const int rt = role_k ? tid : tid - HALF;
    const int rt0 = role_k ? 64 * w : 64 * w - HALF;  // rt of lane 0 (unit counts are multiples of 64)
    constexpr int NPRE = KUPT * 4 > VCH ? KUPT * 4 : VCH;
    u32x4_t pre[NPRE];
    auto load_tile = [&](int kt) {
        if (role_k) {
#pragma unroll
            for (int uu = 0; uu < KUPT; ++uu) {
                const int u = rt + HALF * uu;
                if (rt0 + HALF * uu < KUNITS) {
                    const int dc = u % (D / 8), kg = u / (D / 8);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = min(kt + 4 * kg + i, kv_len - 1);   // masked past the end
                        pre[4 * uu + i] = ld16(kbase + (int64_t)key * p.k_rs + 8 * dc);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const int cid = rt + HALF * i;
                const int key = min(kt + cid / (D / 8), kv_len - 1);
                pre[i] = ld16(vbase + (int64_t)key * p.v_rs + 8 * (cid % (D / 8)));
            }
        }
    };
    auto store_tile = [&](int buf) {
        char* Ks = smem + buf * STAGE;
        char* Vs = Ks + TILE_BYTES;
        char* Kt = Vs + TILE_BYTES;
        if (role_k) {
#pragma unroll
            for (int uu = 0; uu < KUPT; ++uu) {
                const int u = rt + HALF * uu;
                if (rt0 + HALF * uu < KUNITS) {
                    const int dc = u % (D / 8), kg = u / (D / 8);
#pragma unroll
                    for (int i = 0; i < 4; ++i) st16(Ks + rm_offset<D>(4 * kg + i, dc), pre[4 * uu + i]);
                    u32x2_t tr[8];
                    transpose4x8(&pre[4 * uu], tr);
#pragma unroll
                    for (int i = 0; i < 8; ++i) st8(Kt + tr_store_offset(8 * dc + i, kg), tr[i]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const int cid = rt + HALF * i;
                st16(Vs + rm_offset<D>(cid / (D / 8), cid % (D / 8)), pre[i]);
            }
        }
    };

    // Per-lane LDS read offsets (see the forward kernel): row-major operands
    // for rows 32 kb + l32, transposed K^T operands for rows 32 db + l32.
    uint32_t rofs[4], tofs[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        rofs[c] = rm_offset<D>(l32, 2 * c + hi);
        tofs[c] = tr_load_offset(l32, c, hi);
    }

    f32x16_t dqacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) dqacc[db] = f32x16_t{};

    if (n_kv_tiles > 0) {
        load_tile(kv_lo);
        store_tile(0);
        __syncthreads();
        for (int it = 0; it < n_kv_tiles; ++it) {
            const int kt = kv_lo + it * kKT;
            const bool has_next = it + 1 < n_kv_tiles;
            if (has_next) load_tile(kt + kKT);

            bool skip = !wave_active;
            if (p.causal && kt > wq_last + coff) skip = true;
            if (p.window > 0 && kt + kKT - 1 < qa + coff - p.window + 1) skip = true;
            if (!skip) {
                const char* Ks = smem + (it & 1) * STAGE;
                const char* Vs = Ks + TILE_BYTES;
                const char* Kt = Vs + TILE_BYTES;
                const bool need_mask = (kt + kKT > kv_len) || (p.causal && kt + kKT - 1 > qa + coff) ||
                                       (p.window > 0 && kt < wq_last + coff - p.window + 1);
                // Two independent 32-key halves: P = exp(S - lse) needs no running max.
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    f32x16_t sacc = f32x16_t{}, pacc = f32x16_t{};
#pragma unroll
                    for (int kc = 0; kc < DC; ++kc) {
                        const uint32_t o = rofs[kc & 3] + (kc >> 2) * 128 + kb * 32 * 2 * D;
                        sacc = mfma32<T>(ld16(Ks + o), qf[kc], sacc);
                        pacc = mfma32<T>(ld16(Vs + o), df[kc], pacc);
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kt + 32 * kb + 8 * (r >> 2) + 4 * hi + (r & 3);
                        const bool ok = !need_mask || allowed(qrow, key, coff, kv_len, p.causal, p.window);
                        float x = sacc[r] * p.scale_log2;
                        if (BIAS && ok && brow != nullptr && key < p.bias_cols) x += brow[key] * kLog2e;
                        const float pr = ok ? __builtin_amdgcn_exp2f(x - lse2) : 0.f;
                        sacc[r] = pr * (pacc[r] - dlt);        // dS^T
                    }
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) {
                        const int c = 2 * kb + cc, r0 = 8 * cc;
                        const u32x4_t bs = u32x4_t{T::pack2(sacc[r0 + 0], sacc[r0 + 1]),
                                                   T::pack2(sacc[r0 + 2], sacc[r0 + 3]),
                                                   T::pack2(sacc[r0 + 4], sacc[r0 + 5]),
                                                   T::pack2(sacc[r0 + 6], sacc[r0 + 7])};
#pragma unroll
                        for (int db = 0; db < DB; ++db) {
                            const u32x4_t a = ld16(Kt + tofs[c ^ (2 * (db & 1))] + db * 32 * 128);
                            dqacc[db] = mfma32<T>(a, bs, dqacc[db]);
                        }
                    }
                }
            }
            if (has_next) store_tile((it + 1) & 1);
            __syncthreads();
        }
    }

    if (wave_active && row_ok) {
        const int64_t off = grow * ((int64_t)p.hq * D) + (int64_t)head * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                store4<T, OUT_F32>(p.dq, off + d, dqacc[db][4 * rg] * p.scale, dqacc[db][4 * rg + 1] * p.scale,
                                   dqacc[db][4 * rg + 2] * p.scale, dqacc[db][4 * rg + 3] * p.scale);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK / dV.  NW waves of 32 keys each: 8 waves at D = 64; at D = 128 the
// per-wave state (K, V operands + two D x 32 fp32 accumulators) needs the
// full 512-register budget, so 4 waves (one per SIMD).
// ---------------------------------------------------------------------------
template <int D> struct DkvCfg { static constexpr int NW = D >= 128 ? 4 : 8; };

template <typename T, int D, bool BIAS, bool OUT_F32>
__global__ __launch_bounds__(DkvCfg<D>::NW * 64, 1) void bwd_dkv_kernel(BwdKParams p) {
    constexpr int NW = DkvCfg<D>::NW;
    constexpr int NT = NW * 64;
    constexpr int HALF = NT / 2;                           // loader threads per role
    constexpr int DC = D / 16, DB = D / 32;
    constexpr int TILE_BYTES = kQT * D * 2;
    constexpr int STAGE = 4 * TILE_BYTES + 2 * kQT * 4;  // Q, Q^T, dO, dO^T, lse2, delta
    constexpr int UNITS = 2 * D;                           // (4 rows x 8 d) units per tile
    constexpr int UPT = (UNITS + HALF - 1) / HALF;         // units per loader thread
    constexpr int KB = NW * kKW;                           // keys per workgroup
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.hkv);
    const int hk = L / p.n_tiles;
    const int t = L - hk * p.n_tiles;                      // early key blocks (heavier when causal) first
    const int s = find_seq_for_tile(p.cu_kv, p.num_seqs, KB, t, p.total_kv);
    const int tb = tile_base(p.cu_kv, s, KB, p.total_kv);
    if (t < tb) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int k0 = (t - tb) * KB;
    if (k0 >= kv_len) return;
    const int coff = kv_len - q_len;

    const int kw = k0 + kKW * w;                 // first key of this wave (seq-local)
    const bool wave_active = kw < kv_len;
    const int wk_last = min(kv_len, kw + kKW) - 1;
    const int key = kw + l32;                    // this lane's key column
    const bool key_ok = key < kv_len;

    // K^T / V^T B operands: lane = key, d = 16 kc + 8 hi + j.
    u32x4_t kf[DC], vf[DC];
    {
        const int64_t grow = kr.start + min(key, kv_len - 1);     // masked past the end
        const uint16_t* kp = p.k + grow * p.k_rs + (int64_t)hk * D + 8 * hi;
        const uint16_t* vp = p.v + grow * p.v_rs + (int64_t)hk * D + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc) {
            kf[kc] = ld16(kp + 16 * kc);
            vf[kc] = ld16(vp + 16 * kc);
        }
    }

    // Query range that can see any key of this workgroup.
    const int k_last_wg = min(kv_len, k0 + KB) - 1;
    const int q_lo = p.causal ? max(0, k0 - coff) : 0;
    const int q_hi = p.window > 0 ? min(q_len, k_last_wg - coff + p.window) : q_len;
    const int n_q_tiles = q_hi > q_lo ? (q_hi - q_lo + kQT - 1) / kQT : 0;
    const int n_stages = n_q_tiles * p.g;

    // Loader roles: the first half of the threads stage Q (row-major +
    // transposed) and lse, the second half dO (row-major + transposed) and delta.
    const bool role_q = w < NW / 2;               // wave-uniform roles
    const int rt = role_q ? tid : tid - HALF;
    const int rt0 = role_q ? 64 * w : 64 * w - HALF;  // rt of lane 0 (unit counts are multiples of 64)
    u32x4_t pre[UPT][4];
    float pre_s = 0.f;
    auto load_stage = [&](int st) {
        const int h = hk * p.g + st / n_q_tiles;
        const int qt = q_lo + (st % n_q_tiles) * kQT;
        const uint16_t* base = role_q ? p.q : p.dout;
        const int64_t rs = role_q ? p.q_rs : p.do_rs;
#pragma unroll
        for (int uu = 0; uu < UPT; ++uu) {
            const int u = rt + HALF * uu;
            if (rt0 + HALF * uu < UNITS) {
                const int dc = u % (D / 8), qg = u / (D / 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // rows past the end read the last row; their lse is +inf, so P = dS = 0
                    const int q = min(qt + 4 * qg + i, q_len - 1);
                    pre[uu][i] = ld16(base + (int64_t)(qr.start + q) * rs + (int64_t)h * D + 8 * dc);
                }
            }
        }
        if (rt0 == 0) {                          // first wave of each role: 64 rows
            const int q = qt + rt;
            if (role_q) {
                float l2 = kPosInf;
                if (q < q_len) {
                    const float l = p.lse[(int64_t)(qr.start + q) * p.hq + h];
                    l2 = l == kNegInf ? kPosInf : l * kLog2e;
                }
                pre_s = l2;
            } else {
                pre_s = q < q_len ? p.delta[(int64_t)(qr.start + q) * p.hq + h] : 0.f;
            }
        }
    };
    auto store_stage = [&](int buf) {
        char* Qs = smem + buf * STAGE;
        char* Qt = Qs + TILE_BYTES;
        char* Ds = Qt + TILE_BYTES;
        char* Dt = Ds + TILE_BYTES;
        float* ls = reinterpret_cast<float*>(Dt + TILE_BYTES);
        float* ds = ls + kQT;
        char* rm = role_q ? Qs : Ds;
        char* tr = role_q ? Qt : Dt;
#pragma unroll
        for (int uu = 0; uu < UPT; ++uu) {
            const int u = rt + HALF * uu;
            if (rt0 + HALF * uu < UNITS) {
                const int dc = u % (D / 8), qg = u / (D / 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) st16(rm + rm_offset<D>(4 * qg + i, dc), pre[uu][i]);
                u32x2_t trv[8];
                transpose4x8(pre[uu], trv);
#pragma unroll
                for (int i = 0; i < 8; ++i) st8(tr + tr_store_offset(8 * dc + i, qg), trv[i]);
            }
        }
        if (rt0 == 0) (role_q ? ls : ds)[rt] = pre_s;
    };

    uint32_t rofs[4], tofs[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        rofs[c] = rm_offset<D>(l32, 2 * c + hi);
        tofs[c] = tr_load_offset(l32, c, hi);
    }

    f32x16_t dkacc[DB], dvacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) { dkacc[db] = f32x16_t{}; dvacc[db] = f32x16_t{}; }

    if (n_stages > 0) {
        load_stage(0);
        store_stage(0);
        __syncthreads();
        for (int st = 0; st < n_stages; ++st) {
            const bool has_next = st + 1 < n_stages;
            if (has_next) load_stage(st + 1);
            const int h = hk * p.g + st / n_q_tiles;
            const int qt = q_lo + (st % n_q_tiles) * kQT;
            const char* Qs = smem + (st & 1) * STAGE;
            const char* Qt = Qs + TILE_BYTES;
            const char* Ds = Qt + TILE_BYTES;
            const char* Dt = Ds + TILE_BYTES;
            const float* ls = reinterpret_cast<const float*>(Dt + TILE_BYTES);
            const float* dls = ls + kQT;
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                const int qf0 = qt + 32 * qb;            // first query of this block
                const int qf1 = min(q_len, qf0 + 32) - 1;
                bool skip = !wave_active || qf0 >= q_len;
                if (p.causal && kw > qf1 + coff) skip = true;
                if (p.window > 0 && wk_last < qf0 + coff - p.window + 1) skip = true;
                if (skip) continue;
                const bool need_mask = (kw + kKW > kv_len) || (qf0 + 32 > q_len) ||
                                       (p.causal && wk_last > qf0 + coff) ||
                                       (p.window > 0 && kw < qf1 + coff - p.window + 1);
                f32x16_t sacc = f32x16_t{}, pacc = f32x16_t{};
#pragma unroll
                for (int kc = 0; kc < DC; ++kc) {
                    const uint32_t o = rofs[kc & 3] + (kc >> 2) * 128 + qb * 32 * 2 * D;
                    sacc = mfma32<T>(ld16(Qs + o), kf[kc], sacc);
                    pacc = mfma32<T>(ld16(Ds + o), vf[kc], pacc);
                }
                const float* brow0 = nullptr;
                if (BIAS) brow0 = p.bias + (int64_t)h * p.bias_hs + key;
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    const int qi = 32 * qb + 8 * rg + 4 * hi;   // stage-local query of r = 4 rg
                    const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(ls + qi);
                    const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(dls + qi);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * rg + e;
                        const int qrow = qt + qi + e;
                        const bool ok = !need_mask ||
                                        (qrow < q_len && allowed(qrow, key, coff, kv_len, p.causal, p.window));
                        float x = sacc[r] * p.scale_log2;
                        if (BIAS && ok && key < p.bias_cols)
                            x += brow0[(int64_t)(qr.start + qrow) * p.bias_qs] * kLog2e;
                        const float pr = ok ? __builtin_amdgcn_exp2f(x - l4[e]) : 0.f;
                        sacc[r] = pr;                               // P
                        pacc[r] = pr * (pacc[r] - d4[e]);           // dS
                    }
                }
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int r0 = 8 * c;
                    const u32x4_t bp = u32x4_t{T::pack2(sacc[r0 + 0], sacc[r0 + 1]), T::pack2(sacc[r0 + 2], sacc[r0 + 3]),
                                               T::pack2(sacc[r0 + 4], sacc[r0 + 5]), T::pack2(sacc[r0 + 6], sacc[r0 + 7])};
                    const u32x4_t bs = u32x4_t{T::pack2(pacc[r0 + 0], pacc[r0 + 1]), T::pack2(pacc[r0 + 2], pacc[r0 + 3]),
                                               T::pack2(pacc[r0 + 4], pacc[r0 + 5]), T::pack2(pacc[r0 + 6], pacc[r0 + 7])};
                    const int cc = 2 * qb + c;                 // 16-query chunk within the stage
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const uint32_t o = tofs[cc ^ (2 * (db & 1))] + db * 32 * 128;
                        dvacc[db] = mfma32<T>(ld16(Dt + o), bp, dvacc[db]);
                        dkacc[db] = mfma32<T>(ld16(Qt + o), bs, dkacc[db]);
                    }
                }
            }
            if (has_next) store_stage((st + 1) & 1);
            __syncthreads();
        }
    }

    if (wave_active && key_ok) {
        const int64_t off = (int64_t)(kr.start + key) * ((int64_t)p.hkv * D) + (int64_t)hk * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                store4<T, OUT_F32>(p.dk, off + d, dkacc[db][4 * rg] * p.scale, dkacc[db][4 * rg + 1] * p.scale,
                                   dkacc[db][4 * rg + 2] * p.scale, dkacc[db][4 * rg + 3] * p.scale);
                store4<T, OUT_F32>(p.dv, off + d, dvacc[db][4 * rg], dvacc[db][4 * rg + 1],
                                   dvacc[db][4 * rg + 2], dvacc[db][4 * rg + 3]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O). 16-bit types with D % 8 == 0 and 16 | D * 4 lanes:
// one wave per row, every lane streams 16-byte chunks of the contiguous
// [H * D] row (coalesced), lanes sharing a head reduce with DPP shuffles.
// Other cases: one thread per (row, head).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_preprocess_row_kernel(const uint16_t* __restrict__ o, int64_t o_rs,
                                                                 const uint16_t* __restrict__ dout, int64_t do_rs,
                                                                 float* __restrict__ delta, int64_t total_q, int hq,
                                                                 int d) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= total_q) return;
    const int lpg = d / 8;                         // lanes per head: 8 (D=64) or 16 (D=128)
    const int chunks = hq * lpg;                   // 16-byte chunks per row
    const uint16_t* op = o + row * o_rs;
    const uint16_t* dp = dout + row * do_rs;
    for (int c0 = 0; c0 < chunks; c0 += 64) {
        const int c = c0 + lane;
        float acc = 0.f;
        if (c < chunks) {
            const u32x4_t a = ld16(op + 8 * c), b = ld16(dp + 8 * c);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc += lo16<T>(a[e]) * lo16<T>(b[e]) + hi16<T>(a[e]) * hi16<T>(b[e]);
        }
        for (int off = lpg >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        if (c < chunks && (c % lpg) == 0) delta[row * hq + c / lpg] = acc;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const typename T::raw* __restrict__ o, int64_t o_rs,
                                                             const typename T::raw* __restrict__ dout, int64_t do_rs,
                                                             float* __restrict__ delta, int64_t total_q, int hq, int d) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_q * hq) return;
    const int64_t row = i / hq;
    const int h = (int)(i - row * hq);
    const typename T::raw* op = o + row * o_rs + (int64_t)h * d;
    const typename T::raw* dp = dout + row * do_rs + (int64_t)h * d;
    float acc = 0.f;
    for (int c = 0; c < d; ++c) acc += T::to_float(op[c]) * T::to_float(dp[c]);
    delta[i] = acc;
}

// Zero the rows of a [total_rows, row_elems] 16/32-bit tensor that lie outside
// [cu[0], cu[num_seqs]) -- rows no sequence owns receive no gradient.
__global__ __launch_bounds__(256) void zero_outside_kernel(uint16_t* __restrict__ ptr, int64_t row_halves,
                                                           int64_t total_rows, const int* __restrict__ cu,
                                                           int num_seqs) {
    int64_t first = cu[0], last = cu[num_seqs];
    first = first < 0 ? 0 : (first > total_rows ? total_rows : first);
    last = last < first ? first : (last > total_rows ? total_rows : last);
    const int64_t head_end = first * row_halves, tail_begin = last * row_halves, end = total_rows * row_halves;
    const int64_t n = head_end + (end - tail_begin);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        ptr[i < head_end ? i : tail_begin + (i - head_end)] = 0;
}

int gcd_int(int a, int b) { while (b) { const int t = a % b; a = b; b = t; } return a; }

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
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.hkv = g.hkv; p.g = g.g;
    p.hpw = 1;
    p.n_tiles = 0; p.n_hg = 0;
    p.scale = g.scale; p.scale_log2 = g.scale * kLog2e;
    p.causal = g.causal; p.window = g.window > 0 ? g.window : 0;
    return p;
}

template <typename T, int D, bool OUT_F32>
hipError_t launch_dq_typed(const BwdArgs& a, hipStream_t st) {
    constexpr int NW = DqCfg<D>::NW;
    BwdKParams p = make_params(a);
    p.hpw = gcd_int(a.geo.g, NW);
    const int QT = 32 * (NW / p.hpw);
    p.n_tiles = (int)(a.geo.total_q / QT) + a.geo.num_seqs + 1;
    p.n_hg = a.geo.hq / p.hpw;
    const int64_t blocks = (int64_t)p.n_tiles * p.n_hg;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (a.geo.bias != nullptr)
        hipLaunchKernelGGL((bwd_dq_kernel<T, D, true, OUT_F32>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, p);
    else
        hipLaunchKernelGGL((bwd_dq_kernel<T, D, false, OUT_F32>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, p);
    return hipGetLastError();
}

template <typename T, int D, bool OUT_F32>
hipError_t launch_dkv_typed(const BwdArgs& a, hipStream_t st) {
    BwdKParams p = make_params(a);
    constexpr int NW = DkvCfg<D>::NW;
    p.n_tiles = (int)(a.geo.total_kv / (NW * kKW)) + a.geo.num_seqs + 1;
    const int64_t blocks = (int64_t)p.n_tiles * a.geo.hkv;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (a.geo.bias != nullptr)
        hipLaunchKernelGGL((bwd_dkv_kernel<T, D, true, OUT_F32>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, p);
    else
        hipLaunchKernelGGL((bwd_dkv_kernel<T, D, false, OUT_F32>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_preprocess(int dtype, const Geometry& geo, const void* o, int64_t o_rs,
                                 const void* dout, int64_t do_rs, float* delta, hipStream_t st) {
    const int64_t n = geo.total_q * geo.hq;
    if (n == 0) return hipSuccess;
    const bool rowwise = dtype != MTLATTN_DTYPE_F32 && (geo.d == 64 || geo.d == 128) &&
                         ((uintptr_t)o & 15u) == 0 && ((uintptr_t)dout & 15u) == 0 && (o_rs % 8) == 0 &&
                         (do_rs % 8) == 0;
    if (rowwise) {
        const dim3 grid((unsigned)((geo.total_q + 3) / 4));
        if (dtype == MTLATTN_DTYPE_BF16)
            hipLaunchKernelGGL(bwd_preprocess_row_kernel<BF16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                               (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d);
        else
            hipLaunchKernelGGL(bwd_preprocess_row_kernel<F16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                               (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((n + 255) / 256));
    if (dtype == MTLATTN_DTYPE_BF16)
        hipLaunchKernelGGL(bwd_preprocess_kernel<BF16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                           (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d);
    else if (dtype == MTLATTN_DTYPE_F16)
        hipLaunchKernelGGL(bwd_preprocess_kernel<F16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                           (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d);
    else
        hipLaunchKernelGGL(bwd_preprocess_kernel<F32>, grid, dim3(256), 0, st, (const float*)o, o_rs,
                           (const float*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d);
    return hipGetLastError();
}

hipError_t launch_zero_outside(void* ptr, int64_t row_bytes, int64_t total_rows, const int* cu, int num_seqs,
                               hipStream_t st) {
    if (total_rows <= 0 || row_bytes <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_outside_kernel, dim3(64), dim3(256), 0, st, (uint16_t*)ptr, row_bytes / 2, total_rows,
                       cu, num_seqs);
    return hipGetLastError();
}

hipError_t launch_bwd_dq_mfma(int dtype, const BwdArgs& a, hipStream_t st) {
    const int d = a.geo.d;
    const bool f = a.out_f32 != 0;
    if (dtype == MTLATTN_DTYPE_BF16) {
        if (d == 128) return f ? launch_dq_typed<BF16, 128, true>(a, st) : launch_dq_typed<BF16, 128, false>(a, st);
        if (d == 64) return f ? launch_dq_typed<BF16, 64, true>(a, st) : launch_dq_typed<BF16, 64, false>(a, st);
    } else if (dtype == MTLATTN_DTYPE_F16) {
        if (d == 128) return f ? launch_dq_typed<F16, 128, true>(a, st) : launch_dq_typed<F16, 128, false>(a, st);
        if (d == 64) return f ? launch_dq_typed<F16, 64, true>(a, st) : launch_dq_typed<F16, 64, false>(a, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_bwd_dkv_mfma(int dtype, const BwdArgs& a, hipStream_t st) {
    const int d = a.geo.d;
    const bool f = a.out_f32 != 0;
    if (dtype == MTLATTN_DTYPE_BF16) {
        if (d == 128) return f ? launch_dkv_typed<BF16, 128, true>(a, st) : launch_dkv_typed<BF16, 128, false>(a, st);
        if (d == 64) return f ? launch_dkv_typed<BF16, 64, true>(a, st) : launch_dkv_typed<BF16, 64, false>(a, st);
    } else if (dtype == MTLATTN_DTYPE_F16) {
        if (d == 128) return f ? launch_dkv_typed<F16, 128, true>(a, st) : launch_dkv_typed<F16, 128, false>(a, st);
        if (d == 64) return f ? launch_dkv_typed<F16, 64, true>(a, st) : launch_dkv_typed<F16, 64, false>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace mtlattn
