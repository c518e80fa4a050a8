// Backward for fp16/bf16 on gfx950 MFMA: the delta preprocess, a dQ kernel
// and a dK/dV kernel (counterparts of the reference's bwd_dq_mpp /
// bwd_dkv_mpp, src/attn_mpp.metal:546-799, and the delta reduction at
// src/ext.mm:518). No atomics anywhere: every output element is written by
// exactly one lane, so results are bitwise run-to-run deterministic. At head
// dims 64 and 128 the full backward has the dQ kernel compute delta itself
// (bitwise equal to the preprocess) and hand it to the dK/dV kernel.
//
// Shared mathematics (src/attention.metal:707-717):
//   P = exp(scale q.k + bias - lse), dP = dO.v, dS = P (dP - delta),
//   dQ = scale dS K, dK = scale dS^T Q (summed over the GQA group), dV = P^T dO.
// P and dS are rounded to the input type before the second products, as the
// forward rounds P before P.V.
//
// dQ kernel: workgroup of 8 waves (2 per SIMD), 32 query rows x 1 head per
//   wave, GQA heads packed like the forward. Per 64-key tile staged in LDS by
//   direct loads (K, V row-major, swizzled): S^T = K Q^T and dP^T = V dO^T
//   (C layout: lane = query), dS^T in registers, dQ^T += K^T dS^T with K^T
//   read through transposing LDS loads.
// dK/dV kernel: workgroup of 4 wave pairs, 32 keys per pair (128 keys of one
//   kv head). Loops over the g query heads of the group and over 64-query
//   stages staged by direct loads (Q, dO, lse, delta). Wave A of a pair:
//   S = Q K^T, P, dV^T += dO^T P; wave B, one stage behind: dP = dO V^T,
//   dS = P (dP - delta) with P handed over through LDS, dK^T += Q^T dS.
//   Causal and window bands skip whole query blocks (the reference skips
//   causal only, src/attn_mpp.metal:591). At head dims <= 64 without a bias
//   a variant runs 4-wave workgroups (two per CU) in which every wave
//   computes all four products for its own 32 keys.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "bwd_common.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kKW = 32;   // dK/dV: keys per wave

// ---------------------------------------------------------------------------
// dQ.  8 waves (2 per SIMD), 32 query rows x 1 head per wave, the heads of a
// GQA group packed as in the forward; without a bias at D <= 128 workgroups
// of 4 waves, two per CU; at D = 256 one workgroup of 4 waves per CU (one
// per SIMD, 512 registers each). Key tiles of 32 * KB rows (64; 32 for the
// 256-wide tiles) go straight from HBM into an LDS ring of NBUF slots (3;
// 2 for the 4-wave D = 128 workgroups) (K and V row-major, swizzled); K^T
// operands of the dQ product are transposed LDS reads of the same K tile.
// ---------------------------------------------------------------------------
// D is the tile width (64, 128 or 256) and DV <= D the head dim, as in the
// forward. This launch outputs the DO columns from C0 (head dims above 128
// take several launches, the S and dP products recomputed in each: their
// accumulators would not fit otherwise). Key tiles hold 32 * KB keys.
// BROWS > 0: a head-broadcast bias staged in the LDS ring with the K/V tiles
// (workgroups of BROWS query rows, 64-key tiles), as in the forward.
template <typename T, int D, int DV, int DO, int C0, int KB, bool BIAS, bool OUT_F32, int BROWS = 0, int NW = kWaves,
          int OCC = 1, int NBUF = 3>
__global__ __launch_bounds__(NW * 64, OCC) void bwd_dq_kernel(BwdKParams p) {
    constexpr int DC = (DV + 15) / 16, DB = (DO + 31) / 32;
    constexpr int KT = 32 * KB;               // keys per tile
    static_assert(C0 % 32 == 0 && C0 + DO <= D, "output slice");
    constexpr bool LDSB = BROWS > 0;
    static_assert(!LDSB || (BIAS && KT == 64 && NW == 8), "staged bias: 64-key tiles, 8 waves");
    constexpr int TILE = KT * D * 2;
    constexpr int BTILE = BROWS * KT * 4;
    constexpr int STAGE = 2 * TILE + BTILE;   // K, V, staged bias
    static_assert(NBUF == 2 || NBUF == 3, "ring depth");
    constexpr int AHEAD = NBUF - 1;           // tiles in flight ahead of the one in use
    constexpr int LOADS = STAGE / 1024 / NW;
    __shared__ __attribute__((aligned(1024))) char smem[NBUF * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const int QT = 32 * (NW / p.hpw);
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.n_hg);
    const int hg = L / p.n_tiles;
    const int t = p.n_tiles - 1 - (L - hg * p.n_tiles);   // late (heavier) tiles first
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
    const Band band = key_band(qrow, coff, kv_len, p.causal, p.window);
    // rows past the sequence end read its last row (finite, never stored)
    const int64_t grow = qr.start + min(qrow, q_len - 1);

    // B operands: Q^T and dO^T fragments (lane = query, d = 16 kc + 8 hi + j).
    u32x4_t qf[DC], df[DC];
    {
        const uint16_t* qp = p.q + grow * p.q_rs + (int64_t)head * DV + 8 * hi;
        const uint16_t* dp = p.dout + grow * p.do_rs + (int64_t)head * DV + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc) {
            const bool in = DV % 16 == 0 || 16 * kc + 8 * hi < DV;    // columns past DV are zero
            qf[kc] = in ? ld16(qp + 16 * kc) : u32x4_t{};
            df[kc] = in ? ld16(dp + 16 * kc) : u32x4_t{};
        }
    }
    float lse2 = kPosInf, dlt = 0.f;
    // fused delta (single launch over the whole head): this lane holds chunks
    // 2 kc + hi (8 columns each) of its row, so the preprocess's butterfly
    // over 16-column-group lanes (partners i ^ DC, ..., i ^ 1) becomes an
    // in-register tree over kc followed by one exchange across hi.
    constexpr bool kFuseDelta = C0 == 0 && DO == DV && DV == D && D <= 128;
    bool fused = false;
    if constexpr (kFuseDelta) {
        if (p.delta_w != nullptr) {
            fused = true;
            const uint16_t* op = p.o + grow * p.o_rs + (int64_t)head * D + 8 * hi;
            float cs[DC];
#pragma unroll
            for (int kc = 0; kc < DC; ++kc) cs[kc] = dot8<T>(ld16(op + 16 * kc), df[kc]);
#pragma unroll
            for (int off = DC / 2; off > 0; off >>= 1)
#pragma unroll
                for (int kc = 0; kc < off; ++kc) cs[kc] = cs[kc] + cs[kc + off];
            const float dsum = cs[0] + __shfl_xor(cs[0], 32);
            if (row_ok) {
                dlt = dsum;
                if (hi == 0) p.delta_w[grow * p.hq + head] = dsum;
            }
        }
    }
    if (row_ok) {
        const float l = p.lse[grow * p.hq + head];
        lse2 = l == kNegInf ? kPosInf : l * kLog2e;   // empty rows: P = 0
        if (!fused) dlt = p.delta[grow * p.hq + head];
    }
    // bias row of this lane's query (rows past the end read the last row);
    // columns at or past bias_cols read as 0
    constexpr bool reg_bias = BIAS && !LDSB;     // bias loaded into registers per tile
    const float* brow = nullptr;
    if (reg_bias)
        brow = p.bias + bias_row_offset(grow, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) +
               (int64_t)head * p.bias_hs;
    // settle these loads here: the key loop's own wait counts cover only the
    // staging loads
    wait_vmcnt<0>();

    const int q_last_wg = min(q_len, q0 + QT) - 1;
    const int kv_hi = p.causal ? min(kv_len, q_last_wg + coff + 1) : kv_len;
    int kv_lo = 0;
    if (p.window > 0) {
        kv_lo = max(0, q0 + coff - p.window + 1);
        kv_lo = (kv_lo / KT) * KT;
    }
    const int n_kv_tiles = kv_hi > kv_lo ? (kv_hi - kv_lo + KT - 1) / KT : 0;
    const uint16_t* kbase = p.k + (int64_t)kr.start * p.k_rs + (int64_t)hk * DV;
    const uint16_t* vbase = p.v + (int64_t)kr.start * p.v_rs + (int64_t)hk * DV;
    TileStager<D, KT, NW, DV> kst, vst;
    kst.init(p.k_rs, w, lane);
    vst.init(p.v_rs, w, lane);
    // staged bias: WG row r is query q0 + r (rows past the end repeat the last)
    BiasStager<LDSB ? BROWS : 32> bst;
    const float* brow0 = nullptr;
    if (LDSB) {
        auto row_off = [&](int r) {
            return bias_row_offset(qr.start + min(q0 + r, q_len - 1), s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows);
        };
        bst.init(row_off, w, lane);
        brow0 = p.bias + row_off(0);
    }
    // Tiles are staged in order: the next tile's ring slot, first key and
    // K / V rows advance by one tile per call (no division, no row product).
    int ld_slot = 0, ld_kt = kv_lo;
    const uint16_t* ld_k = kbase + (int64_t)kv_lo * p.k_rs;
    const uint16_t* ld_v = vbase + (int64_t)kv_lo * p.v_rs;
    auto stage = [&]() {
        char* buf = smem + ld_slot * STAGE;
        kst.issue_at(buf, ld_k, p.k_rs, kv_len - ld_kt, w, lane);
        vst.issue_at(buf + TILE, ld_v, p.v_rs, kv_len - ld_kt, w, lane);
        if (LDSB) bst.issue(buf + 2 * TILE, brow0, ld_kt, (int)p.bias_cols, w);
        ld_slot = ld_slot == NBUF - 1 ? 0 : ld_slot + 1;
        ld_kt += KT;
        ld_k += (int64_t)KT * p.k_rs;
        ld_v += (int64_t)KT * p.v_rs;
    };

    const uint32_t rbase = row_base<D>(l32, hi), tbase = tr_base<D>(lane);
    const float c2 = p.scale_log2;

    f32x16_t dqacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) dqacc[db] = f32x16_t{};
    // Without a bias dP^T accumulates onto -delta (this lane's query in all
    // 16 C slots), so dS^T = P^T (dP^T - delta) is one multiply per element.
    // (The biased variants have no registers to spare for the block.)
    f32x16_t ndlt;
#pragma unroll
    for (int r = 0; r < 16; ++r) ndlt[r] = -dlt;

    if (n_kv_tiles > 0) stage();
    if (AHEAD > 1 && n_kv_tiles > 1) stage();
    int slot = 0;                                // ring slot of tile it
    for (int it = 0; it < n_kv_tiles; ++it, slot = slot == NBUF - 1 ? 0 : slot + 1) {
        if (AHEAD > 1 && it + 1 < n_kv_tiles) wait_vmcnt<LOADS * (AHEAD - 1)>(); else wait_vmcnt<0>();
        __syncthreads();
        // (with a bias, the tile loads go out after the bias is consumed: the
        // bias loads' wait would otherwise also wait for them)
        if (!reg_bias && it + AHEAD < n_kv_tiles) stage();
        const int kt = kv_lo + it * KT;
        // the bias of the whole tile, all loads in flight together (4-key
        // groups at 32 kb + 8 g + 4 hi)
        f32x4_t bv[4 * KB];
        if (LDSB) {   // from the staged tile: this lane's query row
            const char* bt = opaque(smem + slot * STAGE + 2 * TILE + bias_base(32 * (w % wph) + l32, hi));
#pragma unroll
            for (int i = 0; i < 4 * KB; ++i)
                bv[i] = *reinterpret_cast<const f32x4_t*>(lds_xor(bt, 16 * (8 * (i >> 2) + 2 * (i & 3))));
            if (kt + KT > p.bias_cols) {   // keys at or past the bias columns read as 0
                asm volatile("");
#pragma unroll
                for (int i = 0; i < 4 * KB; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi + j >= p.bias_cols) bv[i][j] = 0.f;
            }
            // (keeps these reads out of the operand read pipeline below)
            __builtin_amdgcn_sched_barrier(0);
        }
        if (reg_bias) {
            if (kt + KT <= p.bias_cols && p.bias_v4) {
#pragma unroll
                for (int i = 0; i < 4 * KB; ++i)
                    bv[i] = *reinterpret_cast<const f32x4_t*>(brow + kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi);
            } else {
#pragma unroll
                for (int i = 0; i < 4 * KB; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int key = kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi + j;
                        const float b = brow[min(key, (int)p.bias_cols - 1)];
                        bv[i][j] = key < p.bias_cols ? b : 0.f;
                    }
            }
        }
        // tiles outside this wave's band are computed fully masked, not
        // skipped (a branch around the MFMAs costs accumulator copies)
        // (bitwise | and &: these uniform tests must not become branches,
        // which would split the loop body into separately scheduled blocks)
        const bool skip = !wave_active | ((p.causal != 0) & (kt > wq_last + coff)) |
                          ((p.window > 0) & (kt + KT - 1 < qa + coff - p.window + 1));
        const char* Ks = smem + slot * STAGE;
        const char* krb = opaque(Ks + rbase);
        const char* ktb = opaque(Ks + tbase);
        const bool need_mask = skip | (kt + KT > kv_len) | ((p.causal != 0) & (kt + KT - 1 > qa + coff)) |
                               ((p.window > 0) & (kt < wq_last + coff - p.window + 1));
        const int d0 = kt + 4 * hi - band.lo;
        const uint32_t wdt = skip ? 0u : band.width;
        // S^T and dP^T of both 32-key halves on the matrix cores first; half
        // 0's elementwise work overlaps half 1's MFMAs, half 1's overlaps
        // half 0's dQ products. P = exp2(S - lse) needs no running max.
        f32x16_t sacc[KB], pacc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sacc[kb] = pacc[kb] = BIAS ? f32x16_t{} : ndlt;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sacc[kb] = f32x16_t{};
#pragma unroll
        for (int kc = 0; kc < DC; ++kc) {
            const char* a = lds_xor(krb, 32 * kc);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                sacc[kb] = mfma32<T>(ld16(a + kb * 32 * 2 * D), qf[kc], sacc[kb]);
                pacc[kb] = mfma32<T>(ld16(a + kb * 32 * 2 * D + TILE), df[kc], pacc[kb]);
            }
        }
        pipe_reads<1, 2 * KB * DC, 4>();
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = fmaf(sacc[kb][r], c2, -lse2);
                if (BIAS) x = fmaf(bv[4 * kb + (r >> 2)][r & 3], kLog2e, x);
                sacc[kb][r] = __builtin_amdgcn_exp2f(x);
            }
            if (reg_bias && kb == KB - 1 && it + AHEAD < n_kv_tiles) stage();
            if (need_mask) {     // out-of-band keys -> P = 0
                asm volatile("");   // keep a real branch (no speculated selects on every tile)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
                    sacc[kb][r] = (uint32_t)(d0 + c) < wdt ? sacc[kb][r] : 0.f;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] *= BIAS ? pacc[kb][r] - dlt : pacc[kb][r];   // dS^T
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int c = 2 * kb + cc, r0 = 8 * cc;
                const u32x4_t bs = u32x4_t{T::pack2(sacc[kb][r0 + 0], sacc[kb][r0 + 1]),
                                           T::pack2(sacc[kb][r0 + 2], sacc[kb][r0 + 3]),
                                           T::pack2(sacc[kb][r0 + 4], sacc[kb][r0 + 5]),
                                           T::pack2(sacc[kb][r0 + 6], sacc[kb][r0 + 7])};
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    dqacc[db] = mfma32<T>(tr_operand<D>(ktb, c, db + C0 / 32), bs, dqacc[db]);
            }
        }
    }

    if (wave_active && row_ok) {
        const int64_t off = grow * ((int64_t)p.hq * DV) + (int64_t)head * DV + C0;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                if ((DO % 32 != 0 && d >= DO) || (C0 + DO > DV && C0 + d >= DV)) continue;
                store4<T, OUT_F32>(p.dq, off + d, dqacc[db][4 * rg] * p.scale, dqacc[db][4 * rg + 1] * p.scale,
                                   dqacc[db][4 * rg + 2] * p.scale, dqacc[db][4 * rg + 3] * p.scale);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK / dV.  8 waves = 4 pairs; pair i is waves i and i + 4 (the same SIMD)
// and owns 32 keys of one kv head, so a workgroup owns 128 keys. The pair
// splits the four products between its two waves:
//   wave A (i):     S = Q K^T,  P = exp2(S c - lse2),  dV^T += dO^T P
//   wave B (i + 4): dP = dO V^T, dS = P (dP - delta),   dK^T += Q^T dS
//                   (the dP products start from -delta)
// A hands P (rounded to the input type, C layout) to B through LDS; B runs
// one stage behind A, so one barrier per stage orders everything. Each wave
// holds one operand (K or V) and one accumulator set in registers, which keeps
// both waves of a SIMD resident: one's softmax overlaps the other's MFMAs.
// A stage is (query head h of the group, tile of 32 * NQB queries): Q, lse
// and delta go straight from HBM into a 3-deep LDS ring, dO into a 2-deep one
// (row-major, swizzled); Q^T and dO^T operands are transposed LDS reads. The
// loop covers the g heads of the group, so the GQA reduction of dK/dV
// happens in registers.
// ---------------------------------------------------------------------------
// D is the tile width (64, 128 or 256) and DV <= D the head dim; a
// workgroup outputs the DO columns of dK and dV from C0 + DO * blockIdx.y
// (DO < DV: the slices run as workgroups of one launch, each recomputing the
// S and dP products). A stage holds 32 * NQB queries.
template <typename T, int D, int DV, int DO, int C0, int NQB, bool BIAS, bool OUT_F32>
__global__ __launch_bounds__(kThreads, 1) void bwd_dkv_kernel(BwdKParams p) {
    constexpr int DC = (DV + 15) / 16, DB = (DO + 31) / 32;
    static_assert(C0 % 32 == 0 && C0 + DO <= D, "output slice");
    // first output column of this workgroup's slice: C0, plus DO per slice
    // when the columns are split (a multiple of 128 in a 256-wide tile, so
    // the transposed reads of the slice are those of slice 0 with the byte
    // offset's bit 8 flipped)
    constexpr bool SLICED = DO < DV;
    static_assert(!SLICED || (C0 == 0 && DO == 128 && D == 256), "column slices of the 256-wide tiles");
    const int c0 = SLICED ? DO * (int)blockIdx.y : C0;
    const uint32_t tslice = SLICED ? 2u * (uint32_t)c0 : 0u;
    constexpr int QTL = 32 * NQB;                       // queries per stage
    constexpr int NP = kWaves / 2;                      // wave pairs
    constexpr int KB = NP * kKW;                        // keys per workgroup
    constexpr int TILE = QTL * D * 2;
    constexpr int LROWS = QTL > 64 ? QTL : 64;          // rows of a staged lse / delta column
    constexpr int LPIECES = LROWS / 64;                 // 64-row loads per column
    static_assert(2 * LPIECES <= NP, "one loader wave per lse / delta piece");
    // Q ring: Q tile, lse and delta columns of a stage. Wave B reads Q one
    // stage behind wave A, and stage st + 1 loads meanwhile: three slots.
    constexpr int QSTAGE = TILE + 2 * LROWS * 4;
    constexpr int NBUF = 3;
    // dO ring: a stage's dO is read only during that stage (wave A's dV,
    // wave B's dP), so the loads of stage st + 1 reuse the slot of st - 1.
    constexpr int NDO = 2;
    constexpr int DO_OFF = NBUF * QSTAGE;
    constexpr int PBLK = 2 * 1024;                      // packed P of one 32x32 block
    constexpr int PSTAGE = NP * NQB * PBLK;             // one stage, all pairs
    constexpr int P_OFF = DO_OFF + NDO * TILE;
    __shared__ __attribute__((aligned(1024))) char smem[P_OFF + 2 * PSTAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const bool role_a = w < NP;
    const int pair = w & (NP - 1);
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.hkv);
    const int hk = L / p.n_tiles;
    const int t = L - hk * p.n_tiles;                  // early key blocks (heavier when causal) first
    const int s = find_seq_for_tile(p.cu_kv, p.num_seqs, KB, t, p.total_kv);
    const int tb = tile_base(p.cu_kv, s, KB, p.total_kv);
    if (t < tb) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int k0 = (t - tb) * KB;
    if (k0 >= kv_len) return;
    const int coff = kv_len - q_len;

    const int kw = k0 + kKW * pair;              // first key of this pair (seq-local)
    const bool pair_active = kw < kv_len;
    const int wk_last = min(kv_len, kw + kKW) - 1;
    const int key = kw + l32;                    // this lane's key column
    const bool key_ok = key < kv_len;

    // B operand of this wave's first product: K^T (wave A) or V^T (wave B),
    // lane = key, d = 16 kc + 8 hi + j.
    u32x4_t kvf[DC];
    {
        const int64_t grow = kr.start + min(key, kv_len - 1);     // masked past the end
        const uint16_t* kp = role_a ? p.k + grow * p.k_rs : p.v + grow * p.v_rs;
        kp += (int64_t)hk * DV + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc)     // columns past DV are zero
            kvf[kc] = (DV % 16 == 0 || 16 * kc + 8 * hi < DV) ? ld16(kp + 16 * kc) : u32x4_t{};
    }

    // Query range that can see any key of this workgroup.
    const int k_last_wg = min(kv_len, k0 + KB) - 1;
    // (tile grid aligned to QTL so workgroups of a sequence share tiles)
    const int q_lo = p.causal ? max(0, k0 - coff) / QTL * QTL : 0;
    const int q_hi = p.window > 0 ? min(q_len, k_last_wg - coff + p.window) : q_len;
    const int n_q_tiles = q_hi > q_lo ? (q_hi - q_lo + QTL - 1) / QTL : 0;
    const int n_stages = n_q_tiles * p.g;

    // Stages run over the query tiles top-down with the heads inner, so every
    // workgroup of a sequence reads the same (tile, head) at the same time and
    // the L2 serves the repeats (each workgroup stops at its own causal start
    // q_lo); under a sliding window the walk starts at a tile fixed by the
    // tile index and wraps (first_q_tile), which keeps that property.
    // Stages are visited in order, so each per-stage quantity (head, first
    // query, ring slot, source rows) is a cursor advanced one stage at a time:
    // no division by g or by the ring depth in the loop.
    const int qt_first = first_q_tile(q_lo, n_q_tiles, QTL, p.window > 0);
    const int64_t cyc = (int64_t)n_q_tiles * QTL;        // rows of the walk's wrap
    // Direct loads of stage `st`: Q and dO tiles by four loader waves
    // (ldw = 0..3); lse by loaders 0 (and 2), delta by loaders 1 (and 3):
    // column ldw & 1, rows 64 (ldw >> 1) + lane, 4 bytes per lane.
    const int ldw = BIAS ? (role_a ? -1 : w - NP) : (role_a ? w : -1);
    TileStager<D, QTL, NP, DV> qst, dost;
    if (ldw >= 0) {
        qst.init(p.q_rs, ldw, lane);
        dost.init(p.do_rs, ldw, lane);
    }
    // Loader cursor: the next stage to issue. Advancing to the next head
    // moves the rows by DV columns (lse / delta by one); past the group's
    // last head they move to head 0 of the tile QTL rows up.
    int ld_hl = 0, ld_qt = qt_first, ld_slot = 0, ld_dslot = 0;
    const int l_col = ldw & 1, l_piece = ldw >> 1;   // (loaders with ldw < 2 * LPIECES)
    const uint16_t* ld_q = p.q + (int64_t)(qr.start + qt_first) * p.q_rs + (int64_t)hk * p.g * DV;
    const uint16_t* ld_do = p.dout + (int64_t)(qr.start + qt_first) * p.do_rs + (int64_t)hk * p.g * DV;
    const float* ld_l = (l_col == 0 ? p.lse : p.delta) + (int64_t)(qr.start + qt_first) * p.hq + hk * p.g;
    const int64_t q_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.q_rs;
    const int64_t do_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.do_rs;
    const int64_t l_wrap = -(int64_t)(p.g - 1) - (int64_t)QTL * p.hq;
    const int l_row = 64 * l_piece + lane;           // stage-local row this lane loads
    const uint32_t l_voff = (uint32_t)l_row * (uint32_t)p.hq * 4u;
    // stage() issues the loader cursor's stage and advance()s the cursor.
    // Without a bias the A waves issue the tile loads: wave B, one stage
    // behind, is the longer of the two and should not stall on issue. With
    // a bias the A waves keep their own bias loads in flight, and the wait
    // for those would also cover tile loads issued after them, so the B
    // waves load the tiles.
    auto advance = [&]() {
        ld_slot = ld_slot == NBUF - 1 ? 0 : ld_slot + 1;
        ld_dslot ^= 1;
        if (++ld_hl == p.g) {
            ld_hl = 0;
            ld_qt -= QTL;
            ld_q += q_wrap;
            ld_do += do_wrap;
            ld_l += l_wrap;
            if (ld_qt < q_lo) {   // wrap to the top tile (first_q_tile)
                ld_qt += (int)cyc;
                ld_q += cyc * p.q_rs;
                ld_do += cyc * p.do_rs;
                ld_l += cyc * p.hq;
            }
        } else {
            ld_q += DV;
            ld_do += DV;
            ld_l += 1;
        }
    };
    auto stage = [&]() {
        if (ldw < 0) return;
        char* buf = smem + ld_slot * QSTAGE;
        const int avail = q_len - ld_qt;                    // >= 1
        qst.issue_at(buf, ld_q, p.q_rs, avail, ldw, lane);
        dost.issue_at(smem + DO_OFF + ld_dslot * TILE, ld_do, p.do_rs, avail, ldw, lane);
        if (ldw < 2 * LPIECES) {   // rows past the end repeat the last row (masked)
            const uint32_t voff = avail >= LROWS ? l_voff : (uint32_t)min(l_row, avail - 1) * (uint32_t)p.hq * 4u;
            lds_dma4s(ld_l, voff, buf + TILE + (l_col * LROWS + 64 * l_piece) * 4);
        }
        advance();
    };
    // For the 256-wide tiles without a bias, the A waves issue their loads of
    // stage st + 1 one at a time between their S products of stage st
    // instead of in a burst at its start (D = 256 backward -3.5%; at D <= 128
    // within noise, so those keep the burst).
    constexpr bool SPREAD = !BIAS && D > 128 && NQB * DC >= 4 * ((QTL * D * 2 / 1024 + NP - 1) / NP);
    // Compute cursor: stage st (wave A, and wave B's dP) and the ring slot of
    // stage st - 1 (wave B's dS and dK).
    int c_hl = 0, c_qt = qt_first, c_slot = 0, p_slot = NBUF - 1, c_dslot = 0;
    float bvals[NQB][16];                       // wave A: bias of the current query tile
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) bvals[qb][r] = 0.f;

    const uint32_t rbase = row_base<D>(l32, hi), tbase = tr_base<D>(lane);
    const float c2 = p.scale_log2;

    f32x16_t acc[DB];                            // dV^T (wave A) or dK^T (wave B)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16_t{};
    f32x16_t pacc[NQB];                          // wave B: dP of the previous stage
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) pacc[qb] = f32x16_t{};

    // Is the 32x32 block (queries qf0.., this pair's keys) of stage st empty
    // or does it need per-element masking? Identical in both waves of a pair.
    // Does the 32x32 block (queries qf0.., this pair's keys) need per-element
    // masking? Blocks entirely outside the band (nothing to add) are also
    // "masked": they are computed with P = 0 rather than skipped, because a
    // branch around the MFMAs costs accumulator copies.
    auto block_needs_mask = [&](int qb) {
        const int qf0 = c_qt + 32 * qb;
        const int qf1 = min(q_len, qf0 + 32) - 1;
        return (kw + kKW > kv_len) | (qf0 + 32 > q_len) | ((p.causal != 0) & (wk_last > qf0 + coff)) |
               ((p.window > 0) & (kw < qf1 + coff - p.window + 1));
    };
    // Does any block of the stage need masking? Each term is the per-block
    // test at the block that decides it (the first block for the causal
    // edge, the last for the sequence end and the window edge), so the
    // common unmasked stage costs one test, not one per block.
    auto stage_needs_mask = [&]() {
        return (kw + kKW > kv_len) | (c_qt + QTL > q_len) | ((p.causal != 0) & (wk_last > c_qt + coff)) |
               ((p.window > 0) & (kw < min(q_len, c_qt + QTL) + coff - p.window));
    };
    const Band band = query_band(key, coff, q_len, kv_len, p.causal, p.window);

    if (n_stages > 0) {
        stage();
        wait_vmcnt<0>();
        if (ldw >= 0 && ldw < 2 * LPIECES) neg_col(reinterpret_cast<float*>(smem + TILE) + l_col * LROWS + l_row, l_col);
        __syncthreads();
    }
    for (int st = 0; n_stages > 0 && st <= n_stages; ++st) {
        const bool load_next = st + 1 < n_stages;
        if (load_next && !(SPREAD && role_a && st < n_stages)) stage();
        if (role_a && st < n_stages) {
            const char* Qs = smem + c_slot * QSTAGE;
            const char* Ds = smem + DO_OFF + c_dslot * TILE;
            const float* ls = reinterpret_cast<const float*>(Qs + TILE);   // -lse log2(e)
            const char* qrb = opaque(Qs + rbase);
            const char* dtb = opaque(Ds + (tbase ^ tslice));
            char* pb = smem + P_OFF + (st & 1) * PSTAGE + pair * NQB * PBLK;
            const int h = hk * p.g + c_hl;
            const int qt = c_qt;
            // The stage's bias (this lane's key column, 32 query rows per
            // block), all loads in flight together under the S products;
            // columns at or past bias_cols read as 0, rows past the end read
            // the last row. A bias shared by all heads is loaded at the first
            // head of each query tile and kept for the group's other heads.
            // Fast path -- whole stage inside the sequence (and its bias
            // rows), every key of the pair inside the bias columns: buffer
            // loads from the stage's first bias row, the lane's column and 4
            // hi rows in the per-lane offset, each element's row in the
            // scalar offset (no per-element address arithmetic, no select).
            const bool fast_bias = BIAS && p.bias_b32 && (qt + QTL <= q_len) &&
                                   ((p.bias_ss < 0) | (qt + QTL <= p.bias_rows)) && (kw + kKW <= p.bias_cols);
            const bool load_bias = BIAS && ((c_hl == 0) | (p.bias_hs != 0));
            if (!load_bias) {
            } else if (fast_bias) {
                const float* b0 = p.bias + bias_row_offset(qr.start + qt, s, qr.start, p.bias_qs, p.bias_ss,
                                                           p.bias_rows) + (int64_t)h * p.bias_hs;
                const __amdgpu_buffer_rsrc_t rs =
                    __builtin_amdgcn_make_buffer_rsrc((void*)b0, (short)0, (int)0xffffffff, 0x00020000);
                const int voff = (int)((4 * hi * p.bias_qs + key) * 4);
                // row stride in bytes, opaque here so that the 32 per-row
                // scalar offsets are formed per stage (one s_mul each) rather
                // than hoisted out of the loop into 32 live SGPRs
                int rs4 = (int)(p.bias_qs * 4);
                asm volatile("" : "+s"(rs4));
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        bvals[qb][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rs, voff, (32 * qb + 8 * (r >> 2) + (r & 3)) * rs4, 0));
            } else if (BIAS) {
                const float* bcol = p.bias + (int64_t)h * p.bias_hs + min(key, (int)p.bias_cols - 1);
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int qrow = min(qt + 32 * qb + 8 * (r >> 2) + 4 * hi + (r & 3), q_len - 1);
                        bvals[qb][r] =
                            bcol[bias_row_offset(qr.start + qrow, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows)];
                    }
            }
            f32x16_t sacc[NQB];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) sacc[qb] = f32x16_t{};
            if constexpr (SPREAD) {
                // one group per S product: the MFMA, the operand read four
                // products ahead and, every second product, one load of
                // stage st + 1 (groups kept in order by scheduling barriers)
                constexpr int NS = NQB * DC;
                constexpr int LQ = decltype(qst)::N;             // Q (and dO) loads per loader wave
                static_assert(decltype(qst)::PER % NP == 0, "whole loads per loader wave");
                char* lbuf = smem + ld_slot * QSTAGE;
                char* dbuf = smem + DO_OFF + ld_dslot * TILE;
                const int avail = q_len - ld_qt;
                uint32_t qo[LQ], dso[LQ];
                if (avail >= QTL) {
#pragma unroll
                    for (int j = 0; j < LQ; ++j) { qo[j] = qst.off[j]; dso[j] = dost.off[j]; }
                } else {
                    const int rmax = max(avail - 1, 0);
#pragma unroll
                    for (int j = 0; j < LQ; ++j) {
                        const int i = ldw + j * NP;
                        const int r = min(decltype(qst)::row_of(i, lane), rmax);
                        qo[j] = decltype(qst)::lane_off(i, lane, r, (uint32_t)(2 * p.q_rs));
                        dso[j] = decltype(dost)::lane_off(i, lane, r, (uint32_t)(2 * p.do_rs));
                    }
                }
                const uint32_t lvoff = avail >= LROWS ? l_voff : (uint32_t)min(l_row, avail - 1) * (uint32_t)p.hq * 4u;
                auto products = [&](auto with_loads) {
                    u32x4_t qa[NS];
#pragma unroll
                    for (int i = 0; i < 4; ++i) qa[i] = row_operand<D>(qrb, i / NQB, 32 * (i % NQB));
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < NS; ++i) {
                        sacc[i % NQB] = mfma32<T>(qa[i], kvf[i / NQB], sacc[i % NQB]);
                        if (i + 4 < NS) qa[i + 4] = row_operand<D>(qrb, (i + 4) / NQB, 32 * ((i + 4) % NQB));
                        if (decltype(with_loads)::value && (i == 0 || (i & 1))) {
                            // load 0: lse / delta, 1..LQ: Q, LQ+1..2LQ: dO
                            const int j = i == 0 ? 0 : (i + 1) >> 1;
                            if (j == 0) {
                                if (ldw < 2 * LPIECES)
                                    lds_dma4s(ld_l, lvoff, lbuf + TILE + (l_col * LROWS + 64 * l_piece) * 4);
                            } else if (j <= LQ) {
                                lds_dma16s(ld_q, qo[j - 1], lbuf + (ldw + (j - 1) * NP) * 1024);
                            } else if (j <= 2 * LQ) {
                                lds_dma16s(ld_do, dso[j - 1 - LQ], dbuf + (ldw + (j - 1 - LQ) * NP) * 1024);
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                };
                if (load_next) {
                    products(std::integral_constant<bool, true>{});
                    advance();
                } else {
                    products(std::integral_constant<bool, false>{});
                }
            } else {
#pragma unroll
            for (int kc = 0; kc < DC; ++kc)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
                    sacc[qb] = mfma32<T>(row_operand<D>(qrb, kc, 32 * qb), kvf[kc], sacc[qb]);
            }
            // exponentials of both blocks (overlapping the S MFMAs in flight),
            // then the rarely needed masks, then the dV products
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    const int qi = 32 * qb + 8 * rg + 4 * hi;    // stage-local query of r = 4 rg
                    const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(ls + qi);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * rg + e;
                        float arg;
                        // (rows with no allowed key or every logit -inf
                        // have lse = -inf and l4 = -inf: P = 0)
                        if (fast_bias) {
                            arg = fmaf(bvals[qb][r], kLog2e, fmaf(sacc[qb][r], c2, l4[e]));
                        } else if (BIAS) {   // the same arithmetic, keys past the bias columns read 0
                            arg = fmaf(key < p.bias_cols ? bvals[qb][r] : 0.f, kLog2e, fmaf(sacc[qb][r], c2, l4[e]));
                        } else {
                            arg = fmaf(sacc[qb][r], c2, l4[e]);
                        }
                        sacc[qb][r] = __builtin_amdgcn_exp2f(arg);
                    }
                }
            }
            if (stage_needs_mask()) {
                asm volatile("");
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    // out-of-band elements (and rows with no allowed key) -> P = 0
                    if (block_needs_mask(qb)) {
                        asm volatile("");   // keep a real branch (no speculated selects on every block)
                        const int d0 = qt + 32 * qb + 4 * hi - band.lo;   // query - band.lo at r = 0
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            sacc[qb][r] = (uint32_t)(d0 + 8 * (r >> 2) + (r & 3)) < band.width ? sacc[qb][r] : 0.f;
                    }
                }
            }
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    const int r0 = 8 * cc;
                    const u32x4_t bp = u32x4_t{T::pack2(sacc[qb][r0 + 0], sacc[qb][r0 + 1]),
                                               T::pack2(sacc[qb][r0 + 2], sacc[qb][r0 + 3]),
                                               T::pack2(sacc[qb][r0 + 4], sacc[qb][r0 + 5]),
                                               T::pack2(sacc[qb][r0 + 6], sacc[qb][r0 + 7])};
                    st16(pb + qb * PBLK + cc * 1024 + lane * 16, bp);
#pragma unroll
                    for (int db = 0; db < DB; ++db)
                        acc[db] = mfma32<T>(tr_operand<D>(dtb, 2 * qb + cc, db + C0 / 32), bp, acc[db]);
                }
            }
        }
        if (!role_a) {
            // Wave B runs a software pipeline one stage behind wave A: first
            // dS and dK of stage st - 1 (dP of that stage is already in
            // registers), then dP of stage st. Its VALU phase (dS) thus meets
            // wave A's S products and its dK products meet wave A's
            // exponentials, instead of both waves of a SIMD issuing matrix
            // work and then VALU work at the same time.
            if (st > 0) {
                const char* Qs = smem + p_slot * QSTAGE;
                const char* qtb = opaque(Qs + (tbase ^ tslice));
                const char* pb = smem + P_OFF + ((st - 1) & 1) * PSTAGE + pair * NQB * PBLK;
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) {
                        const u32x4_t pp = ld16(pb + qb * PBLK + cc * 1024 + lane * 16);
                        float dsv[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const float pr = (j & 1) ? hi16<T>(pp[j >> 1]) : lo16<T>(pp[j >> 1]);
                            dsv[j] = pr * pacc[qb][8 * cc + j];
                        }
                        const u32x4_t bs = u32x4_t{T::pack2(dsv[0], dsv[1]), T::pack2(dsv[2], dsv[3]),
                                                   T::pack2(dsv[4], dsv[5]), T::pack2(dsv[6], dsv[7])};
#pragma unroll
                        for (int db = 0; db < DB; ++db)
                            acc[db] = mfma32<T>(tr_operand<D>(qtb, 2 * qb + cc, db + C0 / 32), bs, acc[db]);
                    }
                }
            }
            if (st < n_stages) {
                // dP - delta: the products accumulate onto -delta (the staged
                // delta column is negated), so dS is one multiply per element
                const char* drb = opaque(smem + DO_OFF + c_dslot * TILE + rbase);
                const float* dls = reinterpret_cast<const float*>(smem + c_slot * QSTAGE + TILE) + LROWS;
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
                    for (int rg = 0; rg < 4; ++rg) {
                        const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(dls + 32 * qb + 8 * rg + 4 * hi);
#pragma unroll
                        for (int e = 0; e < 4; ++e) pacc[qb][4 * rg + e] = d4[e];
                    }
#pragma unroll
                for (int kc = 0; kc < DC; ++kc)
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb)
                        pacc[qb] = mfma32<T>(row_operand<D>(drb, kc, 32 * qb), kvf[kc], pacc[qb]);
            }
        }
        // stage st + 1 landed for this wave; the lse / delta loaders turn
        // their pieces into -lse log2 e and -delta before the barrier
        // publishes the stage
        const int n_slot = c_slot == NBUF - 1 ? 0 : c_slot + 1;
        wait_vmcnt<0>();
        if (ldw >= 0 && ldw < 2 * LPIECES && st + 1 < n_stages) {
            float* l = reinterpret_cast<float*>(smem + n_slot * QSTAGE + TILE);
            neg_col(l + l_col * LROWS + l_row, l_col);
        }
        __syncthreads();
        p_slot = c_slot;
        c_slot = n_slot;
        c_dslot ^= 1;
        if (++c_hl == p.g) {
            c_hl = 0;
            c_qt -= QTL;
            if (c_qt < q_lo) c_qt += (int)cyc;
        }
    }

    if (pair_active && key_ok) {
        const int64_t off = (int64_t)(kr.start + key) * ((int64_t)p.hkv * DV) + (int64_t)hk * DV + c0;
        void* dst = role_a ? p.dv : p.dk;
        const float sc = role_a ? 1.f : p.scale;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                if ((DO % 32 != 0 && d >= DO) || (c0 + d >= DV)) continue;
                store4<T, OUT_F32>(dst, off + d, acc[db][4 * rg] * sc, acc[db][4 * rg + 1] * sc,
                                   acc[db][4 * rg + 2] * sc, acc[db][4 * rg + 3] * sc);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK/dV at head dims <= 64 without a bias: every wave computes all four
// products for its own 32 keys -- S = Q K^T, P, dV^T += dO^T P,
// dP = dO V^T, dS = P (dP - delta), dK^T += Q^T dS -- so nothing passes
// between waves. A wave's dK and dV accumulators take 64 registers at
// D = 64, which leaves room at 2 waves per SIMD; at D = 128 they would not
// fit, and the wave-pair kernel above splits the products between two
// waves instead. Workgroups of NW = 4 waves (128 keys), two per CU: the two
// waves of a SIMD belong to different workgroups, so their tile barriers do
// not hold them in step (measured 5-8% faster than 8-wave workgroups at
// D = 64, which stage each Q / dO tile for 256 keys but keep both waves of
// a SIMD in step). The arithmetic is that of the wave-pair kernel (P
// rounded to T, dP accumulated onto -delta, dS = P * (dP - delta) rounded
// to T), visited in 64-query stages.
// ---------------------------------------------------------------------------
template <typename T, int D, int DV, bool OUT_F32, int NW>
__global__ __launch_bounds__(NW * 64, kWaves / NW) void bwd_dkv_sym_kernel(BwdKParams p) {
    static_assert(D == 64, "64-wide tiles");
    constexpr int NQB = 2;
    constexpr int DC = (DV + 15) / 16, DB = (DV + 31) / 32;
    constexpr int QTL = 32 * NQB;                       // queries per stage
    constexpr int KB = NW * kKW;                        // keys per workgroup
    constexpr int TILE = QTL * D * 2;
    constexpr int SLOT = (2 * TILE + 2 * QTL * 4 + 1023) / 1024 * 1024;   // Q, dO, lse, delta
    constexpr int NBUF = 2;
    __shared__ __attribute__((aligned(1024))) char smem[NBUF * SLOT];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.hkv);
    const int hk = L / p.n_tiles;
    const int t = L - hk * p.n_tiles;                  // early key blocks (heavier when causal) first
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

    // B operands of the S and dP products: K^T and V^T, lane = key,
    // d = 16 kc + 8 hi + j (rows past the end read the last key: masked)
    u32x4_t kf[DC], vf[DC];
    {
        const int64_t grow = kr.start + min(key, kv_len - 1);
        const uint16_t* kp = p.k + grow * p.k_rs + (int64_t)hk * DV + 8 * hi;
        const uint16_t* vp = p.v + grow * p.v_rs + (int64_t)hk * DV + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc) {   // columns past DV are zero
            const bool in = DV % 16 == 0 || 16 * kc + 8 * hi < DV;
            kf[kc] = in ? ld16(kp + 16 * kc) : u32x4_t{};
            vf[kc] = in ? ld16(vp + 16 * kc) : u32x4_t{};
        }
    }

    // Query tiles that can see any key of the workgroup, visited top-down
    // with the GQA group's heads inner (as in the wave-pair kernel).
    const int k_last_wg = min(kv_len, k0 + KB) - 1;
    const int q_lo = p.causal ? max(0, k0 - coff) / QTL * QTL : 0;
    const int q_hi = p.window > 0 ? min(q_len, k_last_wg - coff + p.window) : q_len;
    const int n_q_tiles = q_hi > q_lo ? (q_hi - q_lo + QTL - 1) / QTL : 0;
    const int n_stages = n_q_tiles * p.g;
    const int qt_first = first_q_tile(q_lo, n_q_tiles, QTL, p.window > 0);
    const int64_t cyc = (int64_t)n_q_tiles * QTL;        // rows of the walk's wrap

    // Direct loads of a stage: the Q and dO tiles by all NW waves, the lse
    // column by wave 0 and the delta column by wave 1 (one row per lane).
    TileStager<D, QTL, NW, DV> qst, dost;
    qst.init(p.q_rs, w, lane);
    dost.init(p.do_rs, w, lane);
    int ld_hl = 0, ld_qt = qt_first, ld_slot = 0;
    const uint16_t* ld_q = p.q + (int64_t)(qr.start + qt_first) * p.q_rs + (int64_t)hk * p.g * DV;
    const uint16_t* ld_do = p.dout + (int64_t)(qr.start + qt_first) * p.do_rs + (int64_t)hk * p.g * DV;
    const float* ld_l = (w == 0 ? p.lse : p.delta) + (int64_t)(qr.start + qt_first) * p.hq + hk * p.g;
    const int64_t q_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.q_rs;
    const int64_t do_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.do_rs;
    const int64_t l_wrap = -(int64_t)(p.g - 1) - (int64_t)QTL * p.hq;
    const uint32_t l_voff = (uint32_t)lane * (uint32_t)p.hq * 4u;
    auto stage = [&]() {
        char* buf = smem + ld_slot * SLOT;
        const int avail = q_len - ld_qt;                    // >= 1
        qst.issue_at(buf, ld_q, p.q_rs, avail, w, lane);
        dost.issue_at(buf + TILE, ld_do, p.do_rs, avail, w, lane);
        if (w < 2) {   // rows past the end repeat the last row (masked)
            const uint32_t voff = avail >= QTL ? l_voff : (uint32_t)min(lane, avail - 1) * (uint32_t)p.hq * 4u;
            lds_dma4s(ld_l, voff, buf + 2 * TILE + w * QTL * 4);
        }
        ld_slot ^= 1;
        if (++ld_hl == p.g) {
            ld_hl = 0;
            ld_qt -= QTL;
            ld_q += q_wrap;
            ld_do += do_wrap;
            ld_l += l_wrap;
            if (ld_qt < q_lo) {   // wrap to the top tile (first_q_tile)
                ld_qt += (int)cyc;
                ld_q += cyc * p.q_rs;
                ld_do += cyc * p.do_rs;
                ld_l += cyc * p.hq;
            }
        } else {
            ld_q += DV;
            ld_do += DV;
            ld_l += 1;
        }
    };

    int c_hl = 0, c_qt = qt_first, c_slot = 0;
    const uint32_t rbase = row_base<D>(l32, hi), tbase = tr_base<D>(lane);
    const float c2 = p.scale_log2;
    f32x16_t accv[DB], acck[DB];                 // dV^T, dK^T
#pragma unroll
    for (int db = 0; db < DB; ++db) accv[db] = acck[db] = f32x16_t{};

    // masking tests, as in the wave-pair kernel (for this wave's keys)
    auto block_needs_mask = [&](int qb) {
        const int qf0 = c_qt + 32 * qb;
        const int qf1 = min(q_len, qf0 + 32) - 1;
        return (kw + kKW > kv_len) | (qf0 + 32 > q_len) | ((p.causal != 0) & (wk_last > qf0 + coff)) |
               ((p.window > 0) & (kw < qf1 + coff - p.window + 1));
    };
    auto stage_needs_mask = [&]() {
        return (kw + kKW > kv_len) | (c_qt + QTL > q_len) | ((p.causal != 0) & (wk_last > c_qt + coff)) |
               ((p.window > 0) & (kw < min(q_len, c_qt + QTL) + coff - p.window));
    };
    const Band band = query_band(key, coff, q_len, kv_len, p.causal, p.window);

    if (n_stages > 0) {
        stage();
        wait_vmcnt<0>();
        if (w < 2) neg_col(reinterpret_cast<float*>(smem + 2 * TILE) + w * QTL + lane, w);
        __syncthreads();
    }
    for (int st = 0; st < n_stages; ++st) {
        // the other slot was read in the previous stage, which every wave
        // has finished (barrier below)
        if (st + 1 < n_stages) stage();
        const char* Qs = smem + c_slot * SLOT;
        const char* Ds = Qs + TILE;
        const float* ls = reinterpret_cast<const float*>(Qs + 2 * TILE);   // -lse log2(e)
        const float* dls = ls + QTL;                                         // -delta
        const char* qrb = opaque(Qs + rbase);
        const char* drb = opaque(Ds + rbase);
        const int qt = c_qt;
        f32x16_t sacc[NQB], pacc[NQB];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sacc[qb] = f32x16_t{};
#pragma unroll
        for (int kc = 0; kc < DC; ++kc)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) sacc[qb] = mfma32<T>(row_operand<D>(qrb, kc, 32 * qb), kf[kc], sacc[qb]);
        // dP - delta: the products accumulate onto -delta
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(dls + 32 * qb + 8 * rg + 4 * hi);
#pragma unroll
                for (int e = 0; e < 4; ++e) pacc[qb][4 * rg + e] = d4[e];
            }
#pragma unroll
        for (int kc = 0; kc < DC; ++kc)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) pacc[qb] = mfma32<T>(row_operand<D>(drb, kc, 32 * qb), vf[kc], pacc[qb]);
        // P (rows with no allowed key have lse = -inf: P = 0)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(ls + 32 * qb + 8 * rg + 4 * hi);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    sacc[qb][4 * rg + e] = __builtin_amdgcn_exp2f(fmaf(sacc[qb][4 * rg + e], c2, l4[e]));
            }
        if (stage_needs_mask()) {
            asm volatile("");
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                if (block_needs_mask(qb)) {   // out-of-band elements -> P = 0
                    asm volatile("");
                    const int d0 = qt + 32 * qb + 4 * hi - band.lo;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        sacc[qb][r] = (uint32_t)(d0 + 8 * (r >> 2) + (r & 3)) < band.width ? sacc[qb][r] : 0.f;
                }
            }
        }
        const char* dtb = opaque(Ds + tbase);
        const char* qtb = opaque(Qs + tbase);
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int r0 = 8 * cc;
                const u32x4_t bp = u32x4_t{T::pack2(sacc[qb][r0 + 0], sacc[qb][r0 + 1]),
                                           T::pack2(sacc[qb][r0 + 2], sacc[qb][r0 + 3]),
                                           T::pack2(sacc[qb][r0 + 4], sacc[qb][r0 + 5]),
                                           T::pack2(sacc[qb][r0 + 6], sacc[qb][r0 + 7])};
#pragma unroll
                for (int db = 0; db < DB; ++db) accv[db] = mfma32<T>(tr_operand<D>(dtb, 2 * qb + cc, db), bp, accv[db]);
                float dsv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float pr = (j & 1) ? hi16<T>(bp[j >> 1]) : lo16<T>(bp[j >> 1]);
                    dsv[j] = pr * pacc[qb][r0 + j];
                }
                const u32x4_t bs = u32x4_t{T::pack2(dsv[0], dsv[1]), T::pack2(dsv[2], dsv[3]),
                                           T::pack2(dsv[4], dsv[5]), T::pack2(dsv[6], dsv[7])};
#pragma unroll
                for (int db = 0; db < DB; ++db) acck[db] = mfma32<T>(tr_operand<D>(qtb, 2 * qb + cc, db), bs, acck[db]);
            }
        }
        // the next stage landed for this wave; the lse / delta loaders turn
        // their columns into -lse log2 e and -delta before the barrier
        // publishes it
        wait_vmcnt<0>();
        if (w < 2 && st + 1 < n_stages) neg_col(reinterpret_cast<float*>(smem + (c_slot ^ 1) * SLOT + 2 * TILE) + w * QTL + lane, w);
        __syncthreads();
        c_slot ^= 1;
        if (++c_hl == p.g) {
            c_hl = 0;
            c_qt -= QTL;
            if (c_qt < q_lo) c_qt += (int)cyc;
        }
    }

    if (wave_active && key_ok) {
        const int64_t off = (int64_t)(kr.start + key) * ((int64_t)p.hkv * DV) + (int64_t)hk * DV;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                if (DV % 32 != 0 && d >= DV) continue;
                store4<T, OUT_F32>(p.dv, off + d, accv[db][4 * rg], accv[db][4 * rg + 1], accv[db][4 * rg + 2],
                                   accv[db][4 * rg + 3]);
                store4<T, OUT_F32>(p.dk, off + d, acck[db][4 * rg] * p.scale, acck[db][4 * rg + 1] * p.scale,
                                   acck[db][4 * rg + 2] * p.scale, acck[db][4 * rg + 3] * p.scale);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O). 16-bit types with D % 8 == 0 (D <= 512): one wave
// per row; a head's D / 8 sixteen-byte chunks go to a group of lg lanes (the
// next power of two, so groups never straddle), 64 / lg heads per pass, and
// each group reduces with shuffles. Reads are coalesced: consecutive lanes
// read consecutive chunks of the contiguous [H * D] row. Other cases: one
// thread per (row, head).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void bwd_preprocess_row_kernel(const uint16_t* __restrict__ o, int64_t o_rs,
                                                                 const uint16_t* __restrict__ dout, int64_t do_rs,
                                                                 float* __restrict__ delta, int64_t total_q, int hq,
                                                                 int d, int lg) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= total_q) return;
    const int lpg = d / 8;                         // 16-byte chunks per head
    const int hl = lane / lg, j = lane - hl * lg;  // head within the pass, chunk
    const uint16_t* op = o + row * o_rs;
    const uint16_t* dp = dout + row * do_rs;
    for (int h0 = 0; h0 < hq; h0 += 64 / lg) {
        const int h = h0 + hl;
        float acc = 0.f;
        if (h < hq && j < lpg) acc = dot8<T>(ld16(op + h * d + 8 * j), ld16(dp + h * d + 8 * j));
        for (int off = lg >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        if (h < hq && j == 0) delta[row * hq + h] = acc;
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

// Zero the rows of [total_rows, row_elems] 16/32-bit tensors that lie outside
// [cu[0], cu[num_seqs]) -- rows no sequence owns receive no gradient. One
// launch covers up to three tensors (blockIdx.y picks the job).
struct ZeroJob {
    uint16_t* ptr;
    int64_t row_halves, total_rows;
    const int* cu;
};
struct ZeroJobs {
    ZeroJob job[3];
    int num_seqs;
};
__global__ __launch_bounds__(256) void zero_outside_kernel(ZeroJobs jobs) {
    const ZeroJob& j = jobs.job[blockIdx.y];
    uint16_t* __restrict__ ptr = j.ptr;
    const int64_t row_halves = j.row_halves, total_rows = j.total_rows;
    int64_t first = j.cu[0], last = j.cu[jobs.num_seqs];
    first = first < 0 ? 0 : (first > total_rows ? total_rows : first);
    last = last < first ? first : (last > total_rows ? total_rows : last);
    const int64_t head_end = first * row_halves, tail_begin = last * row_halves, end = total_rows * row_halves;
    const int64_t n = head_end + (end - tail_begin);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        ptr[i < head_end ? i : tail_begin + (i - head_end)] = 0;
}

int gcd_int(int a, int b) { while (b) { const int t = a % b; a = b; b = t; } return a; }



template <typename T, int D, int DV, int DO, int C0, int KB, bool OUT_F32, int NW = kWaves, int OCC = 1, int NB = 3>
hipError_t launch_dq_typed(const BwdArgs& a, hipStream_t st) {
    // the fused delta needs the whole head in one launch
    if (a.delta_out != nullptr && !(C0 == 0 && DO == DV && DV == D && D <= 128)) return hipErrorInvalidValue;
    BwdKParams p = make_params(a);
    p.hpw = gcd_int(a.geo.g, NW);
    const int QT = 32 * (NW / p.hpw);
    p.n_tiles = (int)(a.geo.total_q / QT) + a.geo.num_seqs + 1;
    p.n_hg = a.geo.hq / p.hpw;
    const int64_t blocks = (int64_t)p.n_tiles * p.n_hg;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    // head-broadcast bias staged in LDS: the forward's conditions
    const Geometry& g = a.geo;
    if (NW == 8 && KB == 2 && D <= 128 && g.bias != nullptr && g.bias_hs == 0 && p.bias_v4 && g.bias_cols >= 4 &&
        g.bias_cols % 4 == 0 && (QT == 32 || QT == 64) && ((int64_t)QT * g.bias_qs + g.bias_cols) * 4 < ((int64_t)1 << 32)) {
        if constexpr (NW == 8 && KB == 2 && D <= 128) {
            if (QT == 32)
                hipLaunchKernelGGL((bwd_dq_kernel<T, D, DV, DO, C0, KB, true, OUT_F32, 32, NW>), dim3((unsigned)blocks),
                                   dim3(NW * 64), 0, st, p);
            else
                hipLaunchKernelGGL((bwd_dq_kernel<T, D, DV, DO, C0, KB, true, OUT_F32, 64, NW>), dim3((unsigned)blocks),
                                   dim3(NW * 64), 0, st, p);
            return hipGetLastError();
        }
    }
    if constexpr (KB > 2) {
        if (a.geo.bias != nullptr) return hipErrorInvalidValue;   // (not dispatched: registers)
    } else if (a.geo.bias != nullptr) {
        hipLaunchKernelGGL((bwd_dq_kernel<T, D, DV, DO, C0, KB, true, OUT_F32, 0, NW, OCC, NB>), dim3((unsigned)blocks), dim3(NW * 64),
                           0, st, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, DV, DO, C0, KB, false, OUT_F32, 0, NW, OCC, NB>), dim3((unsigned)blocks), dim3(NW * 64), 0,
                       st, p);
    return hipGetLastError();
}

template <typename T, int D, int DV, int DO, int C0, int NQB, bool OUT_F32>
hipError_t launch_dkv_typed(const BwdArgs& a, hipStream_t st) {
    BwdKParams p = make_params(a);
    constexpr int NW = kWaves;
    p.n_tiles = (int)(a.geo.total_kv / (NW / 2 * kKW)) + a.geo.num_seqs + 1;
    const int64_t blocks = (int64_t)p.n_tiles * a.geo.hkv;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    // column slices (DO < DV) are the grid's second dimension: one launch,
    // so the slices' workgroups share the GPU instead of running one after
    // the other (a causal grid's tail is one heavy workgroup per CU)
    const dim3 grid((unsigned)blocks, (unsigned)((DV - C0 + DO - 1) / DO));
    if constexpr (NQB > 2) {
        if (a.geo.bias != nullptr) return hipErrorInvalidValue;   // (not dispatched: registers)
    } else if (a.geo.bias != nullptr) {
        hipLaunchKernelGGL((bwd_dkv_kernel<T, D, DV, DO, C0, NQB, true, OUT_F32>), grid, dim3(NW * 64), 0, st, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((bwd_dkv_kernel<T, D, DV, DO, C0, NQB, false, OUT_F32>), grid, dim3(NW * 64), 0, st, p);
    return hipGetLastError();
}

template <typename T, int D, int DV, bool OUT_F32, int NW>
hipError_t launch_dkv_sym(const BwdArgs& a, hipStream_t st) {
    BwdKParams p = make_params(a);
    p.n_tiles = (int)(a.geo.total_kv / (NW * kKW)) + a.geo.num_seqs + 1;
    const int64_t blocks = (int64_t)p.n_tiles * a.geo.hkv;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((bwd_dkv_sym_kernel<T, D, DV, OUT_F32, NW>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, p);
    return hipGetLastError();
}


}  // namespace

hipError_t launch_bwd_preprocess(int dtype, const Geometry& geo, const void* o, int64_t o_rs,
                                 const void* dout, int64_t do_rs, float* delta, hipStream_t st) {
    const int64_t n = geo.total_q * geo.hq;
    if (n == 0) return hipSuccess;
    const bool rowwise = dtype != MTLATTN_DTYPE_F32 && geo.d % 8 == 0 && geo.d <= 512 &&
                         ((uintptr_t)o & 15u) == 0 && ((uintptr_t)dout & 15u) == 0 && (o_rs % 8) == 0 &&
                         (do_rs % 8) == 0;
    if (rowwise) {
        int lg = 1;
        while (lg < geo.d / 8) lg *= 2;                 // lanes per head: a power of two <= 64
        const dim3 grid((unsigned)((geo.total_q + 3) / 4));
        if (dtype == MTLATTN_DTYPE_BF16)
            hipLaunchKernelGGL(bwd_preprocess_row_kernel<BF16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                               (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d, lg);
        else
            hipLaunchKernelGGL(bwd_preprocess_row_kernel<F16>, grid, dim3(256), 0, st, (const uint16_t*)o, o_rs,
                               (const uint16_t*)dout, do_rs, delta, geo.total_q, geo.hq, geo.d, lg);
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

hipError_t launch_zero_outside(const ZeroFill* fills, int n, int num_seqs, hipStream_t st) {
    ZeroJobs jobs{};
    jobs.num_seqs = num_seqs;
    int used = 0;
    for (int i = 0; i < n && i < 3; ++i) {
        if (fills[i].total_rows <= 0 || fills[i].row_bytes <= 0) continue;
        jobs.job[used++] = ZeroJob{(uint16_t*)fills[i].ptr, fills[i].row_bytes / 2, fills[i].total_rows, fills[i].cu};
    }
    if (used == 0) return hipSuccess;
    hipLaunchKernelGGL(zero_outside_kernel, dim3(64, used), dim3(256), 0, st, jobs);
    return hipGetLastError();
}

// the tile width and head dim of each supported head dim (see the forward)
template <typename T, template <typename, int, int, bool> class L>
hipError_t dispatch_dims(const BwdArgs& a, hipStream_t st) {
    const bool f = a.out_f32 != 0;
    switch (a.geo.d) {
        case 64: return f ? L<T, 64, 64, true>::run(a, st) : L<T, 64, 64, false>::run(a, st);
        case 80: return f ? L<T, 128, 80, true>::run(a, st) : L<T, 128, 80, false>::run(a, st);
        case 88: return f ? L<T, 128, 88, true>::run(a, st) : L<T, 128, 88, false>::run(a, st);
        case 96: return f ? L<T, 128, 96, true>::run(a, st) : L<T, 128, 96, false>::run(a, st);
        case 128: return f ? L<T, 128, 128, true>::run(a, st) : L<T, 128, 128, false>::run(a, st);
        case 160: return f ? L<T, 256, 160, true>::run(a, st) : L<T, 256, 160, false>::run(a, st);
        case 256: return f ? L<T, 256, 256, true>::run(a, st) : L<T, 256, 256, false>::run(a, st);
        default: return hipErrorInvalidValue;
    }
}
template <typename T, int D, int DV, bool F>
struct DqLaunch {
    static hipError_t run(const BwdArgs& a, hipStream_t st) {
        if constexpr (D <= 64) {
            // without a bias: workgroups of 4 waves, two per CU (48 KB of
            // LDS each), whose tile barriers do not hold the two waves of a
            // SIMD in step; 2-3% faster than one 8-wave workgroup with
            // 128-key tiles
            if (a.geo.bias == nullptr) return launch_dq_typed<T, D, DV, DV, 0, 2, F, 4, 2>(a, st);
            return launch_dq_typed<T, D, DV, DV, 0, 2, F>(a, st);
        } else if constexpr (D <= 128) {
            // the same with a 2-deep ring of 64-key tiles (64 KB of LDS per
            // workgroup): 0-3% faster than one 8-wave workgroup with a 3-deep
            // ring (GQA, MHA, ragged, windowed)
            if (a.geo.bias == nullptr) return launch_dq_typed<T, D, DV, DV, 0, 2, F, 4, 2, 2>(a, st);
            return launch_dq_typed<T, D, DV, DV, 0, 2, F>(a, st);
        } else {
            // 256-wide tiles: 32-key tiles (three K + V stages fit the LDS).
            // D = 160 computes the whole output in one launch (249 VGPRs).
            // At D = 256 the Q^T and dO^T fragments alone take 128 registers:
            // workgroups of 4 waves (one per SIMD, 512 registers each, the
            // accumulators in AGPRs) compute the whole output in one launch.
            if constexpr (DV > 192) {
                return launch_dq_typed<T, D, DV, DV, 0, 1, F, 4>(a, st);
            } else {
                return launch_dq_typed<T, D, DV, DV, 0, 1, F>(a, st);
            }
        }
    }
};
template <typename T, int D, int DV, bool F>
struct DkvLaunch {
    static hipError_t run(const BwdArgs& a, hipStream_t st) {
        if constexpr (D <= 64) {
            // without a bias: every wave computes all four products for its
            // keys, 4-wave workgroups
            if (a.geo.bias == nullptr) return launch_dkv_sym<T, D, DV, F, 4>(a, st);
            return launch_dkv_typed<T, D, DV, DV, 0, 2, F>(a, st);
        } else if constexpr (D <= 128) {
            // without a bias: one wave per SIMD, 64 keys per wave
            if (a.geo.bias == nullptr) {
                const hipError_t e = launch_bwd_dkv_wide(T::code, a, st);
                if (e != hipErrorNotSupported) return e;
            }
            return launch_dkv_typed<T, D, DV, DV, 0, 2, F>(a, st);
        } else {
            // D = 256 without a bias: one wave per SIMD, 32 keys per wave,
            // all 256 columns in one pass (0.92 vs 1.12 ms at 2 x 4096
            // causal, 16/4 heads; at D = 160 the kernel below was faster)
            if (DV > 192 && a.geo.bias == nullptr) {
                const hipError_t e = launch_bwd_dkv_wide(T::code, a, st);
                if (e != hipErrorNotSupported) return e;
            }
            // 256-wide tiles: 32-query stages. D = 160 computes the whole
            // output in each workgroup (207 VGPRs); D = 256 in 128-column
            // slices, each workgroup one slice (the whole output would spill
            // its accumulators), both slices in one launch
            if constexpr (DV > 192) {
                return launch_dkv_typed<T, D, DV, 128, 0, 1, F>(a, st);
            } else {
                return launch_dkv_typed<T, D, DV, DV, 0, 1, F>(a, st);
            }
        }
    }
};

hipError_t launch_bwd_dq_mfma(int dtype, const BwdArgs& a, hipStream_t st) {
    if (dtype == MTLATTN_DTYPE_BF16) return dispatch_dims<BF16, DqLaunch>(a, st);
    if (dtype == MTLATTN_DTYPE_F16) return dispatch_dims<F16, DqLaunch>(a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_bwd_dkv_mfma(int dtype, const BwdArgs& a, hipStream_t st) {
    if (dtype == MTLATTN_DTYPE_BF16) return dispatch_dims<BF16, DkvLaunch>(a, st);
    if (dtype == MTLATTN_DTYPE_F16) return dispatch_dims<F16, DkvLaunch>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace mtlattn
