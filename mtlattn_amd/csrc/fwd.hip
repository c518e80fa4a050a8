// Flash forward for fp16/bf16 on gfx950 MFMA (counterpart of the reference's
// attn_vl, src/attn_mpp.metal:178-317, redesigned for CDNA4).
//
// Work decomposition
//   * Workgroup = 8 waves (512 threads, 2 waves per SIMD). Each wave owns 32
//     query rows of one query head. The workgroup packs `hpw` = gcd(g, 8) query
//     heads of one GQA group, so every K/V tile staged in LDS serves
//     hpw * (8 / hpw) * 32 = 256 query-head rows. Small grids without a
//     bias (D = 128; D = 64 causal) run 4-wave workgroups instead, two per
//     CU (hpw = gcd(g, 2), a 2-deep ring).
//   * Key tiles of 64 rows (128 on a 2-deep ring at the 128-wide head dims
//     without a bias; 32 at D = 256 and 64 on a 2-deep ring at D = 160 in
//     one launch) go straight
//     from HBM into a 3-deep (or 2-deep) LDS ring with
//     global_load_lds_dwordx4 (no register staging), K and V both row-major
//     and swizzled; the P.V product reads V^T operands with
//     ds_read_b64_tr_b16 transposed loads. Without a bias, each wave's loads
//     of tile i + AHEAD are issued one at a time between its S products of
//     tile i rather than all at once after the tile barrier.
//   * Per wave and key tile:  S^T = K Q^T  (v_mfma_f32_32x32x16, 2 x D/16
//     instructions), online softmax in base 2 on the C registers (each lane
//     holds one query column, so max/sum need one cross-half exchange), then
//     O^T += V^T P^T (4 x D/32 instructions) with P rounded to the input type.
//   * Causal/window tiles outside a wave's band are skipped; the workgroup's
//     key loop starts at the window bottom and stops at the causal horizon, so
//     sliding-window cost is O(W) (src/attn_mpp.metal:216-225).
//   * Varlen tiles are numbered without a host sync (common.h), blocks are
//     remapped so neighbouring query tiles of one (sequence, head) share an XCD.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kKT = 64;          // keys per tile

struct FwdKParams {
    const uint16_t* q; const uint16_t* k; const uint16_t* v;
    uint16_t* o; float* lse;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs;
    int64_t bias_qs, bias_hs, bias_cols, bias_ss, bias_rows;
    int64_t total_q, total_kv;
    int num_seqs, hq, g, hpw, n_tiles, n_hg;
    float scale, scale_log2;
    int causal, window;
    int bias_v4;      // bias rows 16-byte aligned (pointer and strides)
    int col0;         // first output (and V) column of this launch
};

// Softmax modes (SM). 0: no bias, scale > 0: the running max is taken over
// raw scores and the scale folded into one FMA per element. 1: bias,
// scale > 0: logits y = s * scale + bias (one FMA), the max taken over y and
// log2(e) folded into the exponent's FMA. 2: any scale, optional bias:
// explicit per-element scaling (scale <= 0 flips the order of raw scores).
// DV is the head dim (a multiple of 8). K tiles are DK wide (64, 128 or 256
// >= DV): the S contraction uses ceil(DV / 16) k-chunks, Q's columns past DV
// are zero. V tiles hold the DO columns [col0, col0 + DO) that this launch
// outputs, DVL wide (64 or 128 >= DO); P.V computes ceil(DO / 32) output
// blocks and stores the DO valid columns. Head dims above 128 run as two
// launches that each produce half of the output columns (the S products are
// recomputed; their accumulators would not fit otherwise).
// BROWS > 0 (SM 1 only): the bias is one block broadcast over heads and a
// workgroup covers BROWS query rows; each key tile's bias block is staged in
// the LDS ring with the K/V tiles (read from LDS by all waves of all heads)
// instead of every wave loading its rows from global memory.
template <typename T, int DK, int DV, int DVL, int DO, int SM, int BROWS = 0, int KT = kKT, int NW = kWaves, int NBUF = 3>
__global__ __launch_bounds__(NW * 64, kWaves / NW) void fwd_mfma_kernel(FwdKParams p) {
    static_assert(KT == 64 || ((KT == 32 || KT == 128) && BROWS == 0), "32- and 128-key tiles: no staged bias");
    constexpr int NKB = KT / 32;             // 32-key blocks per tile
    constexpr int NPC = KT / 16;             // 16-key P chunks per tile
    constexpr bool BIAS = SM != 0;
    constexpr bool LDSB = BROWS > 0;
    static_assert(!LDSB || SM == 1, "staged bias is for the biased raw-max softmax");
    constexpr int DC = (DV + 15) / 16;       // MFMA k-chunks over the head dim
    constexpr int DB = (DO + 31) / 32;       // 32-row output blocks
    constexpr int KTILE = KT * DK * 2;      // bytes of one K tile
    constexpr int VTILE = KT * DVL * 2;     // bytes of one V tile
    constexpr int BTILE = BROWS * KT * 4;   // bytes of one staged bias tile
    constexpr int STAGE = KTILE + VTILE + BTILE;   // K, V (row-major), bias
    constexpr int AHEAD = NBUF - 1;          // tiles loading ahead of the one in use (ring of NBUF)
    static_assert(NBUF == 2 || NBUF == 3, "the prologue and the waits below assume one or two tiles ahead");
    constexpr int LOADS = STAGE / 1024 / NW;   // direct loads per wave per tile
    static_assert(LOADS <= 15 && STAGE % (1024 * NW) == 0 && (!LDSB || NW == kWaves), "staging");
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
    const int qa = q0 + 32 * (w % wph);          // first query row of this wave (seq-local)
    const int coff = kv_len - q_len;
    const bool wave_active = qa < q_len;
    const int wq_last = min(q_len, qa + 32) - 1;

    // Q^T operand fragments: lane holds query qa + l32, d = 16 kc + 8 hi + (0..7).
    // Rows past the sequence end read its last row (finite, never stored).
    u32x4_t qf[DC];
    {
        const int row = min(qa + l32, q_len - 1);
        const uint16_t* qp = p.q + (int64_t)(qr.start + row) * p.q_rs + (int64_t)head * DV + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < DC; ++kc)
            qf[kc] = (DV % 16 == 0 || 16 * kc + 8 * hi < DV) ? ld16(qp + 16 * kc) : u32x4_t{};
        // settle the fragments here: the key loop's own wait counts cover
        // only the staging loads
        wait_vmcnt<0>();
    }

    // Key range of the whole workgroup.
    const int q_last_wg = min(q_len, q0 + QT) - 1;
    const int kv_hi = p.causal ? min(kv_len, q_last_wg + coff + 1) : kv_len;
    int kv_lo = 0;
    if (p.window > 0) {
        kv_lo = max(0, q0 + coff - p.window + 1);
        kv_lo = (kv_lo / KT) * KT;
    }
    const int n_kv_tiles = kv_hi > kv_lo ? (kv_hi - kv_lo + KT - 1) / KT : 0;

    const uint16_t* kbase = p.k + (int64_t)kr.start * p.k_rs + (int64_t)hk * DV;
    const uint16_t* vbase = p.v + (int64_t)kr.start * p.v_rs + (int64_t)hk * DV + p.col0;
    // The NW waves stage each tile straight from HBM into LDS (K then V).
    TileStager<DK, KT, NW, DV> kst;
    TileStager<DVL, KT, NW, DO> vst;
    kst.init(p.k_rs, w, lane);
    vst.init(p.v_rs, w, lane);
    // Staged bias: WG row r is query q0 + r (rows past the end repeat the last)
    BiasStager<LDSB ? BROWS : 32> bst;
    const float* brow0 = nullptr;
    if (LDSB) {
        auto row_off = [&](int r) {
            return bias_row_offset(qr.start + min(q0 + r, q_len - 1), s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows);
        };
        bst.init(row_off, w, lane);
        brow0 = p.bias + row_off(0);
    }
    auto stage = [&](int it) {
        char* buf = smem + (it % NBUF) * STAGE;
        const int kt = kv_lo + it * KT;
        kst.issue(buf, kbase, p.k_rs, kt, kv_len, w, lane);
        vst.issue(buf + KTILE, vbase, p.v_rs, kt, kv_len, w, lane);
        if (LDSB) bst.issue(buf + KTILE + VTILE, brow0, kt, (int)p.bias_cols, w);
    };

    // per-lane LDS offsets: K operand rows 32 kb + l32 (chunk 2 kc + hi) and
    // the transposed V^T operand reads
    const uint32_t rbase = row_base<DK>(l32, hi), tbase = tr_base<DVL>(lane);

    float m_run = kNegInf, l_run = 0.f;
    f32x16_t oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};

    const int qrow = qa + l32;
    const Band band = key_band(qrow, coff, kv_len, p.causal, p.window);
    // Bias row of this lane's query (rows past the sequence end read its last
    // row: finite, never stored). Columns at or past bias_cols read as 0.
    const bool has_bias = BIAS && p.bias != nullptr;
    const bool reg_bias = has_bias && !LDSB;     // bias loaded into registers per tile
    const float* brow = nullptr;
    if (reg_bias)
        brow = p.bias +
               bias_row_offset(qr.start + min(qrow, q_len - 1), s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) +
               (int64_t)head * p.bias_hs;
    // The bias of a whole tile (this lane's 32 keys: 4-key groups at
    // 32 kb + 8 g + 4 hi) is loaded up front, all loads in flight together,
    // and consumed after the S products; 16-byte loads when aligned.
    auto load_bias = [&](int kt, f32x4_t (&bv)[4 * NKB]) {
        if (kt + KT <= p.bias_cols && p.bias_v4) {
#pragma unroll
            for (int i = 0; i < 4 * NKB; ++i)
                bv[i] = *reinterpret_cast<const f32x4_t*>(brow + kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi);
        } else {
#pragma unroll
            for (int i = 0; i < 4 * NKB; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int key = kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi + j;
                    const float b = brow[min(key, (int)p.bias_cols - 1)];
                    bv[i][j] = key < p.bias_cols ? b : 0.f;
                }
        }
    };
    const float c2 = p.scale_log2;
    // raw-max modes: the max is taken over x (raw scores, or s * scale + bias)
    // and cmul * x is the base-2 logit; max(cmul * x) = cmul * max(x) needs
    // cmul > 0 (scale > 0, host-checked)
    constexpr bool raw_max = SM != 2;
    const float cmul = SM == 1 ? kLog2e : c2;
    // Rescale O only when the running max grows by more than kRescale (log2
    // units): the unnormalised weights then stay <= 2^kRescale, exact after
    // the final division by the row sum. bf16 P keeps its relative precision
    // up to 2^127, so the slack is 32 (the fp32 row sum stays below 2^63 and O
    // below 2^79 for 2^31 keys of fp16-range V); fp16 P must stay below its
    // largest finite value, 65504 < 2^16, so the slack is 15. A bias that grows
    // along the keys (ALiBi-like) raises the max every tile; a wide slack
    // turns those into rare rescales.
    constexpr float kRescale = std::is_same<T, F16>::value ? 15.f : 32.f;
    // For DK <= 64 the softmax VALU work is a larger share of a tile than the
    // MFMAs, so the tile max is skipped: weights are taken against the running
    // max and the max is recomputed only when a row's tile sum reaches
    // kMaxTileSum (weights up to 2^12, still exact in fp32 after the final
    // division) or a live row has no finite max yet.
    constexpr bool kDeferMax = DK <= 64;
    constexpr float kMaxTileSum = 4096.f;
    const bool row_live = wave_active & (band.width > 0);

    if (n_kv_tiles > 0) stage(0);
    if (AHEAD > 1 && n_kv_tiles > 1) stage(1);
    for (int it = 0; it < n_kv_tiles; ++it) {
        // tile `it` landed (the next one may still be in flight), then publish
        if (AHEAD > 1 && it + 1 < n_kv_tiles) wait_vmcnt<LOADS>(); else wait_vmcnt<0>();
        __syncthreads();
        // the buffer of tile it + AHEAD was last read in iteration it - 1 (with a
        // bias, the tile loads go out after the bias is consumed: the bias
        // loads' wait would otherwise also wait for them)
        // Without a bias, the loads of tile it + 2 go out one by one between
        // the S products below instead of in a burst here, where every wave
        // of the CU would queue its loads at the same moment (not at D = 256
        // in one launch: its O and Q registers leave no room for the operand
        // reads held ahead).
        constexpr bool SPREAD = SM == 0 && DB * 16 + DC * 4 <= 160;
        if (!SPREAD && !reg_bias && it + AHEAD < n_kv_tiles) stage(it + AHEAD);
        const int kt = kv_lo + it * KT;
        f32x4_t bv[4 * NKB];
        if (reg_bias) load_bias(kt, bv);
        if (LDSB) {
            // this lane's 4-key groups of its query row from the staged tile
            const char* bt = opaque(smem + (it % NBUF) * STAGE + KTILE + VTILE + bias_base(32 * (w % wph) + l32, hi));
#pragma unroll
            for (int i = 0; i < 4 * NKB; ++i)
                bv[i] = *reinterpret_cast<const f32x4_t*>(lds_xor(bt, 16 * (8 * (i >> 2) + 2 * (i & 3))));
            if (kt + KT > p.bias_cols) {   // keys at or past the bias columns read as 0
                asm volatile("");
#pragma unroll
                for (int i = 0; i < 4 * NKB; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (kt + 32 * (i >> 2) + 8 * (i & 3) + 4 * hi + j >= p.bias_cols) bv[i][j] = 0.f;
            }
            // (keeps these reads out of the K operand read pipeline below)
            __builtin_amdgcn_sched_barrier(0);
        }

        // A tile outside this wave's band is computed fully masked (P = 0)
        // rather than skipped: a branch around the MFMAs makes the compiler
        // copy the 64 O accumulator registers twice per tile.
        // (bitwise | and &: these uniform tests must not become branches,
        // which would split the loop body into separately scheduled blocks)
        const bool skip = !wave_active | ((p.causal != 0) & (kt > wq_last + coff)) |
                          ((p.window > 0) & (kt + KT - 1 < qa + coff - p.window + 1));
        const char* Ks = smem + (it % NBUF) * STAGE;
        const char* kb_ = opaque(Ks + rbase);
        const char* vtb = opaque(Ks + KTILE + tbase);
        f32x16_t sacc[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sacc[kb] = f32x16_t{};
        // raised priority while issuing the S products: when the other wave
        // of the SIMD is in its softmax, the matrix core gets the issue slot
        // (measured +1%)
        __builtin_amdgcn_s_setprio(1);
        if constexpr (SPREAD) {
            // One group per S product: the MFMA, the operand read four
            // products ahead and, at evenly spaced products, one of this
            // wave's tile loads; groups are kept in this order by scheduling
            // barriers (the loads' memory clobber would otherwise stop the
            // reads from being issued ahead of them).
            constexpr int NS = NKB * DC;
            constexpr int LK = decltype(kst)::N, LV = decltype(vst)::N, NL = LK + LV;
            static_assert(decltype(kst)::PER % NW == 0 && decltype(vst)::PER % NW == 0 && NL <= NS,
                          "whole loads per wave");
            const bool load_next = it + AHEAD < n_kv_tiles;
            const int kt2 = kt + AHEAD * KT;
            char* buf2 = smem + ((it + AHEAD) % NBUF) * STAGE;
            const char* ksrc = reinterpret_cast<const char*>(kbase + (int64_t)kt2 * p.k_rs);
            const char* vsrc = reinterpret_cast<const char*>(vbase + (int64_t)kt2 * p.v_rs);
            uint32_t lo[NL];   // per-lane source offsets (rows past the end read the last row)
            if (kv_len - kt2 >= KT) {
#pragma unroll
                for (int j = 0; j < LK; ++j) lo[j] = kst.off[j];
#pragma unroll
                for (int j = 0; j < LV; ++j) lo[LK + j] = vst.off[j];
            } else {
                const int rmax = max(kv_len - kt2 - 1, 0);
#pragma unroll
                for (int j = 0; j < LK; ++j) {
                    const int i = w + j * NW;
                    lo[j] = decltype(kst)::lane_off(i, lane, min(decltype(kst)::row_of(i, lane), rmax),
                                                    (uint32_t)(2 * p.k_rs));
                }
#pragma unroll
                for (int j = 0; j < LV; ++j) {
                    const int i = w + j * NW;
                    lo[LK + j] = decltype(vst)::lane_off(i, lane, min(decltype(vst)::row_of(i, lane), rmax),
                                                         (uint32_t)(2 * p.v_rs));
                }
            }
            auto products = [&](auto with_loads) {
                u32x4_t ka[NS];
#pragma unroll
                for (int i = 0; i < 4 && i < NS; ++i) ka[i] = row_operand<DK>(kb_, i / NKB, 32 * (i % NKB));
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    sacc[i % NKB] = mfma32<T>(ka[i], qf[i / NKB], sacc[i % NKB]);
                    if (i + 4 < NS) ka[i + 4] = row_operand<DK>(kb_, (i + 4) / NKB, 32 * ((i + 4) % NKB));
                    if (decltype(with_loads)::value && i % (NS / NL) == 1 % (NS / NL) && i / (NS / NL) < NL) {
                        const int j = i / (NS / NL);
                        const int row = w + (j < LK ? j : j - LK) * NW;   // 1 KB instruction of the tile
                        if (j < LK) lds_dma16s(ksrc, lo[j], buf2 + row * 1024);
                        else lds_dma16s(vsrc, lo[j], buf2 + KTILE + row * 1024);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            if (load_next) products(std::integral_constant<bool, true>{});
            else products(std::integral_constant<bool, false>{});
        } else {
#pragma unroll
            for (int kc = 0; kc < DC; ++kc) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const u32x4_t a = row_operand<DK>(kb_, kc, 32 * kb);
                    sacc[kb] = mfma32<T>(a, qf[kc], sacc[kb]);
                }
            }
            pipe_reads<1, NKB * DC, 4>();
        }
        // keep the V^T reads of the P.V phase from being hoisted above the
        // softmax (they would pin 64 registers across it)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        const bool need_mask = skip | (kt + KT > kv_len) | ((p.causal != 0) & (kt + KT - 1 > qa + coff)) |
                               ((p.window > 0) & (kt < wq_last + coff - p.window + 1));
        if (need_mask) {
            // (the empty asm keeps this a real branch: speculating the selects
            // into every tile would cost ~100 VALU per tile)
            asm volatile("");
            const int d0 = kt + 4 * hi - band.lo;
            const uint32_t wdt = skip ? 0u : band.width;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int c = 32 * kb + 8 * (r >> 2) + (r & 3);    // key - (kt + 4 hi)
                    sacc[kb][r] = (uint32_t)(d0 + c) < wdt ? sacc[kb][r] : kNegInf;
                }
            }
        }
        // P (rounded to T) as B operands; chunk c covers tile keys
        // 16c + 8(j/4) + 4hi + j%4. The row sum adds the rounded values.
        u32x4_t pf[NPC];
        auto weights = [&](float m_use, float sum) {
#pragma unroll
            for (int c = 0; c < NPC; ++c) {
                const int kb = c >> 1, r0 = 8 * (c & 1);
                float e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = sacc[kb][r0 + j];
                    e[j] = __builtin_amdgcn_exp2f(raw_max ? fmaf(x, cmul, -m_use) : x - m_use);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    pf[c][j] = T::pack2(e[2 * j], e[2 * j + 1]);
                    sum = dot2_ones<T>(pf[c][j], sum);
                }
            }
            return sum;
        };
        if (SM == 1) {   // x = s * scale + bias (masked s = -inf stays -inf: scale > 0)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[kb][r] = fmaf(sacc[kb][r], p.scale, bv[4 * kb + (r >> 2)][r & 3]);
        }
        if (SM == 2) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float sv = sacc[kb][r];
                    float x = sv == kNegInf ? kNegInf : sv * c2;   // masked stays -inf for any sign of c2
                    if (has_bias) x = fmaf(bv[4 * kb + (r >> 2)][r & 3], kLog2e, x);
                    sacc[kb][r] = x;
                }
            }
        }
        // the running max after the tile: the tile max when it exceeds m_run by
        // more than `slack`, else m_run; O and l are rescaled when it changes
        auto update_max = [&](float slack) {
            float mx = kNegInf;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
            if (raw_max) mx *= cmul;
            mx = pair_max(mx);
            const float m_new = mx > m_run + slack ? mx : m_run;
            if (__any(m_new != m_run)) {
                const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == kNegInf ? 0.f : m_new));
                l_run *= corr;
#pragma unroll
                for (int db = 0; db < DB; ++db) oacc[db] *= corr;
            }
            m_run = m_new;
        };
        if constexpr (kDeferMax) {
            if (reg_bias && it + AHEAD < n_kv_tiles) stage(it + AHEAD);
            float ts = weights(m_run == kNegInf ? 0.f : m_run, 0.f);
            if (__any(!(ts < kMaxTileSum) | ((m_run == kNegInf) & row_live))) {
                asm volatile("");
                update_max(0.f);
                ts = weights(m_run == kNegInf ? 0.f : m_run, 0.f);
            }
            l_run += ts;
        } else {
            update_max(kRescale);
            if (reg_bias && it + AHEAD < n_kv_tiles) stage(it + AHEAD);
            l_run = weights(m_run == kNegInf ? 0.f : m_run, l_run);
        }
        // O^T += V^T P^T; V^T operands are transposed reads of the row-major V tile
#pragma unroll
        for (int c = 0; c < NPC; ++c) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
                oacc[db] = mfma32<T>(tr_operand<DVL>(vtb, c, db), pf[c], oacc[db]);
        }
    }

    // Epilogue: lanes l and l^32 hold the two halves of one query's row sum.
    const float lt = pair_sum(l_run);
    if (wave_active && qrow < q_len) {
        const float inv = !(lt <= 0.f) ? 1.f / lt : 0.f;
        uint16_t* op = p.o + (int64_t)(qr.start + qrow) * ((int64_t)p.hq * DV) + (int64_t)head * DV + p.col0;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d = 32 * db + 8 * rg + 4 * hi;
                if (DO % 32 != 0 && d >= DO) continue;
                st8(op + d, u32x2_t{T::pack2(oacc[db][4 * rg + 0] * inv, oacc[db][4 * rg + 1] * inv),
                                    T::pack2(oacc[db][4 * rg + 2] * inv, oacc[db][4 * rg + 3] * inv)});
            }
        }
        if (p.lse != nullptr && hi == 0)
            p.lse[(int64_t)(qr.start + qrow) * p.hq + head] = !(lt <= 0.f) ? m_run * kLn2 + logf(lt) : kNegInf;
    }
}

int gcd_int(int a, int b) { while (b) { const int t = a % b; a = b; b = t; } return a; }

// CUs of the current device (cached per device; 256 if unknown)
int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

template <typename T, int DK, int DV, int DVL, int DO>
hipError_t launch_typed(const FwdArgs& a, hipStream_t st) {
    const Geometry& g = a.geo;
    FwdKParams p;
    p.q = (const uint16_t*)a.q; p.k = (const uint16_t*)a.k; p.v = (const uint16_t*)a.v;
    p.o = (uint16_t*)a.o; p.lse = a.lse;
    p.cu_q = g.cu_q; p.cu_kv = g.cu_kv; p.bias = g.bias;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs;
    p.bias_qs = g.bias_qs; p.bias_hs = g.bias_hs; p.bias_cols = g.bias_cols;
    p.bias_ss = g.bias_ss; p.bias_rows = g.bias_rows;
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.g = g.g;
    p.hpw = gcd_int(g.g, kWaves);
    const int QT = 32 * (kWaves / p.hpw);
    p.n_tiles = (int)(g.total_q / QT) + g.num_seqs + 1;
    p.n_hg = g.hq / p.hpw;
    p.scale = g.scale;
    p.scale_log2 = g.scale * kLog2e;
    p.causal = g.causal; p.window = g.window > 0 ? g.window : 0;
    p.bias_v4 = g.bias != nullptr && ((uintptr_t)g.bias % 16 == 0) && g.bias_qs % 4 == 0 && g.bias_hs % 4 == 0 &&
                (g.bias_ss < 0 || g.bias_ss % 4 == 0);
    const int64_t blocks = (int64_t)p.n_tiles * p.n_hg;
    if (blocks <= 0) return hipSuccess;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    // A head-broadcast bias whose rows are 16-byte aligned is staged in LDS
    // when a workgroup covers 32 or 64 query rows (the staged tile's byte
    // offsets, rows plus columns, stay below 2^32)
    int brows = 0;
    const int sm = !(p.scale_log2 > 0.f) ? 2 : g.bias != nullptr ? 1 : 0;
    if (DK <= 128 && sm == 1 && g.bias_hs == 0 && p.bias_v4 && g.bias_cols >= 4 && g.bias_cols % 4 == 0 &&
        (QT == 32 || QT == 64) && ((int64_t)QT * g.bias_qs + g.bias_cols) * 4 < ((int64_t)1 << 32))
        brows = QT;
    if constexpr ((DK == 128 && DVL == 128 && DO == 128) || (DK == 64 && DO == 64)) {
        // Small grids (at most two 8-wave workgroups per CU) run 4-wave
        // workgroups, two per CU, on a 2-deep ring (64 KB of LDS each at
        // D = 128), with at most 2 heads of a GQA group per workgroup: 3-25%
        // faster there (MHA and GQA shapes of 2-4 sequences of 2-4K; at
        // D = 64 causal only: non-causal GQA was 8% slower); on larger grids
        // the 8-wave workgroups, whose staged tiles serve twice the query
        // rows, are as fast or faster (C3 +1-4% with the 4-wave ones).
        if (sm == 0 && (DK == 128 || p.causal) && (g.total_q / QT) * p.n_hg <= 2 * (int64_t)device_cus()) {
            p.hpw = gcd_int(g.g, 2);
            const int QT4 = 32 * (4 / p.hpw);
            p.n_tiles = (int)(g.total_q / QT4) + g.num_seqs + 1;
            p.n_hg = g.hq / p.hpw;
            const int64_t blocks4 = (int64_t)p.n_tiles * p.n_hg;
            if (blocks4 > 0x7fffffff) return hipErrorInvalidValue;
            p.col0 = 0;
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 0, 0, 64, 4, 2>), dim3((unsigned)blocks4), dim3(256),
                               0, st, p);
            return hipGetLastError();
        }
    }
    if constexpr (DK > 128) {
        // The wide head dims take the whole output in one launch on 32-key
        // tiles (three 256-wide K + V stages fit the LDS), instead of
        // recomputing S for each output slice; a bias is loaded per row.
        // (D = 256 with a bias keeps the slices: one launch would spill.)
        if (sm == 0 || DV <= 192) {
            p.col0 = 0;
            p.lse = a.lse;
            if constexpr (DV <= 192) {
                if (sm == 2) {
                    hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DK, DV, 2, 0, 32>), dim3((unsigned)blocks),
                                       dim3(kThreads), 0, st, p);
                    return hipGetLastError();
                }
                if (sm == 1) {
                    hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DK, DV, 1, 0, 32>), dim3((unsigned)blocks),
                                       dim3(kThreads), 0, st, p);
                    return hipGetLastError();
                }
            }
            if constexpr (DV <= 192) {
                // D = 160: 64-key tiles on a 2-deep ring (246 VGPRs): 0.278
                // -> 0.258 ms at 2 x 4096 causal, 16/4 heads (at D = 256
                // they spill)
                hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DK, DV, 0, 0, 64, kWaves, 2>), dim3((unsigned)blocks),
                                   dim3(kThreads), 0, st, p);
                return hipGetLastError();
            }
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DK, DV, 0, 0, 32>), dim3((unsigned)blocks), dim3(kThreads),
                               0, st, p);
            return hipGetLastError();
        }
    }
    // DO < DV: one launch per DO-column slice; the first writes the LSE
    for (int c0 = 0; c0 < DV; c0 += DO) {
        p.col0 = c0;
        p.lse = c0 == 0 ? a.lse : nullptr;
        if constexpr (DK <= 128) {
            if (brows == 32) {
                hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 1, 32>), dim3((unsigned)blocks),
                                   dim3(kThreads), 0, st, p);
                continue;
            }
            if (brows == 64) {
                hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 1, 64>), dim3((unsigned)blocks),
                                   dim3(kThreads), 0, st, p);
                continue;
            }
        }
        if (sm == 2)
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 2>), dim3((unsigned)blocks), dim3(kThreads), 0,
                               st, p);
        else if (sm == 1)
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 1>), dim3((unsigned)blocks), dim3(kThreads), 0,
                               st, p);
        else if (DK == 128 && DVL == 128 && !(g.window > 0 && g.window < 1024))
            // 128-key tiles on a 2-deep ring (128 KB): the same keys ahead
            // as 64-key tiles three deep, half the barriers and per-tile
            // softmax bookkeeping (C3 forward 1.15-1.16 -> 1.10-1.13 ms on
            // one box, non-causal -4%, window 4096 -2%); a window below 1024
            // keys keeps 64-key tiles (the band's tile rounding costs more:
            // window 256 +7% with 128)
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 0, 0, (DK == 128 && DVL == 128) ? 128 : 64, kWaves,
                                                (DK == 128 && DVL == 128) ? 2 : 3>),
                               dim3((unsigned)blocks), dim3(kThreads), 0, st, p);
        else
            hipLaunchKernelGGL((fwd_mfma_kernel<T, DK, DV, DVL, DO, 0>), dim3((unsigned)blocks), dim3(kThreads), 0,
                               st, p);
    }
    return hipGetLastError();
}

}  // namespace

template <typename T>
hipError_t launch_dims(const FwdArgs& a, hipStream_t st) {
    switch (a.geo.d) {
        case 64: return launch_typed<T, 64, 64, 64, 64>(a, st);
        case 80: return launch_typed<T, 128, 80, 128, 80>(a, st);
        case 88: return launch_typed<T, 128, 88, 128, 88>(a, st);
        case 96: return launch_typed<T, 128, 96, 128, 96>(a, st);
        case 128: return launch_typed<T, 128, 128, 128, 128>(a, st);
        case 160: return launch_typed<T, 256, 160, 128, 80>(a, st);
        case 256: return launch_typed<T, 256, 256, 128, 128>(a, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_fwd_mfma(int dtype, const FwdArgs& a, hipStream_t st) {
    if (dtype == MTLATTN_DTYPE_BF16) return launch_dims<BF16>(a, st);
    if (dtype == MTLATTN_DTYPE_F16) return launch_dims<F16>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace mtlattn
