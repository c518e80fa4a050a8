// dK/dV for fp16/bf16 on gfx950 without a bias: one wave per SIMD, 64 keys
// per wave at the 128-wide tiles (head dims 80 to 128) and 32 at the 256-wide
// ones (head dim 256: one pass over all output columns; at 160 the wave-pair
// kernel, which holds all 160 columns, measured faster) -- counterpart of the
// reference's bwd_dkv_mpp, src/attn_mpp.metal:546-647 (instances 668-679);
// the arithmetic is that of bwd.hip's dK/dV kernels. Built with the
// compiler's MFMA results kept in VGPRs (-mllvm -amdgpu-mfma-vgpr-form,
// build.py): the dK / dV accumulators are pinned to the AGPRs by inline asm
// (mfma32_acc), and the S and dP products' results, which the VALU reads,
// stay in VGPRs.
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "bwd_common.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

// ---------------------------------------------------------------------------
// dK/dV without a bias: workgroups of 4 waves, one per SIMD (512 registers
// each), every wave computing all four products for its own NKB 32-key
// blocks (two at the 128-wide tiles, one at the 256-wide ones) in stages of
// 32 queries x 1 head.
//  * At 64 keys per wave each Q or dO operand read from LDS feeds the MFMAs
//    of both key blocks (0.5 KB of LDS per MFMA; the wave-pair kernel of
//    bwd.hip reads 1 KB). At 32 keys per wave and 256 columns the K^T and V^T
//    operands and the accumulators of all columns fill the registers, so S
//    and dP are computed once for all output columns (the wave-pair kernel
//    computes the 256 columns as two 128-column slices, each recomputing S
//    and dP).
//  * The K^T and V^T operands of the wave's keys stay in VGPRs; the dK / dV
//    accumulators (256 at D = 128 and D = 256) are pinned to the AGPRs
//    (mfma32_acc, inline asm), which is why this file is built with the
//    compiler's own MFMA results in VGPRs (build.py).
//  * Iteration j is a software pipeline over two stages: S, P, dP and dV of
//    stage j and dS and dK of stage j - 1, in four phases of 16 MFMAs (at
//    DV = 128 or 256), each written in issue order (one MFMA, its share of
//    another product's VALU work, an LDS read ahead; groups kept in order by
//    scheduling barriers), each phase's first operands read during the
//    previous phase's last products:
//      A. S(j)        beside the second half of dS(j - 1)
//      B. dK(j - 1)   beside the first half of P(j)
//      C. dP(j)       beside the second half of P(j)
//      D. dV(j)       beside the first half of dS(j) and stage j + 1's lse
//                     and delta columns turned into -lse log2 e and -delta
//  * Stages visit the query tiles top-down with the GQA group's heads inner,
//    as the other dK/dV kernels do (under a sliding window from the tile that
//    first_q_tile picks, wrapping to the top), on an LDS ring (Q, dO, and each wave's
//    own lse and delta columns; 5 slots of 18 KB or 4 of 34 KB): the loads
//    of stage j + NBUF - 2 go out between the products of iteration j, and
//    every wave waits for its own loads of stage j + 1 in phase C, then one
//    barrier per iteration.
//  * A workgroup takes key blocks b and nb - 1 - b of a sequence (nb
//    blocks): under causal masking every such pair is the same amount of
//    work, which keeps the in-order dispatch balanced (under a sliding window
//    one block: there every block but the last few has the same work).
// The arithmetic is that of the other dK/dV kernels: P and dS rounded to T,
// dS from the rounded P, masks as -inf logits (scale > 0, host-checked).
// ---------------------------------------------------------------------------
template <typename T, int D, int DV, int NKB, bool OUT_F32>
__global__ __launch_bounds__(256, 1) void bwd_dkv_wide_kernel(BwdKParams p) {
    static_assert((D == 128 && NKB == 2) || (D == 256 && NKB == 1), "128-wide tiles: 64 keys per wave; 256-wide: 32");
    constexpr int NW = 4, KPW = 32 * NKB;               // waves, keys per wave
    constexpr int DC = (DV + 15) / 16, DB = (DV + 31) / 32;
    constexpr int QTL = 32;                             // queries per stage
    constexpr int KB = NW * KPW;                        // keys per workgroup
    constexpr int TILE = QTL * D * 2;                   // 8 or 16 KB
    constexpr int LCOL = 64 * 4;                        // one lse / delta column (64 rows loaded)
    constexpr int SLOT = 2 * TILE + NW * 2 * LCOL;      // Q, dO, each wave's own lse and delta columns
    constexpr int NBUF = D == 128 ? 5 : 4;              // slots (90 or 136 KB)
    constexpr int AHEAD = NBUF - 2;                     // stages loading ahead
    __shared__ __attribute__((aligned(1024))) char smem[NBUF * SLOT];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31, hi = lane >> 5;
    const int L = xcd_remap(blockIdx.x, p.n_tiles * p.hkv);
    const int hk = L / p.n_tiles;
    const int t = L - hk * p.n_tiles;                  // early key blocks (heavier when causal) first
    // Tiles are pairs of key blocks, block pi and block nb - 1 - pi of a
    // sequence (nb blocks): with causal masking a pair's work is the same
    // for every pair, so the in-order dispatch of workgroups keeps the CUs
    // evenly loaded (single blocks, heaviest first per sequence, left each
    // XCD's last sequence's heavy blocks running alone at the end).
    // Under a sliding window every block but a sequence's last few has the
    // same work, and pairs would not be: tiles are then single blocks.
    const bool paired = p.window <= 0;
    const int TK = paired ? 2 * KB : KB;               // keys per tile
    const int s = find_seq_for_tile(p.cu_kv, p.num_seqs, TK, t, p.total_kv);
    const int tb = tile_base(p.cu_kv, s, TK, p.total_kv);
    if (t < tb) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    const int pi = t - tb;
    const int nb = (kv_len + KB - 1) / KB;
    if (pi >= (paired ? (nb + 1) / 2 : nb)) return;
    const int coff = kv_len - q_len;
    for (int bi = 0; bi < 2; ++bi) {
        const int blk = bi == 0 ? pi : nb - 1 - pi;
        if (bi == 1 && (!paired || blk == pi)) break;
        // the second block reloads the ring's slots: every wave is done with them
        if (bi == 1) __syncthreads();
        const int k0 = blk * KB;

        const int kw = k0 + KPW * w;                 // first key of this wave (seq-local)
        const bool wave_active = kw < kv_len;
        const int wk_last = min(kv_len, kw + KPW) - 1;

        // B operands of the S and dP products: K^T and V^T of both key blocks,
        // lane = key kw + 32 kb + l32, d = 16 kc + 8 hi + j (keys past the end
        // read the last key: masked; columns past DV are zero)
        u32x4_t kf[NKB][DC], vf[NKB][DC];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const int64_t grow = kr.start + min(kw + 32 * kb + l32, kv_len - 1);
            const uint16_t* kp = p.k + grow * p.k_rs + (int64_t)hk * DV + 8 * hi;
            const uint16_t* vp = p.v + grow * p.v_rs + (int64_t)hk * DV + 8 * hi;
#pragma unroll
            for (int kc = 0; kc < DC; ++kc) {
                const bool in = DV % 16 == 0 || 16 * kc + 8 * hi < DV;
                kf[kb][kc] = in ? ld16(kp + 16 * kc) : u32x4_t{};
                vf[kb][kc] = in ? ld16(vp + 16 * kc) : u32x4_t{};
            }
        }
        // settle the fragments here: the stage loop's own waits count only its
        // direct loads
        wait_vmcnt<0>();

        const int k_last_wg = min(kv_len, k0 + KB) - 1;
        const int q_lo = p.causal ? max(0, k0 - coff) / QTL * QTL : 0;
        const int q_hi = p.window > 0 ? min(q_len, k_last_wg - coff + p.window) : q_len;
        const int n_q_tiles = q_hi > q_lo ? (q_hi - q_lo + QTL - 1) / QTL : 0;
        const int n_stages = n_q_tiles * p.g;
        const int qt_first = first_q_tile(q_lo, n_q_tiles, QTL, p.window > 0);
        const int64_t cyc = (int64_t)n_q_tiles * QTL;        // rows of the walk's wrap

        // Direct loads of a stage: the Q and dO tiles by all four waves (two
        // 1 KB loads of each per wave), and every wave's own copy of the lse and
        // delta columns (one row per lane; rows past the stage are loaded but
        // never read), which the wave itself turns into -lse log2 e and -delta
        // once they land, with no barrier in between. Every stage issues the same
        // loads: past the last stage the loader cursor stays on it and reloads
        // it into the free slot, so the wait counts below are constants.
        using Stager = TileStager<D, QTL, NW, DV>;           // the tiles' load layout
        constexpr int LQ = Stager::N;                        // loads per wave per tile
        static_assert(Stager::PER % NW == 0, "whole tile loads per wave");
        constexpr int NL = 2 * LQ + 2;                       // loads per wave per stage
        int ld_st = 0, ld_hl = 0, ld_qt = qt_first, ld_slot = 0;
        const uint16_t* ld_q = p.q + (int64_t)(qr.start + qt_first) * p.q_rs + (int64_t)hk * p.g * DV;
        const uint16_t* ld_do = p.dout + (int64_t)(qr.start + qt_first) * p.do_rs + (int64_t)hk * p.g * DV;
        const int64_t l0 = (int64_t)(qr.start + qt_first) * p.hq + hk * p.g;
        const float* ld_l = p.lse + l0;
        const float* ld_d = p.delta + l0;
        const int wcol = 2 * TILE + w * 2 * LCOL;            // this wave's lse column in a slot (delta: + LCOL)
        const int64_t q_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.q_rs;
        const int64_t do_wrap = -(int64_t)(p.g - 1) * DV - (int64_t)QTL * p.do_rs;
        const int64_t l_wrap = -(int64_t)(p.g - 1) - (int64_t)QTL * p.hq;
        // The cursor's stage: its LDS slot, the last row that exists (rows
        // past the sequence end read it) and a per-stage copy of the lane
        // index. Each load computes its own per-lane offset from that copy
        // right before it is issued: a few VALU operations between the
        // products, where offsets kept from the start would be loop-invariant
        // registers that the allocator spills (the empty asm keeps the
        // compiler from hoisting them out of the loop).
        char* lbuf = smem;
        int ld_rmax = 0, ln = lane;
        auto prep = [&]() {
            lbuf = smem + ld_slot * SLOT;
            ld_rmax = min(q_len - ld_qt, QTL) - 1;           // >= 0
            ln = lane;
            asm volatile("" : "+v"(ln));
        };
        // load j of the cursor's stage: 0 .. LQ - 1 Q, LQ .. 2 LQ - 1 dO, then
        // this wave's lse and delta columns
        auto load = [&](int j) {
            if (j < 2 * LQ) {
                const int i = w + (j % LQ) * NW;
                const int r = min(Stager::row_of(i, ln), ld_rmax);
                if (j < LQ)
                    lds_dma16s(ld_q, Stager::lane_off(i, ln, r, (uint32_t)(2 * p.q_rs)), lbuf + i * 1024);
                else
                    lds_dma16s(ld_do, Stager::lane_off(i, ln, r, (uint32_t)(2 * p.do_rs)), lbuf + TILE + i * 1024);
            } else {
                const uint32_t lvo = (uint32_t)min(ln, ld_rmax) * (uint32_t)p.hq * 4u;
                if (j == 2 * LQ)
                    lds_dma4s(ld_l, lvo, lbuf + wcol);
                else
                    lds_dma4s(ld_d, lvo, lbuf + wcol + LCOL);
            }
        };
        // next slot; the source moves on only while stages remain
        auto advance = [&]() {
            ld_slot = ld_slot == NBUF - 1 ? 0 : ld_slot + 1;
            if (ld_st + 1 >= n_stages) return;
            ++ld_st;
            if (++ld_hl == p.g) {
                ld_hl = 0;
                ld_qt -= QTL;
                ld_q += q_wrap;
                ld_do += do_wrap;
                ld_l += l_wrap;
                ld_d += l_wrap;
                if (ld_qt < q_lo) {   // wrap to the top tile (first_q_tile)
                    ld_qt += (int)cyc;
                    ld_q += cyc * p.q_rs;
                    ld_do += cyc * p.do_rs;
                    ld_l += cyc * p.hq;
                    ld_d += cyc * p.hq;
                }
            } else {
                ld_q += DV;
                ld_do += DV;
                ld_l += 1;
                ld_d += 1;
            }
        };
        static_assert((AHEAD - 1) * NL < 64, "vmcnt range");
        // this wave's lse and delta columns of stage slot `slot` become -lse
        // log2 e and -delta (lane = row; the wave's own loads, landed): read
        // in one phase, written back in the next
        auto fix_cols = [&](int slot) {
            float* c = reinterpret_cast<float*>(smem + slot * SLOT + wcol) + lane;
            neg_col(c, 0);
            neg_col(c + 64, 1);
        };
        // (in the loop: the lane from the per-stage copy, so that no
        // loop-invariant address is kept, and spilled, across the stages)
        auto fix_read = [&](int slot, float& lv, float& dv) {
            const float* c = reinterpret_cast<const float*>(smem + slot * SLOT + wcol) + ln;
            lv = c[0];
            dv = c[64];
        };
        auto fix_write = [&](int slot, float lv, float dv) {
            float* c = reinterpret_cast<float*>(smem + slot * SLOT + wcol) + ln;
            c[0] = neg_lse2(lv);
            c[64] = -dv;
        };

        const uint32_t rbase = row_base<D>(l32, hi), tbase = tr_base<D>(lane);
        const float c2 = p.scale_log2;
        f32x16_t accv[NKB][DB], acck[NKB][DB];       // dV^T, dK^T of the wave's key blocks
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int db = 0; db < DB; ++db) accv[kb][db] = acck[kb][db] = f32x16_t{};

        Band band[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) band[kb] = query_band(kw + 32 * kb + l32, coff, q_len, kv_len, p.causal, p.window);

        // Compute cursor: stage j (its slot and first query) and the slot of
        // stage j - 1. Iteration j computes S, P, dP and dV of stage j and dS
        // and dK of stage j - 1, in four phases of one MFMA stream each with
        // the VALU work of another product beside it:
        //   A. S(j)        beside half of dS(j - 1) = P (dP - delta), rounded to T
        //   B. dK(j - 1)   beside half of P(j) = exp2(S c - lse'), rounded to T
        //   C. dP(j)       beside the other half of P(j)
        //   D. dV(j)       beside the other half of dS(j)
        // P(j) (packed) and dP(j) - delta stay in registers into iteration
        // j + 1. The loads of stage j + AHEAD go out during phases A (Q),
        // B (dO) and C (lse and delta).
        int c_hl = 0, c_qt = qt_first, c_slot = 0, p_slot = 0;
        u32x4_t pk[NKB][2];                      // P of the stage in flight, rounded to T (B operands of dV)
        f32x16_t pacc[NKB];                      // its dP - delta
        f32x16_t sacc[NKB];
        u32x4_t dsk[NKB][2];                     // dS of the previous stage, rounded to T (B operands of dK)
        constexpr int NS = NKB * DC;             // S or dP products per stage
        constexpr int NP = 2 * DB * NKB;         // dV or dK products per stage
        // operands read ahead: eight MFMAs' worth at 64 keys per wave, four
        // row or six transposed operands at 32
        constexpr int RPF = NKB == 2 ? 2 : 4, TPF = NKB == 2 ? 4 : 6;
        static_assert(DC >= RPF && 2 * DB >= TPF && NS >= 4 && NP >= 4, "prefetch depths");
        constexpr int HP = 4 * NKB;              // dS or P pairs per half stage
        // n loads from `first` spread over a phase of `groups` MFMA groups
        auto loads_at = [&](int i, int groups, int first, int n) {
#pragma unroll
            for (int k = 0; k < n; ++k)
                if (i == 1 + k * groups / n) load(first + k);
        };
        // Does any (query, key) of stage j fall outside the band? (the per-block
        // tests of the other kernels over this wave's keys)
        auto stage_needs_mask = [&]() {
            return (kw + KPW > kv_len) | (c_qt + QTL > q_len) | ((p.causal != 0) & (wk_last > c_qt + coff)) |
                   ((p.window > 0) & (kw < min(q_len, c_qt + QTL) + coff - p.window));
        };
        // pair pr = 0 .. 8 NKB - 1 of a stage's 16 NKB elements per lane: key
        // block pr / 8, rows 2 (pr % 8) and 2 (pr % 8) + 1; the first half
        // stage is pairs 0 .. HP - 1
        // Inside the phases each pair runs as a short pipeline over
        // consecutive MFMA groups -- P: the exponents' FMAs, the
        // exponentials, the rounding to T; dS: the products, the rounding --
        // so no group waits for a result computed in the same group (the
        // exponential's latency alone is most of an MFMA's 32 cycles).
        float xt[8 * NKB][2];                    // pairs between their steps
        auto exp_fma = [&](int pr, const f32x16_t& nl) {
            const int kb = pr >> 3, r0 = 2 * (pr & 7);
            xt[pr][0] = fmaf(sacc[kb][r0], c2, nl[r0]);
            xt[pr][1] = fmaf(sacc[kb][r0 + 1], c2, nl[r0 + 1]);
        };
        auto exp_exp = [&](int pr) {
            xt[pr][0] = __builtin_amdgcn_exp2f(xt[pr][0]);
            xt[pr][1] = __builtin_amdgcn_exp2f(xt[pr][1]);
        };
        auto exp_pack = [&](int pr) {
            const int kb = pr >> 3, r0 = 2 * (pr & 7);
            pk[kb][r0 >> 3][(r0 & 7) >> 1] = T::pack2(xt[pr][0], xt[pr][1]);
        };
        auto exp_pair = [&](int pr, const f32x16_t& nl) {
            exp_fma(pr, nl);
            exp_exp(pr);
            exp_pack(pr);
        };
        auto ds_mul = [&](int pr) {
            const int kb = pr >> 3, r0 = 2 * (pr & 7);
            const uint32_t wv = pk[kb][r0 >> 3][(r0 & 7) >> 1];
            xt[pr][0] = lo16<T>(wv) * pacc[kb][r0];
            xt[pr][1] = hi16<T>(wv) * pacc[kb][r0 + 1];
        };
        // (the empty asm keeps each pair in the phase it is written in: left
        // alone, the compiler moves the pairs next to their use, the dK
        // products, where they run serially)
        auto ds_pack = [&](int pr) {
            const int kb = pr >> 3, r0 = 2 * (pr & 7);
            uint32_t d = T::pack2(xt[pr][0], xt[pr][1]);
            asm volatile("" : "+v"(d));
            dsk[kb][r0 >> 3][(r0 & 7) >> 1] = d;
        };
        auto ds_pair = [&](int pr) {
            ds_mul(pr);
            ds_pack(pr);
        };
        // the steps of pairs first .. first + HP - 1 due in group i of a phase
        // of n groups (pair h starts in group h n / HP; a P pair's rounding
        // past the phase's last group runs after it: ps_tail)
        auto ps_exp = [&](int i, int n, int first, const f32x16_t& nl) {
#pragma unroll
            for (int h = 0; h < HP; ++h) {
                const int g0 = h * n / HP;
                if (i == g0) exp_fma(first + h, nl);
                if (i == g0 + 1) exp_exp(first + h);
                if (i == g0 + 2) exp_pack(first + h);
            }
        };
        auto ps_tail = [&](int n, int first) {
#pragma unroll
            for (int h = 0; h < HP; ++h) {
                const int g0 = h * n / HP;
                if (g0 + 1 >= n) exp_exp(first + h);
                if (g0 + 2 >= n) exp_pack(first + h);
            }
        };
        auto ps_ds = [&](int i, int n, int first) {
#pragma unroll
            for (int h = 0; h < HP; ++h) {
                const int g0 = h * n / HP;
                if (i == g0) ds_mul(first + h);
                if (i == (g0 + 1 < n ? g0 + 1 : n - 1)) ds_pack(first + h);
            }
        };
        // (the lane half from the per-stage lane copy: see prep)
        auto read_col = [&](const char* slot, int which) {   // 16 rows of this wave's column, C layout
            const float* c = reinterpret_cast<const float*>(slot + wcol + which * LCOL);
            f32x16_t x;
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(c + 8 * rg + 4 * (ln >> 5));
#pragma unroll
                for (int e = 0; e < 4; ++e) x[4 * rg + e] = v4[e];
            }
            return x;
        };

        // Each phase's first operands are read during the previous phase's
        // last products, so no phase starts by waiting for the LDS (phase A's
        // Q rows excepted: the barrier before it publishes them).
        auto iter = [&](auto first_t, auto last_t, bool masked, int n_slot) {
            constexpr bool FIRST = decltype(first_t)::value, LAST = decltype(last_t)::value;
            const char* Qc = smem + c_slot * SLOT;   // stage j
            const char* Qp = smem + p_slot * SLOT;   // stage j - 1
            const char* qtb = opaque(Qp + tbase);    // B: Q^T of stage j - 1
            const char* drb = opaque(Qc + TILE + rbase);   // C: dO rows of stage j
            const char* dtb = opaque(Qc + TILE + tbase);   // D: dO^T of stage j
            f32x16_t nl;                             // -lse log2(e) of stage j's rows
            f32x16_t dinit;                          // -delta of stage j's rows
            u32x4_t tq[2 * DB], da[DC], td[2 * DB];  // operands of B, C, D
            float fl = 0.f, fd = 0.f;                // stage j + 1's lse and delta (this wave's rows)
            auto read_tq = [&](int i) { tq[i] = tr_operand<D>(qtb, i / DB, i % DB); };
            auto read_td = [&](int i) { td[i] = tr_operand<D>(dtb, i / DB, i % DB); };
            // A. S(j) beside the second half of dS(j - 1); the loads of stage
            //    j + AHEAD start (Q); B's first operands are read at the end
            if constexpr (!LAST) {
                const char* qrb = opaque(Qc + rbase);
                u32x4_t qa[DC];
#pragma unroll
                for (int i = 0; i < RPF; ++i) qa[i] = row_operand<D>(qrb, i, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int kc = 0; kc < DC; ++kc) {
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int i = NKB * kc + kb;
                        sacc[kb] = mfma32<T>(qa[kc], kf[kb][kc], kc == 0 ? f32x16_t{} : sacc[kb]);
                        __builtin_amdgcn_sched_barrier(0);   // the MFMA first in its group
                        if (kb == NKB - 1 && kc + RPF < DC) qa[kc + RPF] = row_operand<D>(qrb, kc + RPF, 0);
                        loads_at(i, NS, 0, LQ);
                        if constexpr (!FIRST) {
                            ps_ds(i, NS, HP);
                            if (i == NS - 2)
#pragma unroll
                                for (int t = 0; t < TPF / 2; ++t) read_tq(t);
                            if (i == NS - 1)
#pragma unroll
                                for (int t = TPF / 2; t < TPF; ++t) read_tq(t);
                        }
                        if (i == NS - 3) nl = read_col(Qc, 0);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                // out-of-band logits -> -inf (P = exp2(-inf) = 0; scale > 0 is
                // host-checked); a real branch, taken by the stages on a band edge
                if (masked) {
                    asm volatile("");
                    const int qb0 = c_qt + 4 * (ln >> 5);
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int d0 = qb0 - band[kb].lo;
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            sacc[kb][r] = (uint32_t)(d0 + 8 * (r >> 2) + (r & 3)) < band[kb].width ? sacc[kb][r] : kNegInf;
                    }
                }
            } else {
#pragma unroll
                for (int h = 0; h < HP; ++h) ds_pair(HP + h);
#pragma unroll
                for (int i = 0; i < TPF; ++i) read_tq(i);
            }
            // B. dK(j - 1) beside the first half of P(j) (the dK and dV products
            //    are inline asm with their own hazard wait, mfma32_acc); C's
            //    first operands are read at the end
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!FIRST) {
#pragma unroll
                for (int i2 = 0; i2 < 2 * DB; ++i2) {
                    const int qc = i2 / DB, db = i2 % DB;
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int i = NKB * i2 + kb;
                        mfma32_acc<T>(acck[kb][db], tq[i2], dsk[kb][qc]);
                        __builtin_amdgcn_sched_barrier(0);
                        if (kb == NKB - 1 && i2 + TPF < 2 * DB) read_tq(i2 + TPF);
                        if constexpr (!LAST) {
                            loads_at(i, NP, LQ, LQ);
                            ps_exp(i, NP, 0, nl);
                            if (i == NP - 4) dinit = read_col(Qc, 1);
                            if (i == NP - 2)
#pragma unroll
                                for (int r = 0; r < RPF / 2; ++r) da[r] = row_operand<D>(drb, r, 0);
                            if (i == NP - 1)
#pragma unroll
                                for (int r = RPF / 2; r < RPF; ++r) da[r] = row_operand<D>(drb, r, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if constexpr (!LAST) ps_tail(NP, 0);
            } else {
#pragma unroll
                for (int k = 0; k < LQ; ++k) load(LQ + k);
#pragma unroll
                for (int h = 0; h < HP; ++h) exp_pair(h, nl);
                dinit = read_col(Qc, 1);
#pragma unroll
                for (int r = 0; r < RPF; ++r) da[r] = row_operand<D>(drb, r, 0);
            }
            if constexpr (!LAST) {
                // C. dP(j) onto -delta beside the second half of P(j); at the end,
                //    D's first operands and the columns of stage j + 1 (this
                //    wave's own loads of that stage have landed once at most
                //    the two later stages' loads are in flight)
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int kc = 0; kc < DC; ++kc) {
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int i = NKB * kc + kb;
                        pacc[kb] = mfma32<T>(da[kc], vf[kb][kc], kc == 0 ? dinit : pacc[kb]);
                        __builtin_amdgcn_sched_barrier(0);
                        if (kb == NKB - 1 && kc + RPF < DC) da[kc + RPF] = row_operand<D>(drb, kc + RPF, 0);
                        loads_at(i, NS, 2 * LQ, 2);
                        ps_exp(i, NS, HP, nl);
                        if (i == NS - 3) {
                            wait_vmcnt<(AHEAD - 1) * NL>();
                            fix_read(n_slot, fl, fd);
                        }
                        if (i == NS - 2)
#pragma unroll
                            for (int t = 0; t < TPF / 2; ++t) read_td(t);
                        if (i == NS - 1)
#pragma unroll
                            for (int t = TPF / 2; t < TPF; ++t) read_td(t);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                ps_tail(NS, HP);
                // D. dV(j) beside the first half of dS(j) (the second follows in
                //    the next iteration's phase A); stage j + 1's columns written
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i2 = 0; i2 < 2 * DB; ++i2) {
                    const int qc = i2 / DB, db = i2 % DB;
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int i = NKB * i2 + kb;
                        mfma32_acc<T>(accv[kb][db], td[i2], pk[kb][qc]);
                        __builtin_amdgcn_sched_barrier(0);
                        if (kb == NKB - 1 && i2 + TPF < 2 * DB) read_td(i2 + TPF);
                        if (i == 2) fix_write(n_slot, fl, fd);
                        ps_ds(i, NP, 0);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
        };
        // next compute stage: slots and first query
        auto step = [&](int n_slot) {
            p_slot = c_slot;
            c_slot = n_slot;
            if (++c_hl == p.g) {
                c_hl = 0;
                c_qt -= QTL;
                if (c_qt < q_lo) c_qt += (int)cyc;
            }
        };

        if (n_stages > 0) {
#pragma unroll
            for (int i = 0; i < AHEAD; ++i) {
                prep();
#pragma unroll
                for (int l = 0; l < NL; ++l) load(l);
                advance();
            }
            wait_vmcnt<(AHEAD - 1) * NL>();   // the K tile and stage 0
            fix_cols(0);
            __syncthreads();
            // every wave's loads of stage j + 1 have landed by the end of
            // iteration j (each waited for its own in phase C): the barrier
            // after it publishes them
            int n_slot = c_slot == NBUF - 1 ? 0 : c_slot + 1;
            prep();
            iter(std::true_type{}, std::false_type{}, stage_needs_mask(), n_slot);
            advance();
            __syncthreads();
            step(n_slot);
            for (int j = 1; j < n_stages; ++j) {
                n_slot = c_slot == NBUF - 1 ? 0 : c_slot + 1;
                prep();
                iter(std::false_type{}, std::false_type{}, stage_needs_mask(), n_slot);
                advance();
                __syncthreads();
                step(n_slot);
            }
            iter(std::false_type{}, std::true_type{}, false, 0);
            // The last accumulating MFMAs' results settle before anything reads
            // the accumulators (the compiler does not track the inline-asm
            // MFMAs, and may copy accumulators out at the end of this block):
            // these asm statements take every accumulator as an operand, the
            // first one after 32 wait states, so no read can come earlier.
            asm volatile("s_nop 15\n\ts_nop 15" : "+a"(acck[0][0]));
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    if (kb + db > 0) asm volatile("" : "+a"(acck[kb][db]));
                    asm volatile("" : "+a"(accv[kb][db]));
                }
        }
        // the reloads issued past the last stage land before the wave ends
        wait_vmcnt<0>();

        if (wave_active) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const int key = kw + 32 * kb + l32;
                if (key >= kv_len) continue;
                const int64_t off = (int64_t)(kr.start + key) * ((int64_t)p.hkv * DV) + (int64_t)hk * DV;
#pragma unroll
                for (int db = 0; db < DB; ++db) {
#pragma unroll
                    for (int rg = 0; rg < 4; ++rg) {
                        const int d = 32 * db + 8 * rg + 4 * hi;
                        if (DV % 32 != 0 && d >= DV) continue;
                        store4<T, OUT_F32>(p.dv, off + d, accv[kb][db][4 * rg], accv[kb][db][4 * rg + 1],
                                           accv[kb][db][4 * rg + 2], accv[kb][db][4 * rg + 3]);
                        store4<T, OUT_F32>(p.dk, off + d, acck[kb][db][4 * rg] * p.scale,
                                           acck[kb][db][4 * rg + 1] * p.scale, acck[kb][db][4 * rg + 2] * p.scale,
                                           acck[kb][db][4 * rg + 3] * p.scale);
                    }
                }
            }
        }
    }
}


template <typename T, int D, int DV, bool OUT_F32>
hipError_t launch_wide(const BwdArgs& a, hipStream_t st) {
    constexpr int NKB = D == 128 ? 2 : 1, KB = 4 * 32 * NKB;
    BwdKParams p = make_params(a);
    // pairs of key blocks (single blocks under a sliding window)
    const int tk = a.geo.window > 0 ? KB : 2 * KB;
    p.n_tiles = (int)(a.geo.total_kv / tk) + a.geo.num_seqs + 1;
    const int64_t blocks = (int64_t)p.n_tiles * a.geo.hkv;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((bwd_dkv_wide_kernel<T, D, DV, NKB, OUT_F32>), dim3((unsigned)blocks), dim3(256), 0, st, p);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_wide_dims(const BwdArgs& a, hipStream_t st) {
    const bool f = a.out_f32 != 0;
    switch (a.geo.d) {
        case 80: return f ? launch_wide<T, 128, 80, true>(a, st) : launch_wide<T, 128, 80, false>(a, st);
        case 88: return f ? launch_wide<T, 128, 88, true>(a, st) : launch_wide<T, 128, 88, false>(a, st);
        case 96: return f ? launch_wide<T, 128, 96, true>(a, st) : launch_wide<T, 128, 96, false>(a, st);
        case 128: return f ? launch_wide<T, 128, 128, true>(a, st) : launch_wide<T, 128, 128, false>(a, st);
        case 256: return f ? launch_wide<T, 256, 256, true>(a, st) : launch_wide<T, 256, 256, false>(a, st);
        default: return hipErrorNotSupported;
    }
}

// MTLATTN_DKV_WIDE=0 turns this kernel off (the wave-pair kernel of bwd.hip
// then runs these head dims): for A/B measurements.
bool wide_enabled() {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("MTLATTN_DKV_WIDE");
        v = (e == nullptr || e[0] != '0') ? 1 : 0;
    }
    return v != 0;
}

}  // namespace

// hipErrorNotSupported: not this kernel's problem (a bias, another head dim,
// row strides whose 256-row K tile offsets would pass 32 bits); the caller
// runs another kernel.
hipError_t launch_bwd_dkv_wide(int type_code, const BwdArgs& a, hipStream_t st) {
    // (scale > 0: the masks enter as -inf initial S accumulators, which a
    // negative scale would turn into +inf logits)
    if (a.geo.bias != nullptr || !(a.geo.scale > 0.f) || !wide_enabled()) return hipErrorNotSupported;
    if (a.k_rs <= 0 || a.k_rs >= ((int64_t)1 << 23) || a.q_rs >= ((int64_t)1 << 25) || a.do_rs >= ((int64_t)1 << 25))
        return hipErrorNotSupported;
    if (type_code == BF16::code) return launch_wide_dims<BF16>(a, st);
    if (type_code == F16::code) return launch_wide_dims<F16>(a, st);
    return hipErrorNotSupported;
}

}  // namespace mtlattn
