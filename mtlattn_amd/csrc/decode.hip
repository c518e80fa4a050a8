// Split-KV decode for fp16/bf16 on gfx950 (counterpart of the reference's
// attn_vl_split + attn_combine, src/attn_mpp.metal:384-535, redesigned).
//
// Decode is HBM-bound: the design goal is to read every K/V byte exactly once.
//   * GQA packing: the q_len x (heads of one GQA group) query rows that share
//     a kv head form the N dimension (16) of v_mfma_f32_16x16x32, so each K/V
//     row is read once per kv head instead of once per query head (the
//     reference's grid z = Hq re-reads it g times, src/ext.mm:760-761).
//   * One wave = one work item: a KV range of one (sequence, kv head, head
//     group). The automatic path cuts every sequence into fixed-length KV
//     chunks numbered without a host sync (slot = cu_kv[s] / C + s + chunk
//     index, as the prefill tiles are), so every wave streams the same number
//     of bytes whatever the spread of KV lengths; the explicit num_splits entry
//     cuts each sequence into that many equal parts instead. Waves never
//     synchronise with each other, so a workgroup is just 4 independent waves.
//     The kv head varies fastest over the wave index: the Hkv waves of one
//     item start together and read whole K/V rows (all heads) between them,
//     rather than one head's 2*D bytes of each row (1.6% faster at C5).
//   * Per 32-key tile: K goes straight from HBM into MFMA A-operand registers
//     (16 B per lane); V is loaded coalesced and transposed through a per-wave
//     LDS buffer for the P.V product. The next tile's loads are issued before
//     the current tile is computed.
//   * Each work item writes a normalised fp32 partial O and its LSE (16 rows
//     of its group); the combine kernel merges a sequence's items with LSE
//     weights and, unlike the reference's (src/attn_mpp.metal:498-521), also
//     writes the final LSE.
//   * Sliding window and additive bias, which the reference keeps off this
//     path (src/ext.mm:372-374): with a window the equal splits cover only
//     the keys some row of the sequence can see (from coff - W + 1, rounded
//     down to a tile), and elements below a row's band are masked; the fp32
//     bias of the lane's row and keys is loaded with the K/V tile it belongs
//     to and added as bias * log2 e (columns at or past bias_cols read as 0).
//   * Paged KV (no counterpart in the reference): K/V may live in pages of a
//     cache, [num_pages, page_size, Hkv, D], logical key j of sequence s in
//     page block_table[s][j / page_size]. page_size is a multiple of 16 and
//     tiles start at multiples of 32, so each 16-key block lies in one page:
//     two wave-uniform page lookups per tile (clamped to the cache) replace
//     the contiguous row base.
#include "common.h"
#include "kernels.h"
#include "../../include/mtlattn_capi.h"

namespace mtlattn {

namespace {

constexpr int kDecWaves = 4;
constexpr int kDecKT = 32;      // keys per tile

// Work items: chunk > 0 -> fixed KV chunks, slot = cu_kv[s] / chunk + s + c
// (n_slots = total_kv / chunk + num_seqs + 1); chunk == 0 -> ns equal splits
// per sequence, slot = s * ns + split (n_slots = num_seqs * ns). Partials of
// item `slot` for kv head hk and head group hgi live at row
// ((hk * n_hg + hgi) * n_slots + slot) * 16 + n (n = 16-row group row).
struct DecKParams {
    const uint16_t* q; const uint16_t* k; const uint16_t* v;
    float* o_part; float* lse_part;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs;
    int64_t bias_qs, bias_hs, bias_cols, bias_ss, bias_rows;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, hpb, n_hg, ns, chunk, n_slots;
    float scale_log2;
    int causal, window;
    int bias_v4;      // bias rows 16-byte aligned (pointer and strides)
    // paged KV (PAGED kernels): block table rows of bt_stride page indices
    const int* block_table;
    int64_t bt_stride;
    int page_size, num_pages;
};

// KV range [ks, ke) of work item `slot` of sequence s (false: no keys).
__device__ inline bool item_range(const DecKParams& p, int slot, int& s, int& ks, int& ke) {
    int kv_len;
    if (p.chunk > 0) {
        s = find_seq_for_tile(p.cu_kv, p.num_seqs, p.chunk, slot, p.total_kv);
        const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
        kv_len = kr.end - kr.start;
        ks = (slot - tile_base(p.cu_kv, s, p.chunk, p.total_kv)) * p.chunk;
        ke = min(kv_len, ks + p.chunk);
    } else {
        s = slot / p.ns;
        const int split = slot - s * p.ns;
        const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
        kv_len = kr.end - kr.start;
        // with a window, split only the keys the sequence's rows can see
        int lo = 0;
        if (p.window > 0) {
            const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
            lo = max(0, kv_len - (qr.end - qr.start) - p.window + 1) / kDecKT * kDecKT;
        }
        int c = (kv_len - lo + p.ns - 1) / p.ns;
        c = (c + kDecKT - 1) / kDecKT * kDecKT;
        ks = lo + split * c;
        ke = min(kv_len, ks + c);
    }
    return ke > ks;
}

// V^T tile [D][32] (64 B per row); 8-byte groups XOR-swizzled by row.
__device__ inline uint32_t dec_tr_offset(int row, int group) {
    const int f = ((row >> 1) ^ (row >> 3)) & 7;
    return (uint32_t)(row * 64 + ((group ^ f) << 3));
}

template <typename T, int D, bool BIAS, bool PAGED>
__global__ __launch_bounds__(kDecWaves * 64) void decode_split_kernel(DecKParams p) {
    constexpr int KC = D / 32;          // 32-wide k-chunks over D (QK^T)
    constexpr int DB = D / 16;          // 16-row output blocks over D
    constexpr int VU = D / 64;          // (4 keys x 8 d) units per lane per tile: (8 * D/8) / 64
    __shared__ __attribute__((aligned(16))) char smem[kDecWaves * D * kDecKT * 2];

    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int n16 = lane & 15, lg = lane >> 4;
    char* vt = smem + w * (D * kDecKT * 2);

    int wid = blockIdx.x * kDecWaves + w;
    const int hk = wid % p.hkv; wid /= p.hkv;
    const int hgi = wid % p.n_hg;
    const int slot = wid / p.n_hg;
    if (slot >= p.n_slots) return;
    int s, ks, ke;
    const bool has_keys = item_range(p, slot, s, ks, ke);
    // fixed chunks past a sequence's end are not read by the combine
    if (!has_keys && p.chunk > 0) return;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int q_len = qr.end - qr.start, kv_len = kr.end - kr.start;
    if (q_len == 0) return;
    const int coff = kv_len - q_len;

    // Row n of the N dimension: head hh = n / q_len of this group, query qi = n % q_len.
    const int rows = p.hpb * q_len;
    const bool row_ok = n16 < rows && n16 < 16;
    const int hh = row_ok ? n16 / q_len : 0;
    const int qi = row_ok ? n16 - hh * q_len : 0;
    const int head = hk * p.g + hgi * p.hpb + hh;
    const int64_t grow = qr.start + qi;

    u32x4_t qf[KC];
    {
        const uint16_t* qp = p.q + grow * p.q_rs + (int64_t)head * D + 8 * lg;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) qf[kc] = ld16(qp + 32 * kc);
    }

    const int n_tiles = has_keys ? (ke - ks + kDecKT - 1) / kDecKT : 0;

    // K/V rows: the sequence's contiguous rows, or cache rows through pages
    const uint16_t* kbase = p.k + (PAGED ? 0 : (int64_t)kr.start * p.k_rs) + (int64_t)hk * D;
    const uint16_t* vbase = p.v + (PAGED ? 0 : (int64_t)kr.start * p.v_rs) + (int64_t)hk * D;
    const int* bt = PAGED ? p.block_table + (int64_t)s * p.bt_stride : nullptr;
    // cache row of logical key `key` (wave-uniform): the table column is
    // clamped to the row's bt_stride entries and the page index to the cache
    auto page_row = [&](int key) -> int64_t {
        const int col = min(key / p.page_size, (int)min(p.bt_stride, (int64_t)0x7fffffff) - 1);
        const int pg = min(max(bt[col], 0), p.num_pages - 1);
        return (int64_t)pg * p.page_size + key % p.page_size;
    };

    // this lane's bias row (head of the row, or the broadcast head)
    const float* brow = nullptr;
    if (BIAS)
        brow = p.bias + bias_row_offset(grow, s, qr.start, p.bias_qs, p.bias_ss, p.bias_rows) +
               (int64_t)head * p.bias_hs;

    // Register tiles: K A-operands [2 key blocks][KC], V rows [VU units][4 keys],
    // bias of the lane's row for its 8 keys.
    u32x4_t ka[2][KC], vr[VU][4];
    float bb[2][4];
    auto load = [&](int kt, u32x4_t (&ka_)[2][KC], u32x4_t (&vr_)[VU][4], float (&bb_)[2][4]) {
        // row of a (clamped, < ke) key of this tile: keys [kt, kt + 16) lie
        // in the page of kt, keys [kt + 16, ke) in the page of kt + 16
        int64_t r0 = 0, r1 = 0;
        if (PAGED) {
            r0 = page_row(kt);
            r1 = page_row(min(kt + 16, ke - 1));
        }
        auto row = [&](int key) -> int64_t {
            if (!PAGED) return key;
            return key < kt + 16 ? r0 + (key - kt) : r1 + (key - (kt + 16));
        };
        if (BIAS) {
            // the lane's 4 keys of a 16-key block are contiguous: one 16-byte
            // load each when the whole tile lies within the bias columns
            if (p.bias_v4 && kt + kDecKT <= p.bias_cols) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const f32x4_t b4 = *reinterpret_cast<const f32x4_t*>(brow + kt + 16 * mb + 4 * lg);
#pragma unroll
                    for (int r = 0; r < 4; ++r) bb_[mb][r] = b4[r];
                }
            } else {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = kt + 16 * mb + 4 * lg + r;
                        const float b = brow[min(key, (int)p.bias_cols - 1)];
                        bb_[mb][r] = key < p.bias_cols ? b : 0.f;
                    }
            }
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            // keys past the split end read its last key: finite, masked to P = 0
            const int key = min(kt + 16 * mb + n16, ke - 1);
            const uint16_t* kp = kbase + row(key) * p.k_rs + 8 * lg;
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) ka_[mb][kc] = ld16(kp + 32 * kc);
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int uid = lane + 64 * u;
            const int dc = uid % (D / 8), kg = uid / (D / 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = min(kt + 4 * kg + i, ke - 1);
                vr_[u][i] = ld16(vbase + row(key) * p.v_rs + 8 * dc);
            }
        }
    };

    float m_run = kNegInf, l_run = 0.f;
    f32x4_t oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Two register sets alternate: tile it is computed from set it % 2 while
    // the loads of tiles it + 1 and it + 2 are in flight.
    u32x4_t ka2[2][KC], vr2[VU][4];
    float bb2[2][4];
    auto step = [&](int it, u32x4_t (&ka)[2][KC], u32x4_t (&vr)[VU][4], float (&bb)[2][4])
                    __attribute__((always_inline)) {
        const int kt = ks + it * kDecKT;
        // stage V^T of this tile in the wave's LDS buffer
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int uid = lane + 64 * u;
            const int dc = uid % (D / 8), kg = uid / (D / 8);
            u32x2_t tr[8];
            transpose4x8(vr[u], tr);
#pragma unroll
            for (int i = 0; i < 8; ++i) st8(vt + dec_tr_offset(8 * dc + i, kg), tr[i]);
        }
        // S^T = K Q^T for the two 16-key blocks
        f32x4_t sc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) sc[mb] = mfma16<T>(ka[mb][kc], qf[kc], sc[mb]);
        }
        // this tile's bias, before the register set is refilled
        float bt[2][4];
        if (BIAS) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) bt[mb][r] = bb[mb][r];
        }
        // refill this register set with tile it + 2 (two tiles of latency cover)
        if (it + 2 < n_tiles) load(kt + 2 * kDecKT, ka, vr, bb);

        // (rows' window bands start at qi + coff - W + 1 <= coff + q_len - W)
        const bool need_mask = (kt + kDecKT > ke) || (p.causal && kt + kDecKT - 1 > coff) ||
                               (p.window > 0 && kt < coff + q_len - p.window);
        float mx = kNegInf;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kt + 16 * mb + 4 * lg + r;
                bool ok = row_ok;
                if (need_mask) {
                    ok = ok && key < ke;
                    if (p.causal) ok = ok && key <= qi + coff;
                    if (p.window > 0) ok = ok && key > qi + coff - p.window;
                }
                float x = sc[mb][r] * p.scale_log2;
                if (BIAS) x = fmaf(bt[mb][r], kLog2e, x);
                x = ok ? x : kNegInf;
                sc[mb][r] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        float ls = 0.f;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(sc[mb][r] - m_use);
                ls += e;
                sc[mb][r] = e;
            }
        }
        l_run = l_run * corr + ls;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= corr;
        // P^T operand: slot j < 4 -> key 4 lg + j, j >= 4 -> key 16 + 4 lg + j - 4.
        const u32x4_t pf = u32x4_t{T::pack2(sc[0][0], sc[0][1]), T::pack2(sc[0][2], sc[0][3]),
                                   T::pack2(sc[1][0], sc[1][1]), T::pack2(sc[1][2], sc[1][3])};
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 16 * db + n16;
            const u32x2_t x0 = ld8(vt + dec_tr_offset(d, lg));
            const u32x2_t x1 = ld8(vt + dec_tr_offset(d, 4 + lg));
            oacc[db] = mfma16<T>(u32x4_t{x0[0], x0[1], x1[0], x1[1]}, pf, oacc[db]);
        }
    };
    if (n_tiles > 0) load(ks, ka, vr, bb);
    if (n_tiles > 1) load(ks + kDecKT, ka2, vr2, bb2);
    for (int it = 0; it < n_tiles; it += 2) {
        step(it, ka, vr, bb);
        if (it + 1 < n_tiles) step(it + 1, ka2, vr2, bb2);
    }

    // l_run is split over the 4 lane groups holding a row's keys.
    float lt = l_run + __shfl_xor(l_run, 16);
    lt += __shfl_xor(lt, 32);
    if (row_ok) {
        const float inv = !(lt <= 0.f) ? 1.f / lt : 0.f;
        const int64_t prow = ((int64_t)(hk * p.n_hg + hgi) * p.n_slots + slot) * 16 + n16;
        float* op = p.o_part + prow * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 16 * db + 4 * lg;
            *reinterpret_cast<f32x4_t*>(op + d) = oacc[db] * inv;
        }
        if (lg == 0) p.lse_part[prow] = !(lt <= 0.f) ? m_run * kLn2 + logf(lt) : kNegInf;
    }
}

// One wave per (row, head): O = sum_i w_i O_i / sum_i w_i over the work items
// of the row's sequence, w_i = exp(lse_i - max lse). Rows outside every
// sequence, or beyond the 16-row group (max_seqlen_q too small), are left
// untouched as the flash forward leaves them.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecKParams p, typename T::raw* __restrict__ out,
                                                             float* __restrict__ lse_out, int d) {
    const int64_t rh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (rh >= p.total_q * p.hq) return;
    const int64_t row = rh / p.hq;
    const int head = (int)(rh - row * p.hq);
    // sequence of this row (largest s with cu_q[s] <= row)
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.cu_q[mid] <= row) lo = mid; else hi = mid - 1;
    }
    const int s = lo;
    const SeqRange qr = seq_range(p.cu_q, s, p.total_q);
    if (row < qr.start || row >= qr.end) return;
    const int q_len = qr.end - qr.start, qi = (int)(row - qr.start);
    const int hk = head / p.g, hh_full = head - hk * p.g;
    const int hgi = hh_full / p.hpb, n = (hh_full - hgi * p.hpb) * q_len + qi;
    if (n >= 16) return;
    const SeqRange kr = seq_range(p.cu_kv, s, p.total_kv);
    const int kv_len = kr.end - kr.start;
    int first, count;
    if (p.chunk > 0) {
        first = tile_base(p.cu_kv, s, p.chunk, p.total_kv);
        count = (kv_len + p.chunk - 1) / p.chunk;
    } else {
        first = s * p.ns;
        count = p.ns;
    }
    const int64_t base = (int64_t)(hk * p.n_hg + hgi) * p.n_slots;
    // max LSE: lanes over items, then across the wave
    float m = kNegInf;
    // (NaN-preserving: a NaN logit makes its item's LSE NaN, and a row whose
    // items are all NaN must not look empty)
    for (int i = lane; i < count; i += 64) m = nan_max(p.lse_part[(base + first + i) * 16 + n], m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = nan_max(m, __shfl_xor(m, off));
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    if (m != kNegInf) {
        // items in groups of 4 whose loads all go out before the first use;
        // the sums still run in item order
        constexpr int U = 4;
        for (int i0 = 0; i0 < count; i0 += U) {
            float l[U], o[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool in = i0 + u < count;
                const int64_t prow = (base + first + min(i0 + u, count - 1)) * 16 + n;
                l[u] = in ? p.lse_part[prow] : kNegInf;
                const float* op = p.o_part + prow * d;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int dd = lane + 64 * j;
                    o[u][j] = dd < d ? op[dd] : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (l[u] == kNegInf) continue;
                const float wgt = __expf(l[u] - m);
                wsum += wgt;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (lane + 64 * j < d) acc[j] += wgt * o[u][j];
            }
        }
    }
    const float inv = !(wsum <= 0.f) ? 1.f / wsum : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int dd = lane + 64 * j;
        if (dd < d) out[rh * d + dd] = T::from_float(acc[j] * inv);
    }
    if (lse_out != nullptr && lane == 0) lse_out[rh] = !(wsum <= 0.f) ? m + logf(wsum) : kNegInf;
}

template <typename T, int D>
hipError_t launch_typed(const DecodeArgs& a, hipStream_t st) {
    const Geometry& g = a.geo;
    DecKParams p;
    p.q = (const uint16_t*)a.q; p.k = (const uint16_t*)a.k; p.v = (const uint16_t*)a.v;
    p.o_part = a.o_part; p.lse_part = a.lse_part;
    p.cu_q = g.cu_q; p.cu_kv = g.cu_kv;
    p.bias = g.bias; p.bias_qs = g.bias_qs; p.bias_hs = g.bias_hs; p.bias_cols = g.bias_cols;
    p.bias_ss = g.bias_ss; p.bias_rows = g.bias_rows;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs;
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.hkv = g.hkv; p.g = g.g;
    const int mq = a.max_q > 0 ? a.max_q : 1;
    int hpb = 16 / mq;                  // heads per 16-row group: largest divisor of g that fits
    if (hpb < 1) return hipErrorInvalidValue;
    if (hpb > g.g) hpb = g.g;
    while (g.g % hpb != 0) --hpb;
    p.hpb = hpb;
    p.n_hg = g.g / hpb;
    p.ns = a.num_splits;
    p.chunk = a.chunk;
    const int64_t slots = a.chunk > 0 ? g.total_kv / a.chunk + g.num_seqs + 1 : (int64_t)g.num_seqs * a.num_splits;
    if (slots > 0x3fffffff) return hipErrorInvalidValue;
    p.n_slots = (int)slots;
    p.scale_log2 = g.scale * kLog2e;
    p.causal = g.causal;
    p.window = g.window;
    p.bias_v4 = g.bias != nullptr && ((uintptr_t)g.bias % 16 == 0) && g.bias_qs % 4 == 0 && g.bias_hs % 4 == 0 &&
                (g.bias_ss < 0 || g.bias_ss % 4 == 0);
    p.block_table = a.block_table;
    p.bt_stride = a.bt_stride;
    p.page_size = a.page_size;
    p.num_pages = a.num_pages;
    const bool paged = a.block_table != nullptr;
    if (paged && (a.page_size < 16 || a.page_size % 16 != 0 || a.num_pages < 1)) return hipErrorInvalidValue;
    const int64_t waves = (int64_t)g.hkv * p.n_hg * p.n_slots;
    const int64_t blocks = (waves + kDecWaves - 1) / kDecWaves;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (blocks > 0) {
        const dim3 grid((unsigned)blocks), block(kDecWaves * 64);
        if (p.bias != nullptr) {
            if (paged) hipLaunchKernelGGL((decode_split_kernel<T, D, true, true>), grid, block, 0, st, p);
            else hipLaunchKernelGGL((decode_split_kernel<T, D, true, false>), grid, block, 0, st, p);
        } else {
            if (paged) hipLaunchKernelGGL((decode_split_kernel<T, D, false, true>), grid, block, 0, st, p);
            else hipLaunchKernelGGL((decode_split_kernel<T, D, false, false>), grid, block, 0, st, p);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t rh = g.total_q * g.hq;
    if (rh > 0)
        hipLaunchKernelGGL(decode_combine_kernel<T>, dim3((unsigned)((rh + 3) / 4)), dim3(256), 0, st, p,
                           (typename T::raw*)a.o, a.lse, D);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(int dtype, const DecodeArgs& a, hipStream_t st) {
    const int d = a.geo.d;
    if (dtype == MTLATTN_DTYPE_BF16) {
        if (d == 128) return launch_typed<BF16, 128>(a, st);
        if (d == 64) return launch_typed<BF16, 64>(a, st);
    } else if (dtype == MTLATTN_DTYPE_F16) {
        if (d == 128) return launch_typed<F16, 128>(a, st);
        if (d == 64) return launch_typed<F16, 64>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace mtlattn
