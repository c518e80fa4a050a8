// fp32 flash attention on the fp32 matrix cores of gfx950
// (v_mfma_f32_32x32x2_f32): the forward with its LSE, dQ and dK/dV for head
// dims up to 128 that are a multiple of 4, with 16-byte aligned rows. Inputs,
// products, accumulation and softmax stay fp32 end to end (the reference runs
// fp32 inputs on its simdgroup kernels in fp32, src/attention.metal:334, 863;
// the mathematics is src/attention.metal:44-289 forward, 741-784 dQ,
// 788-835 dK/dV). Exponentials use exp_fp32 (common.h). Other fp32 shapes
// take the portable kernels.
//
// v_mfma_f32_32x32x2_f32: C[32x32] += A[32x2] * B[2x32]
//   A: lane l holds A[m = l%32][k = l/32]
//   B: lane l holds B[k = l/32][n = l%32]
//   C: lane l holds column n = l%32, rows m = 8*(r/4) + 4*(l/32) + r%4
// A product contracting over the head dim takes DP/2 instructions
// (DP = D rounded up to 32, zero columns past D): instruction j uses head
// column h*DP/2 + j in lane half h = l/32, so each lane reads its operand
// row's half as consecutive 16-byte words. A product contracting over the 32
// rows of a C tile (P.V, dS.K, P^T.dO, dS^T.Q) takes C register r as
// instruction r's operand: the contraction index of instruction r in half h
// is row 8*(r/4) + 4*h + r%4, and the other operand is read from a
// transposed LDS tile at that column, four instructions per 16-byte read.
//
// A workgroup is 4 waves of 32 rows each:
//   forward / dQ: a wave owns 32 query rows of one head and computes
//     S^T = K.Q^T, so the lane is the query and its softmax row lives in its
//     own registers and those of lane l ^ 32.
//   dK / dV: a wave owns 32 keys of one kv head and computes S = Q.K^T, so
//     the lane is the key; the workgroup loops over the g query heads of the
//     group and the 32-query tiles that can see its 128 keys.
// The shared tiles (K and V, or Q, dO, LSE and delta) are staged by all 256
// threads: float4 global loads one tile ahead into registers, two LDS slots,
// one barrier per tile. Row-major tiles use rows of DP + 4 floats (16-byte
// reads of 16 consecutive rows land in 16 distinct groups of 4 banks),
// transposed tiles DP rows of 36 floats.
#include "common.h"
#include "kernels.h"

namespace mtlattn {

namespace {

constexpr int kWgRows = 128;   // rows per workgroup (4 waves x 32)
constexpr int kTs = 36;        // row stride of a transposed tile, floats

struct F32Params {
    const float* q; const float* k; const float* v; const float* dout;
    float* o; float* lse;
    const float* lse_in; const float* delta;
    float* dq; float* dk; float* dv;
    const int* cu_q; const int* cu_kv;
    const float* bias;
    int64_t q_rs, k_rs, v_rs, do_rs;
    int64_t bias_qs, bias_hs, bias_cols, bias_ss, bias_rows;
    int64_t total_q, total_kv;
    int num_seqs, hq, hkv, g, d;
    float scale;
    int causal, window;
    // The forward and dQ split over their key tiles, dK/dV over its (query
    // head, query tile) iterations. Split z of nsplit writes fp32 partials:
    // forward, normalised O to part + z * total_q * hq * d and its LSE to
    // part + nsplit * total_q * hq * d + z * total_q * hq; dQ, unscaled, to
    // part + z * total_q * hq * d; dK/dV, unscaled, to
    // part + z * 2 * total_kv * hkv * d (dK, then dV). part == nullptr: one
    // split writing o / dq / dk / dv
    float* part;
    int nsplit;
    // dQ only: o != nullptr computes delta = rowsum(dO * O) in the kernel
    // (written to delta_out by split 0) instead of reading delta
    const float* o_in; int64_t o_rs;
    float* delta_out;
};

__device__ inline f32x16_t mma(float a, float b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ inline f32x4_t ld4(const float* p) { return *reinterpret_cast<const f32x4_t*>(p); }

// 32 rows x DP columns of an fp32 tensor, row r at base + r * rs; rows at or
// past nrows and columns at or past d read as zero (d % 4 == 0). Thread t of
// 256 holds chunks t + 256 c: row (t + 256 c) / (DP / 4), 4 columns.
template <int DP>
struct Tile32 {
    static constexpr int CPR = DP / 4;
    static constexpr int N = DP / 32;
    f32x4_t v[N];
    __device__ inline void load(const float* base, int64_t rs, int nrows, int d, int t) {
#pragma unroll
        for (int c = 0; c < N; ++c) {
            const int id = t + 256 * c, r = id / CPR, col = 4 * (id % CPR);
            f32x4_t x = {0.f, 0.f, 0.f, 0.f};
            if (r < nrows && col < d) x = ld4(base + (int64_t)r * rs + col);
            v[c] = x;
        }
    }
    // row-major copy (rows of DP + 4 floats) and/or transposed copy (DP rows
    // of kTs floats)
    template <bool RM, bool TR>
    __device__ inline void store(float* rm, float* tr, int t) const {
#pragma unroll
        for (int c = 0; c < N; ++c) {
            const int id = t + 256 * c, r = id / CPR, col = 4 * (id % CPR);
            if constexpr (RM) *reinterpret_cast<f32x4_t*>(rm + r * (DP + 4) + col) = v[c];
            if constexpr (TR) {
#pragma unroll
                for (int e = 0; e < 4; ++e) tr[(col + e) * kTs + r] = v[c][e];
            }
        }
    }
};

// Lane's half of one operand row (DP/2 floats from column h*DP/2), zero past
// d or for an invalid row.
template <int DP>
__device__ inline void load_half_row(float (&dst)[DP / 2], const float* row, bool valid, int h, int d) {
#pragma unroll
    for (int c = 0; c < DP / 8; ++c) {
        const int col = h * (DP / 2) + 4 * c;
        f32x4_t x = {0.f, 0.f, 0.f, 0.f};
        if (valid && col < d) x = ld4(row + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[4 * c + e] = x[e];
    }
}

// Rounding. One fp32 MFMA adds two products to its accumulator; chains of
// them round more often per term than one FMA per term, so long dependent
// chains are avoided: a head-dim product runs as two interleaved chains
// summed at the end, and a product over the rows of a tile starts from zero
// for every tile, its result added to the running sum once per tile (in the
// forward, in the same FMA as the rescale). The longest chain is then 32
// instructions at D = 128, and sums over many keys or queries take one VALU
// rounding per 32-row tile.

// A.B over the head dim: A rows from a row-major LDS tile (row l%32), B from
// the lane's registers.
template <int DP>
__device__ inline f32x16_t head_product(const float* tile_row_half, const float (&reg)[DP / 2]) {
    f32x16_t acc0 = {}, acc1 = {};
#pragma unroll
    for (int c = 0; c < DP / 8; c += 2) {
        const f32x4_t a0 = ld4(tile_row_half + 4 * c);
        const f32x4_t a1 = ld4(tile_row_half + 4 * c + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc0 = mma(a0[e], reg[4 * c + e], acc0);
            acc1 = mma(a1[e], reg[4 * c + 4 + e], acc1);
        }
    }
    return acc0 + acc1;
}

// For each column block b: T^T.C over the 32 rows of a C tile (register r
// of C against the transposed tile at row 32 b + l%32, column
// 8 (r/4) + 4 h + r%4) from zero, handed to fold(b, partial).
template <int DP, typename F>
__device__ inline void row_product(const float* tr, int l32, int h, const float (&c)[16], F&& fold) {
#pragma unroll
    for (int b = 0; b < DP / 32; ++b) {
        const float* tb = tr + (32 * b + l32) * kTs + 4 * h;
        f32x16_t part = {};
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4_t a = ld4(tb + 8 * q4);
#pragma unroll
            for (int e = 0; e < 4; ++e) part = mma(a[e], c[4 * q4 + e], part);
        }
        fold(b, part);
    }
}

// Store the lane's row of a C-layout accumulator set (column block b, rows
// of register group r/4 at 32 b + 8 (r/4) + 4 h) times `mul`, columns < d.
template <int DP>
__device__ inline void store_row(float* row, const f32x16_t (&acc)[DP / 32], int h, int d, float mul) {
#pragma unroll
    for (int b = 0; b < DP / 32; ++b) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int col = 32 * b + 8 * g4 + 4 * h;
            if (col < d) {
                const f32x4_t x = {acc[b][4 * g4] * mul, acc[b][4 * g4 + 1] * mul, acc[b][4 * g4 + 2] * mul,
                                   acc[b][4 * g4 + 3] * mul};
                *reinterpret_cast<f32x4_t*>(row + col) = x;
            }
        }
    }
}

struct Tiling {
    int s, start, len, other_start, other_len, coff, r0;
};

// Workgroup blockIdx.x -> (sequence, first row) over 128-row tiles of `cu`
// (tile numbering of common.h); r0 >= len means the workgroup has no rows.
// Query tiles run last-first: under a causal mask the last tiles of a
// sequence see the most keys, and dispatching the heaviest workgroups first
// keeps them out of the final round (key tiles are heaviest first already).
__device__ inline Tiling tiling(const int* cu, const int* cu_other, int num_seqs, int64_t total, int64_t total_other,
                                bool rows_are_queries) {
    Tiling t;
    const int bx = rows_are_queries ? (int)(gridDim.x - 1 - blockIdx.x) : (int)blockIdx.x;
    t.s = find_seq_for_tile(cu, num_seqs, kWgRows, bx, total);
    const int tb = tile_base(cu, t.s, kWgRows, total);
    const SeqRange a = seq_range(cu, t.s, total), b = seq_range(cu_other, t.s, total_other);
    t.start = a.start; t.len = a.end - a.start;
    t.other_start = b.start; t.other_len = b.end - b.start;
    t.coff = rows_are_queries ? t.other_len - t.len : t.len - t.other_len;   // kv_len - q_len
    // a block before its sequence's first tile (rows ahead of cu[0]) has no rows
    t.r0 = bx < tb ? t.len : (bx - tb) * kWgRows;
    return t;
}

// ---------------------------------------------------------------------------
// Forward. Grids with fewer workgroups than the GPU holds split each
// workgroup's key tiles over blockIdx.z; f32_fwd_combine_kernel merges the
// splits' normalised O and LSE.
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256, DP <= 96 ? 2 : 1) void f32_fwd_kernel(F32Params p) {
    constexpr int HD = DP / 2, NB = DP / 32, SR = DP + 4;
    constexpr int KSZ = 32 * SR, SLOT = KSZ + DP * kTs;
    __shared__ __attribute__((aligned(16))) float lds[2 * SLOT];
    const int t = threadIdx.x, w = t >> 6, l32 = t & 31, h = (t >> 5) & 1;
    const int head = blockIdx.y, hk = head / p.g;
    const Tiling tl = tiling(p.cu_q, p.cu_kv, p.num_seqs, p.total_q, p.total_kv, true);
    const int q_len = tl.len, kv_len = tl.other_len, coff = tl.coff, q0 = tl.r0;
    if (q0 >= q_len) return;

    const int qlast = min(q0 + kWgRows, q_len) - 1;
    const Band ba = key_band(q0, coff, kv_len, p.causal, p.window);
    const Band bz = key_band(qlast, coff, kv_len, p.causal, p.window);
    const int klo = ba.lo & ~31, khi = bz.lo + (int)bz.width;
    const int ntiles = khi > klo ? (khi - klo + 31) / 32 : 0;
    const int z = (int)blockIdx.z;
    const int it0 = (int)((int64_t)ntiles * z / p.nsplit), it1 = (int)((int64_t)ntiles * (z + 1) / p.nsplit);

    const int wq0 = q0 + 32 * w;
    const bool wave_on = wq0 < q_len;
    int wlo = 0, whi = 0;
    if (wave_on) {
        const Band w0 = key_band(wq0, coff, kv_len, p.causal, p.window);
        const Band w1 = key_band(min(wq0 + 31, q_len - 1), coff, kv_len, p.causal, p.window);
        wlo = w0.lo; whi = w1.lo + (int)w1.width;
    }
    const int qi = wq0 + l32;
    const bool qvalid = qi < q_len;
    const Band qb = qvalid ? key_band(qi, coff, kv_len, p.causal, p.window) : Band{0, 0u};
    const int64_t grow = (int64_t)tl.start + qi;

    float qreg[HD];
    load_half_row<DP>(qreg, p.q + grow * p.q_rs + (int64_t)head * p.d, qvalid, h, p.d);
    const float* brow = (p.bias != nullptr && qvalid)
                            ? p.bias + bias_row_offset(grow, tl.s, tl.start, p.bias_qs, p.bias_ss, p.bias_rows) +
                                  (int64_t)head * p.bias_hs
                            : nullptr;

    const float* kbase = p.k + (int64_t)tl.other_start * p.k_rs + (int64_t)hk * p.d;
    const float* vbase = p.v + (int64_t)tl.other_start * p.v_rs + (int64_t)hk * p.d;
    Tile32<DP> tk, tv;
    float m = kNegInf, lsum = 0.f;
    f32x16_t acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = f32x16_t{};

    if (it1 > it0) {
        const int k0 = klo + 32 * it0;
        tk.load(kbase + (int64_t)k0 * p.k_rs, p.k_rs, kv_len - k0, p.d, t);
        tv.load(vbase + (int64_t)k0 * p.v_rs, p.v_rs, kv_len - k0, p.d, t);
        tk.template store<true, false>(lds, nullptr, t);
        tv.template store<false, true>(nullptr, lds + KSZ, t);
    }
    __syncthreads();
    for (int it = it0; it < it1; ++it) {
        const int kt = klo + 32 * it;
        const bool more = it + 1 < it1;
        if (more) {
            tk.load(kbase + (int64_t)(kt + 32) * p.k_rs, p.k_rs, kv_len - kt - 32, p.d, t);
            tv.load(vbase + (int64_t)(kt + 32) * p.v_rs, p.v_rs, kv_len - kt - 32, p.d, t);
        }
        const float* ks = lds + ((it - it0) & 1) * SLOT;
        if (wave_on && kt < whi && kt + 32 > wlo) {
            const f32x16_t sacc = head_product<DP>(ks + l32 * SR + h * HD, qreg);
            float x[16];
            float mt = kNegInf;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kj = kt + 8 * (r >> 2) + 4 * h + (r & 3);
                float xv = kNegInf;
                if (qb.has(kj)) {
                    xv = sacc[r] * p.scale;
                    if (brow != nullptr && kj < p.bias_cols) xv += brow[kj];
                }
                x[r] = xv;
                mt = fmaxf(mt, xv);
            }
            mt = pair_max(mt);
            const float mn = fmaxf(m, mt);
            const float mu = mn == kNegInf ? 0.f : mn;
            const float corr = exp_fp32(m - mu);
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                x[r] = x[r] == kNegInf ? 0.f : exp_fp32(x[r] - mu);
                ps += x[r];
            }
            lsum = lsum * corr + pair_sum(ps);
            m = mn;
            row_product<DP>(ks + KSZ, l32, h, x, [&](int b, const f32x16_t& part) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[b][r] = fmaf(acc[b][r], corr, part[r]);
            });
        }
        if (more) {
            float* nx = lds + ((it + 1 - it0) & 1) * SLOT;
            tk.template store<true, false>(nx, nullptr, t);
            tv.template store<false, true>(nullptr, nx + KSZ, t);
        }
        __syncthreads();
    }
    if (wave_on && qvalid) {
        const float inv = !(lsum <= 0.f) ? 1.f / lsum : 0.f;
        const float l_out = !(lsum <= 0.f) ? m + logf(lsum) : kNegInf;
        const int64_t rh = grow * p.hq + head;
        if (p.part == nullptr) {
            store_row<DP>(p.o + rh * p.d, acc, h, p.d, inv);
            if (h == 0 && p.lse != nullptr) p.lse[rh] = l_out;
        } else {
            const int64_t plane = p.total_q * p.hq;
            store_row<DP>(p.part + (z * plane + rh) * p.d, acc, h, p.d, inv);
            if (h == 0) p.part[(int64_t)p.nsplit * plane * p.d + z * plane + rh] = l_out;
        }
    }
}

// o and lse of the rows in [cu_q[0], cu_q[num_seqs]) from the forward's
// nsplit partials (normalised O_z, LSE_z): O = sum_z w_z O_z / sum_z w_z with
// w_z = exp(LSE_z - max_z LSE_z), LSE = max + log(sum_z w_z); a row whose
// splits are all empty gets O = 0, LSE = -inf. One thread per 4 columns.
__global__ __launch_bounds__(256) void f32_fwd_combine_kernel(const float* __restrict__ part, int nsplit,
                                                              const int* __restrict__ cu_q, int num_seqs,
                                                              int64_t total_q, int hq, int d, float* __restrict__ o,
                                                              float* __restrict__ lse) {
    const int dq4 = d / 4;
    const int64_t plane = total_q * hq;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= plane * dq4) return;
    const int64_t rh = i / dq4;
    const int c4 = (int)(i - rh * dq4);
    const int64_t row = rh / hq;
    int64_t r0 = cu_q[0], r1 = cu_q[num_seqs];
    r0 = r0 < 0 ? 0 : (r0 > total_q ? total_q : r0);
    r1 = r1 < r0 ? r0 : (r1 > total_q ? total_q : r1);
    if (row < r0 || row >= r1) return;
    const float* lp = part + (int64_t)nsplit * plane * d;
    // max over the splits that keeps a NaN LSE (a NaN logit in the split):
    // fmaxf would drop it and the row would look empty
    float mx = kNegInf;
    for (int z = 0; z < nsplit; ++z) {
        const float lz = lp[z * plane + rh];
        mx = nan_max(lz, mx);
        if (mx != mx) break;
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    float sum = 0.f;
    if (mx != kNegInf) {
        for (int z = 0; z < nsplit; ++z) {
            const float lz = lp[z * plane + rh];
            if (lz == kNegInf) continue;
            const float wz = exp_fp32(lz - mx);
            sum += wz;
            acc += wz * ld4(part + (z * plane + rh) * d + 4 * c4);
        }
    }
    const float inv = !(sum <= 0.f) ? 1.f / sum : 0.f;
    *reinterpret_cast<f32x4_t*>(o + rh * d + 4 * c4) = acc * inv;
    if (c4 == 0 && lse != nullptr) lse[rh] = !(sum <= 0.f) ? mx + logf(sum) : kNegInf;
}

// ---------------------------------------------------------------------------
// dQ = scale * dS.K with dS = P * (dP - delta), dP = dO.V^T. Grids with fewer
// workgroups than the GPU holds split each workgroup's key tiles over
// blockIdx.z; f32_split_sum_kernel adds the splits in order.
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256, 1) void f32_dq_kernel(F32Params p) {
    constexpr int HD = DP / 2, NB = DP / 32, SR = DP + 4;
    constexpr int KSZ = 32 * SR, TSZ = DP * kTs, SLOT = 2 * KSZ + TSZ;   // K, V row-major; K transposed
    __shared__ __attribute__((aligned(16))) float lds[2 * SLOT];
    const int t = threadIdx.x, w = t >> 6, l32 = t & 31, h = (t >> 5) & 1;
    const int head = blockIdx.y, hk = head / p.g;
    const Tiling tl = tiling(p.cu_q, p.cu_kv, p.num_seqs, p.total_q, p.total_kv, true);
    const int q_len = tl.len, kv_len = tl.other_len, coff = tl.coff, q0 = tl.r0;
    if (q0 >= q_len) return;

    const int qlast = min(q0 + kWgRows, q_len) - 1;
    const Band ba = key_band(q0, coff, kv_len, p.causal, p.window);
    const Band bz = key_band(qlast, coff, kv_len, p.causal, p.window);
    const int klo = ba.lo & ~31, khi = bz.lo + (int)bz.width;
    const int ntiles = khi > klo ? (khi - klo + 31) / 32 : 0;
    const int z = (int)blockIdx.z;
    const int it0 = (int)((int64_t)ntiles * z / p.nsplit), it1 = (int)((int64_t)ntiles * (z + 1) / p.nsplit);

    const int wq0 = q0 + 32 * w;
    const bool wave_on = wq0 < q_len;
    int wlo = 0, whi = 0;
    if (wave_on) {
        const Band w0 = key_band(wq0, coff, kv_len, p.causal, p.window);
        const Band w1 = key_band(min(wq0 + 31, q_len - 1), coff, kv_len, p.causal, p.window);
        wlo = w0.lo; whi = w1.lo + (int)w1.width;
    }
    const int qi = wq0 + l32;
    const bool qvalid = qi < q_len;
    const int64_t grow = (int64_t)tl.start + qi;
    const float lse = qvalid ? p.lse_in[grow * p.hq + head] : kNegInf;
    // a row with no keys (LSE -inf) has P = 0 everywhere
    const Band qb = (qvalid && lse != kNegInf) ? key_band(qi, coff, kv_len, p.causal, p.window) : Band{0, 0u};

    float qreg[HD], doreg[HD];
    load_half_row<DP>(qreg, p.q + grow * p.q_rs + (int64_t)head * p.d, qvalid, h, p.d);
    load_half_row<DP>(doreg, p.dout + grow * p.do_rs + (int64_t)head * p.d, qvalid, h, p.d);
    float dlt;
    if (p.o_in != nullptr) {
        // delta over the lane's half row of dO and O, then the two halves
        float oreg[HD];
        load_half_row<DP>(oreg, p.o_in + grow * p.o_rs + (int64_t)head * p.d, qvalid, h, p.d);
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < HD; ++j) part = fmaf(doreg[j], oreg[j], part);
        dlt = pair_sum(part);
        if (qvalid && wave_on && z == 0 && h == 0) p.delta_out[grow * p.hq + head] = dlt;
    } else {
        dlt = qvalid ? p.delta[grow * p.hq + head] : 0.f;
    }
    const float* brow = (p.bias != nullptr && qvalid)
                            ? p.bias + bias_row_offset(grow, tl.s, tl.start, p.bias_qs, p.bias_ss, p.bias_rows) +
                                  (int64_t)head * p.bias_hs
                            : nullptr;

    const float* kbase = p.k + (int64_t)tl.other_start * p.k_rs + (int64_t)hk * p.d;
    const float* vbase = p.v + (int64_t)tl.other_start * p.v_rs + (int64_t)hk * p.d;
    Tile32<DP> tk, tv;
    f32x16_t acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = f32x16_t{};

    if (it1 > it0) {
        const int k0 = klo + 32 * it0;
        tk.load(kbase + (int64_t)k0 * p.k_rs, p.k_rs, kv_len - k0, p.d, t);
        tv.load(vbase + (int64_t)k0 * p.v_rs, p.v_rs, kv_len - k0, p.d, t);
        tk.template store<true, true>(lds, lds + 2 * KSZ, t);
        tv.template store<true, false>(lds + KSZ, nullptr, t);
    }
    __syncthreads();
    for (int it = it0; it < it1; ++it) {
        const int kt = klo + 32 * it;
        const bool more = it + 1 < it1;
        if (more) {
            tk.load(kbase + (int64_t)(kt + 32) * p.k_rs, p.k_rs, kv_len - kt - 32, p.d, t);
            tv.load(vbase + (int64_t)(kt + 32) * p.v_rs, p.v_rs, kv_len - kt - 32, p.d, t);
        }
        const float* ks = lds + ((it - it0) & 1) * SLOT;
        if (wave_on && kt < whi && kt + 32 > wlo) {
            const f32x16_t sacc = head_product<DP>(ks + l32 * SR + h * HD, qreg);
            const f32x16_t pacc = head_product<DP>(ks + KSZ + l32 * SR + h * HD, doreg);
            float ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kj = kt + 8 * (r >> 2) + 4 * h + (r & 3);
                float v = 0.f;
                if (qb.has(kj)) {
                    float xv = sacc[r] * p.scale;
                    if (brow != nullptr && kj < p.bias_cols) xv += brow[kj];
                    v = exp_fp32(xv - lse) * (pacc[r] - dlt);
                }
                ds[r] = v;
            }
            row_product<DP>(ks + 2 * KSZ, l32, h, ds, [&](int b, const f32x16_t& part) { acc[b] += part; });
        }
        if (more) {
            float* nx = lds + ((it + 1 - it0) & 1) * SLOT;
            tk.template store<true, true>(nx, nx + 2 * KSZ, t);
            tv.template store<true, false>(nx + KSZ, nullptr, t);
        }
        __syncthreads();
    }
    if (wave_on && qvalid) {
        const int64_t o = (grow * p.hq + head) * p.d;
        if (p.part == nullptr) store_row<DP>(p.dq + o, acc, h, p.d, p.scale);
        else store_row<DP>(p.part + (int64_t)z * p.total_q * p.hq * p.d + o, acc, h, p.d, 1.f);
    }
}

// ---------------------------------------------------------------------------
// dV = P^T.dO, dK = scale * dS^T.Q, summed over the g query heads of the kv
// head in a fixed order (no atomics). Grids with fewer workgroups than the
// GPU holds split the (head, query tile) iterations of each workgroup over
// blockIdx.z; f32_split_sum_kernel then adds the splits in order z = 0, 1,
// ... (deterministic for a given split count).
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256, 1) void f32_dkv_kernel(F32Params p) {
    constexpr int HD = DP / 2, NB = DP / 32, SR = DP + 4;
    constexpr int KSZ = 32 * SR, TSZ = DP * kTs;
    // Q, dO row-major; Q, dO transposed; LSE and delta of the 32 queries
    constexpr int SLOT = 2 * KSZ + 2 * TSZ + 64;
    __shared__ __attribute__((aligned(16))) float lds[2 * SLOT];
    const int t = threadIdx.x, w = t >> 6, l32 = t & 31, h = (t >> 5) & 1;
    const int hk = blockIdx.y;
    const Tiling tl = tiling(p.cu_kv, p.cu_q, p.num_seqs, p.total_kv, p.total_q, false);
    const int kv_len = tl.len, q_len = tl.other_len, coff = tl.coff, j0 = tl.r0;
    if (j0 >= kv_len) return;

    const int jlast = min(j0 + kWgRows, kv_len) - 1;
    const Band qa = query_band(j0, coff, q_len, kv_len, p.causal, p.window);
    const Band qz = query_band(jlast, coff, q_len, kv_len, p.causal, p.window);
    const int qlo = qa.lo & ~31, qhi = qz.lo + (int)qz.width;
    const int nq = qhi > qlo ? (qhi - qlo + 31) / 32 : 0;
    const int z = (int)blockIdx.z;
    const int it0 = (int)((int64_t)nq * p.g * z / p.nsplit), it1 = (int)((int64_t)nq * p.g * (z + 1) / p.nsplit);

    const int wj0 = j0 + 32 * w;
    const bool wave_on = wj0 < kv_len;
    int wlo = 0, whi = 0;
    if (wave_on) {
        const Band w0 = query_band(wj0, coff, q_len, kv_len, p.causal, p.window);
        const Band w1 = query_band(min(wj0 + 31, kv_len - 1), coff, q_len, kv_len, p.causal, p.window);
        wlo = w0.lo; whi = w1.lo + (int)w1.width;
    }
    const int kj = wj0 + l32;
    const bool kvalid = kj < kv_len;
    const Band kb = query_band(kj, coff, q_len, kv_len, p.causal, p.window);   // empty past kv_len
    const int64_t krow = (int64_t)tl.start + kj;

    float kreg[HD], vreg[HD];
    load_half_row<DP>(kreg, p.k + krow * p.k_rs + (int64_t)hk * p.d, kvalid, h, p.d);
    load_half_row<DP>(vreg, p.v + krow * p.v_rs + (int64_t)hk * p.d, kvalid, h, p.d);

    Tile32<DP> tq, tdo;
    float lse_d = 0.f;   // thread t < 64: LSE (t < 32) or delta of query t % 32 of the next tile
    f32x16_t dka[NB], dva[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) { dka[b] = f32x16_t{}; dva[b] = f32x16_t{}; }

    auto load_tile = [&](int it_) {
        const int hh = it_ / nq, qt = qlo + 32 * (it_ - hh * nq), head = hk * p.g + hh;
        const int64_t r0 = (int64_t)tl.other_start + qt;
        tq.load(p.q + r0 * p.q_rs + (int64_t)head * p.d, p.q_rs, q_len - qt, p.d, t);
        tdo.load(p.dout + r0 * p.do_rs + (int64_t)head * p.d, p.do_rs, q_len - qt, p.d, t);
        if (t < 64) {
            const int qq = qt + (t & 31);
            const int64_t idx = (r0 + (t & 31)) * p.hq + head;
            lse_d = t < 32 ? (qq < q_len ? p.lse_in[idx] : kNegInf) : (qq < q_len ? p.delta[idx] : 0.f);
        }
    };
    auto store_tile = [&](float* slot) {
        tq.template store<true, true>(slot, slot + 2 * KSZ, t);
        tdo.template store<true, true>(slot + KSZ, slot + 2 * KSZ + TSZ, t);
        if (t < 64) slot[2 * KSZ + 2 * TSZ + t] = lse_d;
    };

    if (it1 > it0) {
        load_tile(it0);
        store_tile(lds);
    }
    __syncthreads();
    for (int it = it0; it < it1; ++it) {
        const int hh = it / nq, qt = qlo + 32 * (it - hh * nq), head = hk * p.g + hh;
        const bool more = it + 1 < it1;
        if (more) load_tile(it + 1);
        const float* qs = lds + ((it - it0) & 1) * SLOT;
        if (wave_on && qt < whi && qt + 32 > wlo) {
            // P first and its dV product, then dP and dS (P is 0 wherever
            // the key is masked for the query, so dS is too)
            const f32x16_t sacc = head_product<DP>(qs + l32 * SR + h * HD, kreg);
            const float* ld_ = qs + 2 * KSZ + 2 * TSZ;
            float pr[16];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4_t l4 = ld4(ld_ + 8 * g4 + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * g4 + e, qq = qt + 8 * g4 + 4 * h + e;
                    float pv = 0.f;
                    if (kb.has(qq) && l4[e] != kNegInf) {
                        float xv = sacc[r] * p.scale;
                        if (p.bias != nullptr && kj < p.bias_cols) {
                            const int64_t grow = (int64_t)tl.other_start + qq;
                            xv += p.bias[bias_row_offset(grow, tl.s, tl.other_start, p.bias_qs, p.bias_ss,
                                                         p.bias_rows) +
                                         (int64_t)head * p.bias_hs + kj];
                        }
                        pv = exp_fp32(xv - l4[e]);
                    }
                    pr[r] = pv;
                }
            }
            row_product<DP>(qs + 2 * KSZ + TSZ, l32, h, pr,   // dO transposed
                            [&](int b, const f32x16_t& part) { dva[b] += part; });
            const f32x16_t pacc = head_product<DP>(qs + KSZ + l32 * SR + h * HD, vreg);
            float ds[16];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const f32x4_t d4 = ld4(ld_ + 32 + 8 * g4 + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) ds[4 * g4 + e] = pr[4 * g4 + e] * (pacc[4 * g4 + e] - d4[e]);
            }
            row_product<DP>(qs + 2 * KSZ, l32, h, ds,         // Q transposed
                            [&](int b, const f32x16_t& part) { dka[b] += part; });
        }
        if (more) store_tile(lds + ((it + 1 - it0) & 1) * SLOT);
        __syncthreads();
    }
    if (wave_on && kvalid) {
        const int64_t o = (krow * p.hkv + hk) * p.d;
        if (p.part == nullptr) {
            store_row<DP>(p.dk + o, dka, h, p.d, p.scale);
            store_row<DP>(p.dv + o, dva, h, p.d, 1.f);
        } else {
            float* pk = p.part + (int64_t)z * 2 * p.total_kv * p.hkv * p.d;
            store_row<DP>(pk + o, dka, h, p.d, 1.f);
            store_row<DP>(pk + p.total_kv * p.hkv * p.d + o, dva, h, p.d, 1.f);
        }
    }
}

// Sum of the splits' partials in order z = 0, 1, ...: out0 = scale0 * sum_z
// part[z][0], and with out1, out1 = sum_z part[z][1]; a split holds nout
// arrays of n4 float4 elements (d % 4 == 0).
__global__ __launch_bounds__(256) void f32_split_sum_kernel(const float* __restrict__ part, int nsplit, int64_t n4,
                                                            float scale0, float* __restrict__ out0,
                                                            float* __restrict__ out1) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const int64_t stride = (out1 != nullptr ? 2 : 1) * n4;   // float4 elements per split
    const f32x4_t* src = reinterpret_cast<const f32x4_t*>(part);
    f32x4_t a = src[i];
    for (int z = 1; z < nsplit; ++z) a += src[z * stride + i];
    reinterpret_cast<f32x4_t*>(out0)[i] = a * scale0;
    if (out1 != nullptr) {
        f32x4_t b = src[n4 + i];
        for (int z = 1; z < nsplit; ++z) b += src[z * stride + n4 + i];
        reinterpret_cast<f32x4_t*>(out1)[i] = b;
    }
}

F32Params make_params(const Geometry& g) {
    F32Params p{};
    p.cu_q = g.cu_q; p.cu_kv = g.cu_kv; p.bias = g.bias;
    p.bias_qs = g.bias_qs; p.bias_hs = g.bias_hs; p.bias_cols = g.bias_cols;
    p.bias_ss = g.bias_ss; p.bias_rows = g.bias_rows;
    p.total_q = g.total_q; p.total_kv = g.total_kv;
    p.num_seqs = g.num_seqs; p.hq = g.hq; p.hkv = g.hkv; p.g = g.g; p.d = g.d;
    p.scale = g.scale; p.causal = g.causal; p.window = g.window > 0 ? g.window : 0;
    p.part = nullptr; p.nsplit = 1;
    p.o_in = nullptr; p.o_rs = 0; p.delta_out = nullptr;
    return p;
}

using F32Kernel = void (*)(F32Params);

hipError_t launch(const F32Params& p, int64_t total_rows, int heads, hipStream_t st, F32Kernel k32, F32Kernel k64,
                  F32Kernel k96, F32Kernel k128, int splits = 1) {
    if (total_rows <= 0 || heads <= 0) return hipSuccess;
    if (!f32_mfma_head_dim(p.d) || p.num_seqs <= 0 || heads > 65535 || splits < 1 || splits > 64)
        return hipErrorInvalidValue;
    const int64_t blocks = f32_row_tiles(total_rows, p.num_seqs);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const int dp = (p.d + 31) / 32 * 32;
    const F32Kernel k = dp == 32 ? k32 : dp == 64 ? k64 : dp == 96 ? k96 : k128;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks, (unsigned)heads, (unsigned)splits), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_f32mfma(const FwdArgs& a, hipStream_t st) {
    F32Params p = make_params(a.geo);
    p.q = (const float*)a.q; p.k = (const float*)a.k; p.v = (const float*)a.v;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs;
    p.o = (float*)a.o; p.lse = a.lse;
    const int splits = a.f32_part != nullptr && a.f32_splits > 1 ? a.f32_splits : 1;
    p.part = splits > 1 ? a.f32_part : nullptr;
    p.nsplit = splits;
    hipError_t e = launch(p, a.geo.total_q, a.geo.hq, st, f32_fwd_kernel<32>, f32_fwd_kernel<64>,
                          f32_fwd_kernel<96>, f32_fwd_kernel<128>, splits);
    if (e != hipSuccess || splits == 1 || a.geo.total_q <= 0) return e;
    const int64_t n = a.geo.total_q * a.geo.hq * (a.geo.d / 4);
    hipLaunchKernelGGL(f32_fwd_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.part, splits,
                       a.geo.cu_q, a.geo.num_seqs, a.geo.total_q, a.geo.hq, a.geo.d, p.o, p.lse);
    return hipGetLastError();
}

hipError_t launch_bwd_dq_f32mfma(const BwdArgs& a, hipStream_t st) {
    F32Params p = make_params(a.geo);
    p.q = (const float*)a.q; p.k = (const float*)a.k; p.v = (const float*)a.v; p.dout = (const float*)a.dout;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs; p.do_rs = a.do_rs;
    p.lse_in = a.lse; p.delta = a.delta; p.dq = (float*)a.dq;
    if (a.o != nullptr && a.delta_out != nullptr) {
        p.o_in = (const float*)a.o; p.o_rs = a.o_rs; p.delta_out = a.delta_out;
    }
    const int splits = a.f32_part != nullptr && a.f32_splits > 1 ? a.f32_splits : 1;
    p.part = splits > 1 ? a.f32_part : nullptr;
    p.nsplit = splits;
    hipError_t e = launch(p, a.geo.total_q, a.geo.hq, st, f32_dq_kernel<32>, f32_dq_kernel<64>, f32_dq_kernel<96>,
                          f32_dq_kernel<128>, splits);
    if (e != hipSuccess || splits == 1 || a.geo.total_q <= 0) return e;
    const int64_t n4 = a.geo.total_q * a.geo.hq * a.geo.d / 4;
    hipLaunchKernelGGL(f32_split_sum_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, p.part, splits,
                       n4, p.scale, p.dq, nullptr);
    return hipGetLastError();
}

hipError_t launch_bwd_dkv_f32mfma(const BwdArgs& a, hipStream_t st) {
    F32Params p = make_params(a.geo);
    p.q = (const float*)a.q; p.k = (const float*)a.k; p.v = (const float*)a.v; p.dout = (const float*)a.dout;
    p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs; p.do_rs = a.do_rs;
    p.lse_in = a.lse; p.delta = a.delta; p.dk = (float*)a.dk; p.dv = (float*)a.dv;
    const int splits = a.f32_part != nullptr && a.f32_splits > 1 ? a.f32_splits : 1;
    p.part = splits > 1 ? a.f32_part : nullptr;
    p.nsplit = splits;
    hipError_t e = launch(p, a.geo.total_kv, a.geo.hkv, st, f32_dkv_kernel<32>, f32_dkv_kernel<64>,
                          f32_dkv_kernel<96>, f32_dkv_kernel<128>, splits);
    if (e != hipSuccess || splits == 1 || a.geo.total_kv <= 0) return e;
    const int64_t n4 = a.geo.total_kv * a.geo.hkv * a.geo.d / 4;
    hipLaunchKernelGGL(f32_split_sum_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, p.part, splits,
                       n4, p.scale, p.dk, p.dv);
    return hipGetLastError();
}

}  // namespace mtlattn
