// Device-side building blocks shared by the gfx950 attention kernels:
// element types, bf16/fp16 <-> fp32 conversion, MFMA wrappers with their lane
// layouts, LDS swizzles and varlen tile bookkeeping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtlattn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// ---------------------------------------------------------------------------
// Element types. Storage is the raw 16-bit pattern (or fp32).
// ---------------------------------------------------------------------------
struct BF16 {
    using raw = uint16_t;
    static constexpr int code = 2;
    __device__ static inline float to_float(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
    // lo/hi packed into one dword, round-to-nearest-even (v_cvt_pk_bf16_f32)
    __device__ static inline uint32_t pack2(float lo, float hi) {
        bf16x2_t v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    __device__ static inline uint16_t from_float(float x) {
        __bf16 b = (__bf16)x;
        return __builtin_bit_cast(uint16_t, b);
    }
};

struct F16 {
    using raw = uint16_t;
    static constexpr int code = 1;
    __device__ static inline float to_float(uint16_t x) {
        return (float)__builtin_bit_cast(_Float16, x);
    }
    __device__ static inline uint32_t pack2(float lo, float hi) {
        f16x2_t v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    __device__ static inline uint16_t from_float(float x) {
        _Float16 h = (_Float16)x;
        return __builtin_bit_cast(uint16_t, h);
    }
};

struct F32 {
    using raw = float;
    static constexpr int code = 0;
    __device__ static inline float to_float(float x) { return x; }
    __device__ static inline float from_float(float x) { return x; }
};

// Unpack element e (0/1) of a dword holding two 16-bit values.
template <typename T>
__device__ inline float lo16(uint32_t w) { return T::to_float((uint16_t)(w & 0xffffu)); }
template <typename T>
__device__ inline float hi16(uint32_t w) { return T::to_float((uint16_t)(w >> 16)); }

// ---------------------------------------------------------------------------
// MFMA wrappers. Operands are 8 packed 16-bit values in a u32x4.
//
// v_mfma_f32_32x32x16_{bf16,f16}: C[32x32] += A[32x16] * B[16x32]
//   A: lane l holds row m = l%32, k = 8*(l/32) + j in dword j/2 (j = 0..7)
//   B: lane l holds col n = l%32, k = 8*(l/32) + j
//   C: lane l holds col n = l%32, rows m = 8*(r/4) + 4*(l/32) + r%4, r = 0..15
// v_mfma_f32_16x16x32_{bf16,f16}: C[16x16] += A[16x32] * B[32x16]
//   A: lane l holds row m = l%16, k = 8*(l/16) + j
//   B: lane l holds col n = l%16, k = 8*(l/16) + j
//   C: lane l holds col n = l%16, rows m = 4*(l/16) + r, r = 0..3
// The contraction index k may be permuted freely as long as A and B agree;
// the kernels use that to feed softmax results straight from C registers.
// ---------------------------------------------------------------------------
template <typename T>
__device__ inline f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c);
template <>
__device__ inline f32x16_t mfma32<BF16>(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x16_t mfma32<F16>(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// c += a * b with the accumulator pinned to the accumulation registers
// (AGPRs), as inline asm: for kernels whose accumulators fill the AGPRs while
// the VGPRs hold everything else. The compiler's hazard tracking does not
// see these, so each carries its own s_nop 1: the two wait states an MFMA
// needs after a VALU instruction wrote its a or b (the compiler may copy an
// operand into place right before the asm). Readers of c keep their own
// distance from the last of these.
template <typename T>
__device__ inline void mfma32_acc(f32x16_t& c, const u32x4_t& a, const u32x4_t& b);
template <>
__device__ inline void mfma32_acc<BF16>(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
template <>
__device__ inline void mfma32_acc<F16>(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

template <typename T>
__device__ inline f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c);
template <>
__device__ inline f32x4_t mfma16<BF16>(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x4_t mfma16<F16>(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Global / LDS vector access helpers.
// ---------------------------------------------------------------------------
__device__ inline u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }
__device__ inline void st16(void* p, const u32x4_t& v) { *reinterpret_cast<u32x4_t*>(p) = v; }
__device__ inline u32x2_t ld8(const void* p) { return *reinterpret_cast<const u32x2_t*>(p); }
__device__ inline void st8(void* p, const u32x2_t& v) { *reinterpret_cast<u32x2_t*>(p) = v; }

// Two 16-bit values (low halves / high halves of a and b) packed into a dword.
__device__ inline uint32_t pack_lo16(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ inline uint32_t pack_hi16(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

// Transpose 4 rows x 8 columns of 16-bit values (each row one u32x4) into
// 8 columns x 4 rows: out[c] = {row0[c], row1[c], row2[c], row3[c]} as a u32x2.
__device__ inline void transpose4x8(const u32x4_t r[4], u32x2_t out[8]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        out[2 * w + 0] = u32x2_t{pack_lo16(r[0][w], r[1][w]), pack_lo16(r[2][w], r[3][w])};
        out[2 * w + 1] = u32x2_t{pack_hi16(r[0][w], r[1][w]), pack_hi16(r[2][w], r[3][w])};
    }
}

// Sum of two packed 16-bit values, accumulated in fp32 (v_dot2 with 1.0).
template <typename T> __device__ inline float dot2_ones(uint32_t w, float acc);
template <> __device__ inline float dot2_ones<BF16>(uint32_t w, float acc) {
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, acc, false);
}
template <> __device__ inline float dot2_ones<F16>(uint32_t w, float acc) {
    const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, acc, false);
}

// exp(a) in fp32 for the fp32 kernels. exp2(a * log2 e) with the product
// rounded is off by up to |a log2 e| / 2 ulp (8 ulp at a = 10, which softmax
// arguments reach); here the product's rounding error e (an FMA) and the
// part of log2 e below fp32 are kept and applied to first order:
// exp(a) = 2^t (1 + e ln 2), t = fl(a * L). With 2^t correctly rounded
// this is within 1.9 ulp over [-100, 88] (mean 0.4; the rounded product
// alone: 64 ulp), to which v_exp_f32 adds its own error. a is clamped at
// -104 (exp(-104) is below the smallest fp32 denormal) so -inf gives 0
// without a NaN. The clamp is a compare, not fmaxf: fmaxf(NaN, -104) is
// -104, which would turn a NaN logit into a weight of 0; a NaN compares
// false and passes through.
__device__ inline float exp_fp32(float a) {
    constexpr float kL = 1.44269502162933349609375f;   // log2(e) rounded to fp32
    constexpr float kLlo = 1.925963e-08f;              // log2(e) - kL
    a = a < -104.f ? -104.f : a;
    const float t = a * kL;
    const float e = fmaf(a, kL, -t) + a * kLlo;
    return __builtin_amdgcn_exp2f(t) * fmaf(e, kLn2, 1.f);
}

// max(a, b) that returns NaN when either is NaN (fmaxf returns the other
// operand): used where a NaN must survive a max, e.g. a split's LSE.
__device__ inline float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }

// max / sum of x over lanes l and l ^ 32 via v_permlane32_swap: swapping a
// register with itself across the halves leaves every lane holding its own
// value in one result and its partner's in the other.
__device__ inline float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------------------
// Direct HBM -> LDS staging and transposed operand reads (gfx950).
//
// The gfx950 LDS serves 256 bytes per clock from 64 four-byte banks: a
// ds_read_b128 is served 16 lanes at a time, a ds_read_b64(_tr_b16) 32 lanes
// at a time, and an access is conflict free when those lanes hit 16 (resp.
// 32) distinct bank groups. A row-major tile [rows][D] of 16-bit values keeps
// its 16-byte chunks XOR-swizzled per row so that both operand patterns are:
//  * row reads (ds_read_b128, MFMA operand rows): 16 consecutive rows, one
//    chunk -> the swizzle must be a bijection on 16 consecutive rows;
//  * transposed reads (ds_read_b64_tr_b16, see tr_operand): 4 rows
//    {4a..4a+3} x 4 chunks {4p..4p+3} -> the swizzle's chunk bits 2-3 must
//    separate rows 4a..4a+3.
// D = 128 (one row = 256 B = all banks): s(row) = (row & 3) << 2 | (row >> 2) & 3.
// D = 64 (two rows per 256 B, the odd row in the upper half):
//   s(row) = ((row >> 1) & 1) << 2 | (row >> 2) & 3.
// Direct-load writes (global_load_lds_dwordx4) are 1 KB contiguous per
// instruction and conflict free under any swizzle.
// ---------------------------------------------------------------------------
// D = 256 (512-byte rows, each covering the banks twice): the D = 128
// swizzle on the low 4 chunk bits; both access patterns only constrain a
// chunk's bank group, chunk & 15.
template <int D>
__device__ inline int row_swz(int row) {
    static_assert(D == 64 || D == 128 || D == 256, "swizzled tiles are defined for D = 64, 128 and 256");
    return D != 64 ? (((row & 3) << 2) | ((row >> 2) & 3)) : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

template <int D>
__device__ inline uint32_t tile_offset(int row, int chunk) {   // bytes
    return (uint32_t)(row * (2 * D) + ((chunk ^ row_swz<D>(row)) << 4));
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// Element offset of the bias row of global query row `grow`, in sequence s
// whose rows start at `qstart`: grow * qs (rows indexed globally, the
// reference's layout), or s * ss + min(grow - qstart, rows - 1) * qs when
// ss >= 0 (rows per sequence: a dense [B, H, Nq, Nkv] mask used in place;
// rows past a sequence block read its last row).
__device__ inline int64_t bias_row_offset(int64_t grow, int s, int64_t qstart, int64_t qs, int64_t ss,
                                          int64_t rows) {
    if (ss < 0) return grow * qs;
    const int64_t i = grow - qstart;
    return (int64_t)s * ss + (i < rows ? i : rows - 1) * qs;
}

// LDS direct loads (global_load_lds_*): each lane's data lands at LDS
// lds + (4 or 16) * lane. Issued as inline asm so the compiler's wait-count
// bookkeeping does not see them: the compiler conservatively waits for every
// outstanding direct load before any transposed LDS read (ds_read_b64_tr)
// and before barriers, which would drain the staging pipeline each tile.
// Callers therefore order these loads themselves (wait_vmcnt, then a barrier)
// before LDS reads of the staged data. `lds` (passed in M0) must be
// wave-uniform. The s_nop covers the one wait state required between an M0
// write and an LDS direct load.
//
// 4 bytes per lane from a per-lane address.
__device__ inline void lds_dma4(const void* gptr, const char* lds) {
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(gptr), "{m0}"(a) : "memory");
}
// 4 bytes per lane from a wave-uniform base plus a 32-bit per-lane byte
// offset (the instruction's SADDR form: no 64-bit address arithmetic).
__device__ inline void lds_dma4s(const void* sbase, uint32_t voff, const char* lds) {
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(a) : "memory");
}
// 16 bytes per lane, SADDR form as above.
__device__ inline void lds_dma16s(const void* sbase, uint32_t voff, const char* lds) {
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(a) : "memory");
}

// Stages rows [row0, row0 + ROWS) of a [*, D] 16-bit matrix (row stride rs
// elements) into a swizzled LDS tile with global_load_lds_dwordx4: each
// instruction moves 1 KB and lands lane l's 16 bytes at tile + 16 l, so the
// lane loads the global chunk that the swizzle maps to that LDS position.
// NW waves share the ROWS * D * 2 / 1024 instructions; w must be uniform.
// Rows of the source hold DV <= D values (head dims below the tile width):
// chunks at or past DV / 8 repeat the row's last valid chunk (finite data
// that the kernels' zero operand columns or discarded outputs never use).
// The per-lane part is fixed once: off[j] is the byte offset, from the
// tile's first row, of what this lane loads in its j-th instruction, so a
// full tile costs its DMA instructions and no vector arithmetic (the row
// base is scalar). A tile that runs past row_end recomputes the offsets with
// rows >= row_end reading row row_end - 1 (finite data the kernels mask
// out). The offsets are 32-bit: callers keep ROWS * 2 * rs below 2^32 (row
// strides below 2^25 elements for 64-row tiles).
template <int D, int ROWS, int NW, int DV = D>
struct TileStager {
    static_assert(DV % 8 == 0 && DV <= D, "head dim");
    static_assert(ROWS * D * 2 % 1024 == 0, "tile must be a multiple of 1 KB");
    static constexpr int PER = ROWS * D * 2 / 1024;     // instructions per tile
    static constexpr int N = (PER + NW - 1) / NW;       // per loader wave
    uint32_t off[N];

    __device__ static int row_of(int i, int lane) { return (i * 1024 + lane * 16) / (2 * D); }
    __device__ static uint32_t lane_off(int i, int lane, int grow, uint32_t rs2) {
        const int byte = i * 1024 + lane * 16;
        const int chunk = min(((byte % (2 * D)) >> 4) ^ row_swz<D>(row_of(i, lane)), DV / 8 - 1);
        return (uint32_t)grow * rs2 + (uint32_t)chunk * 16u;
    }
    // w: this wave's loader index in [0, NW)
    __device__ void init(int64_t rs, int w, int lane) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = w + j * NW;
            off[j] = (PER % NW == 0 || i < PER) ? lane_off(i, lane, row_of(i, lane), (uint32_t)(2 * rs)) : 0u;
        }
    }
    // rows [row0, row0 + ROWS) of base (row0 < row_end) into tile
    __device__ void issue(char* tile, const uint16_t* base, int64_t rs, int row0, int row_end, int w,
                          int lane) const {
        issue_at(tile, base + (int64_t)row0 * rs, rs, row_end - row0, w, lane);
    }
    // ROWS rows from tile_row0 (the tile's first row) into tile, when only
    // the first `avail` >= 1 of them exist
    __device__ void issue_at(char* tile, const uint16_t* tile_row0, int64_t rs, int avail, int w,
                             int lane) const {
        const char* tb = reinterpret_cast<const char*>(tile_row0);
        if (avail >= ROWS) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = w + j * NW;
                if (PER % NW != 0 && i >= PER) break;
                lds_dma16s(tb, off[j], tile + i * 1024);
            }
        } else {
            const int rmax = max(avail - 1, 0);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = w + j * NW;
                if (PER % NW != 0 && i >= PER) break;
                lds_dma16s(tb, lane_off(i, lane, min(row_of(i, lane), rmax), (uint32_t)(2 * rs)), tile + i * 1024);
            }
        }
    }
};

// Stages the fp32 bias of a key tile -- ROWS query rows x 64 keys, one
// head-broadcast block shared by every wave of a workgroup -- into LDS with
// global_load_lds_dwordx4: rows of 256 bytes, 16-byte chunk c of row r at
// position c ^ (r & 15), so that 16 consecutive rows read at one chunk (the
// MFMA C layout: lane = query row) hit 16 distinct bank groups. Instruction
// i (1 KB) fills rows 4i .. 4i + 3; 8 waves share the ROWS / 4 instructions.
// A lane's source is its row's bias row plus the tile's first column: the
// row part is a fixed 32-bit byte offset from the workgroup's first row
// (rows past a sequence's end repeat its last row), the column part the
// chunk. Columns at or past `cols` (a multiple of 4) are never read: a
// tile crossing `cols` loads the row's last chunk in their place, and the
// readers zero those keys.
template <int ROWS>
struct BiasStager {
    static_assert(ROWS == 32 || ROWS == 64, "bias tile rows");
    static constexpr int PER = ROWS / 4;   // 1 KB instructions per tile
    static constexpr int N = PER / 8;      // per wave
    uint32_t roff[N];                      // byte offset of the lane's row from row 0
    int chunk[N];                          // chunk the lane loads
    // row_off(r): element offset of WG row r's bias row (r = 0 .. ROWS - 1)
    template <typename RowOff>
    __device__ void init(RowOff row_off, int w, int lane) {
        const int64_t base = row_off(0);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int r = 4 * (w + 8 * j) + (lane >> 4);
            chunk[j] = (lane & 15) ^ (r & 15);
            roff[j] = (uint32_t)((row_off(r) - base) * 4);
        }
    }
    // row0: bias row of WG row 0 (wave-uniform); keys kt .. kt + 63
    __device__ void issue(char* tile, const float* row0, int kt, int cols, int w) const {
        if (kt + 64 <= cols) {
#pragma unroll
            for (int j = 0; j < N; ++j) lds_dma16s(row0 + kt, roff[j] + 16u * (uint32_t)chunk[j], tile + (w + 8 * j) * 1024);
        } else {   // columns clamped to the row's last chunk
#pragma unroll
            for (int j = 0; j < N; ++j)
                lds_dma16s(row0, roff[j] + 4u * (uint32_t)min(kt + 4 * chunk[j], cols - 4), tile + (w + 8 * j) * 1024);
        }
    }
};
// Byte offset, within a staged bias tile, of chunk (8 a + 2 b + hi) of row
// rr is bias_base(rr, hi) ^ (16 (8 a + 2 b)).
__device__ inline uint32_t bias_base(int rr, int hi) { return (uint32_t)(rr * 256 + 16 * (hi ^ (rr & 15))); }

// Wait until at most N of this wave's vector memory operations are pending
// (s_waitcnt vmcnt(N), other counters untouched); N <= 15.
template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");   // 6 bits: [3:0] and [15:14]
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Scheduling hint for the region just emitted: N MFMAs that each consume R
// LDS reads go out with the reads AHEAD operands in front of the MFMA that
// uses them (the default schedule issues each operand's reads just before
// its MFMA and waits for them there).
template <int R, int N, int AHEAD>
__device__ inline void pipe_reads() {
    __builtin_amdgcn_sched_group_barrier(0x100, R * AHEAD, 0);   // LDS reads
#pragma unroll
    for (int i = 0; i < N - AHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
}

// Keeps a per-iteration address opaque to the optimiser, so constant offsets
// fold into the LDS instructions' offset fields and per-lane XOR variants are
// formed per use instead of being hoisted out of the loop as live registers.
__device__ inline const char* opaque(const char* p) {
    uint32_t v = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
    asm volatile("" : "+v"(v));
    return (const char*)(const __attribute__((address_space(3))) char*)(uintptr_t)v;
}
// p ^ x on an LDS address (x below the row size, 512 bytes at most; tiles
// start on row-size boundaries, so this XORs the within-row byte offset).
__device__ inline const char* lds_xor(const char* p, uint32_t x) {
    const uint32_t v = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
    return (const char*)(const __attribute__((address_space(3))) char*)(uintptr_t)(v ^ x);
}

// Row operand reads. Lane (l32, hi) of a 32x32x16 MFMA operand reads row
// l32 (+ any multiple of 16 rows) at chunk 2 kc + hi. Since 2 kc + hi =
// 2 kc ^ hi and the swizzle is an XOR, chunk 2 kc + hi of row l32 sits at
// row_base ^ (32 kc): one per-lane base per tile, one v_xor per k-chunk.
template <int D>
__device__ inline uint32_t row_base(int l32, int hi) { return tile_offset<D>(l32, hi); }
template <int D>
__device__ inline u32x4_t row_operand(const char* rb, int kc, int row_off) {
    return ld16(lds_xor(rb, 32 * kc) + row_off * 2 * D);
}

// 32x32x16 MFMA operand whose M index runs along the D columns of a
// row-major tile and whose K index runs along its rows: M = columns
// 32 db .. 32 db + 31, K slots j of lane half h = rows
// 16 c + 8 (j / 4) + 4 h + j % 4. Two ds_read_b64_tr_b16 (K slots 0-3, then
// 4-7 eight rows down): in each 16-lane group, lane 4e + q addresses row e
// of the group's 4 rows at columns 4q .. 4q + 3, and lane i receives column
// i of all 4 rows.
//
// Addresses: the swizzle depends on row & 15 only, so 16 c rows are a plain
// offset; column block db XORs swizzled chunk bits 2-3 (byte 64 db) and the
// second read (+8 rows) XORs chunk bit 1 (byte 32), so every read is
// tr_base ^ const + const.
template <int D>
__device__ inline uint32_t tr_base(int lane) {
    const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
    const int col = 16 * (g & 1) + 4 * q;
    const int row = 4 * (g >> 1) + e;
    return tile_offset<D>(row, col >> 3) + (col & 7) * 2;
}
template <int D>
__device__ inline u32x4_t tr_operand(const char* tb, int c, int db) {
    const char* p0 = lds_xor(tb, 64 * db) + c * 16 * 2 * D;
    const char* p1 = lds_xor(tb, 64 * db + 32) + (c * 16 + 8) * 2 * D;
    const v4i16_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p0);
    const v4i16_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p1);
    const u32x2_t a2 = __builtin_bit_cast(u32x2_t, a), b2 = __builtin_bit_cast(u32x2_t, b);
    return u32x4_t{a2[0], a2[1], b2[0], b2[1]};
}

// ---------------------------------------------------------------------------
// Mask bands. With end-aligned causal masking (coff = kv_len - q_len) and a
// sliding window W, query i may attend key j iff
//   j < kv_len, (!causal || j <= i + coff), (W <= 0 || j > i + coff - W).
// For one query row the allowed keys form [lo, lo + width); for one key the
// allowed queries (also < q_len) form an interval too. A test is then one
// unsigned compare: (unsigned)(k - lo) < width.
// ---------------------------------------------------------------------------
struct Band {
    int lo;
    uint32_t width;
    __device__ inline bool has(int k) const { return (uint32_t)(k - lo) < width; }
};
__device__ inline Band key_band(int qrow, int coff, int kv_len, int causal, int window) {
    const int lo = window > 0 ? max(0, qrow + coff - window + 1) : 0;
    const int hi = causal ? min(kv_len, qrow + coff + 1) : kv_len;
    return Band{lo, (uint32_t)max(0, hi - lo)};
}
__device__ inline Band query_band(int key, int coff, int q_len, int kv_len, int causal, int window) {
    const int lo = causal ? max(0, key - coff) : 0;
    const int hi = key >= kv_len ? lo : (window > 0 ? min(q_len, key - coff + window) : q_len);
    return Band{lo, (uint32_t)max(0, hi - lo)};
}

// ---------------------------------------------------------------------------
// Wave reductions (64 lanes).
// ---------------------------------------------------------------------------
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ---------------------------------------------------------------------------
// Varlen bookkeeping.
// Tiles of `tile` rows are numbered globally without a host sync: sequence s
// owns tiles [T_s, T_{s+1}) with T_s = cu[s] / tile + s, which always covers
// ceil(len_s / tile) tiles. A grid of total / tile + num_seqs + 1 blocks is an
// upper bound computable from tensor shapes alone.
// ---------------------------------------------------------------------------
struct SeqRange {
    int start, end;   // clamped to [0, total]
};

__device__ inline SeqRange seq_range(const int* __restrict__ cu, int s, int64_t total) {
    int a = cu[s], b = cu[s + 1];
    const int t = (int)total;
    a = a < 0 ? 0 : (a > t ? t : a);
    b = b < a ? a : (b > t ? t : b);
    return {a, b};
}

// Largest s in [0, num_seqs) with cu[s] / tile + s <= t (binary search; all
// lanes compute the same value).
__device__ inline int find_seq_for_tile(const int* __restrict__ cu, int num_seqs, int tile, int t,
                                        int64_t total) {
    int lo = 0, hi = num_seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        int c = cu[mid];
        c = c < 0 ? 0 : (c > (int)total ? (int)total : c);
        if (c / tile + mid <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ inline int tile_base(const int* __restrict__ cu, int s, int tile, int64_t total) {
    int c = cu[s];
    c = c < 0 ? 0 : (c > (int)total ? (int)total : c);
    return c / tile + s;
}

// Map a linear block id so that consecutive logical ids run on the same XCD
// (blocks are dispatched round-robin over the 8 XCDs of an MI355X), keeping
// the K/V of one (sequence, head) in one XCD's L2.
__device__ inline int xcd_remap(int id, int n) {
    if ((n & 7) != 0) return id;
    return (id & 7) * (n >> 3) + (id >> 3);
}

}  // namespace mtlattn
