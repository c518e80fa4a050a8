// Measured ceilings of the GPU this runs on, for bench.py's fractions of
// roofline (libmtlattn_calib.so; not part of the attention library's ABI).
//
//  * mtlattn_calib_mfma: sustained v_mfma_f32_32x32x16_bf16 throughput. Every
//    wave streams `iters` x 8 MFMAs over four independent accumulator chains
//    (operands in registers, no memory traffic in the loop) -- the matrix-core
//    rate the attention kernels' own instruction stream could at best reach
//    at the clock the GPU holds under such load. One block of 8 waves per
//    `blocks`; use a multiple of the CU count.
//  * mtlattn_calib_read: HBM read bandwidth. Each block streams a contiguous
//    span of `bytes` / blocks with 16-byte nontemporal loads, folded into one
//    word per lane and written once per block, so the only traffic is the
//    stream itself.
//
// Both report shader-clock cycles and reference-clock ticks of the first wave
// (s_memtime / s_memrealtime, the latter at 100 MHz) so the caller can derive
// the shader clock during the run.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(512, 1) void calib_mfma_kernel(int iters, float* sink, unsigned long long* clk) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const u32x4_t a = {0x3f803f80u ^ (uint32_t)lane, 0x3f803f80u, 0x3c003c00u, 0x3f803f80u ^ (uint32_t)w};
    const u32x4_t b = {0x3c003c00u, 0x3f803f80u ^ (uint32_t)lane, 0x3f803f80u, 0x3c003c00u};
    const bf16x8_t A = __builtin_bit_cast(bf16x8_t, a), B = __builtin_bit_cast(bf16x8_t, b);
    f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    unsigned long long t0 = 0, r0 = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        t0 = __builtin_amdgcn_s_memtime();
        r0 = __builtin_amdgcn_s_memrealtime();
    }
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c3, 0, 0, 0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
    if (s == 1.2345f) sink[blockIdx.x * 512 + threadIdx.x] = s;   // keeps the chains live
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clk[0] = __builtin_amdgcn_s_memtime() - t0;
        clk[1] = __builtin_amdgcn_s_memrealtime() - r0;
    }
}

// Each block streams one contiguous span; every lane keeps eight 16-byte
// nontemporal loads in flight (each wave instruction covers 1 KB).
constexpr int kReadUnroll = 8;
__global__ __launch_bounds__(256) void calib_read_kernel(const u32x4_t* __restrict__ src, int64_t per_block,
                                                         uint32_t* __restrict__ sink, unsigned long long* clk) {
    unsigned long long t0 = 0, r0 = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        t0 = __builtin_amdgcn_s_memtime();
        r0 = __builtin_amdgcn_s_memrealtime();
    }
    const u32x4_t* p = src + (int64_t)blockIdx.x * per_block + threadIdx.x;
    uint32_t acc = 0;
    for (int64_t i = 0; i < per_block; i += kReadUnroll * 256) {
        u32x4_t x[kReadUnroll];
#pragma unroll
        for (int j = 0; j < kReadUnroll; ++j) x[j] = __builtin_nontemporal_load(p + i + j * 256);
#pragma unroll
        for (int j = 0; j < kReadUnroll; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clk[0] = __builtin_amdgcn_s_memtime() - t0;
        clk[1] = __builtin_amdgcn_s_memrealtime() - r0;
    }
}

// Issue-rate probes. One block of 8 waves per CU; waves w and w + 4 share a
// SIMD. Waves 0-3 run role ra, waves 4-7 role rb, each `iters` iterations:
//   0 idle
//   1 v_exp_f32: 16 independent chains per iteration
//   2 v_fmac_f32: 16 independent chains per iteration
//   3 v_mfma_f32_32x32x16_bf16, accumulators in VGPRs: 8 per iteration over 4
//     independent accumulators
//   4 the same with the accumulators in AGPRs
//   5 ds_read_b128: 16 reads (16 KB per wave) in flight, then a wait
//   6 one wave interleaving both: role 3's 8 MFMAs, each followed by two
//     v_exp_f32 and two v_fmac_f32 of independent chains
//   7 the same with four v_exp_f32 after each MFMA
//   8 role 6 with the MFMA's first operand read from LDS (ds_read_b128 four
//     MFMAs ahead, s_waitcnt lgkmcnt(3) before each MFMA)
//   9 role 6 with the attention softmax's dependences: per MFMA two
//     v_fma_f32 -> v_exp_f32 pairs, one v_cvt_pk_bf16_f32 of the previous
//     pair and one v_dot2c_f32_bf16 row-sum step on the pair before that
//  10 global_load_lds_dwordx4 (1 KB direct-to-LDS loads of an L2-resident
//     1 KB source): 8 per iteration, at most 16 in flight
//  11 role 3's 8 MFMAs per iteration in one wave with 2 of role 10's loads
//     between them (after MFMAs 1 and 5), at most 8 loads in flight
//  12 role 8 with each LDS operand shared by two MFMAs (one ds_read_b128
//     per two MFMAs, four reads ahead): 0.5 KB of LDS per MFMA
// The instructions are inline asm so that their number and order are
// exactly these. Each wave records its s_memtime cycles (shader clock) and
// s_memrealtime ticks (100 MHz).
constexpr int kRateOps[13] = {0, 16, 16, 8, 8, 16, 8, 8, 8, 8, 8, 8, 8};   // roles 6-9, 11, 12: MFMAs

__device__ float rate_role(int role, int iters, int lane, const char* lds, const float* src) {
    float x[18];
#pragma unroll
    for (int j = 0; j < 18; ++j) x[j] = 0.3f + 0.01f * j + 1e-4f * lane;
    const u32x4_t a = {0x3f803f80u ^ (uint32_t)lane, 0x3f803f80u, 0x3c003c00u, 0x3f803f80u};
    const u32x4_t b = {0x3c003c00u, 0x3f803f80u ^ (uint32_t)lane, 0x3f803f80u, 0x3c003c00u};
    f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    u32x4_t r[16];
    if (role == 1) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) asm volatile("v_exp_f32 %0, %0" : "+v"(x[j]));
    } else if (role == 2) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[j]) : "v"(x[16]), "v"(x[17]));
    } else if (role == 3) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
            }
    } else if (role == 4) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c0) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c1) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c2) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c3) : "v"(a), "v"(b));
            }
    } else if (role == 6) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    f32x16_t& c = m == 0 ? c0 : m == 1 ? c1 : m == 2 ? c2 : c3;
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
                    const int j = 4 * m + 2 * u;
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[j]));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 1]));
                    asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 8) & 15]) : "v"(x[16]), "v"(x[17]));
                    asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 9) & 15]) : "v"(x[16]), "v"(x[17]));
                }
    } else if (role == 7) {
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    f32x16_t& c = m == 0 ? c0 : m == 1 ? c1 : m == 2 ? c2 : c3;
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
                    const int j = 4 * m + 2 * u;
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[j]));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 1]));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[(j + 8) & 15]));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[(j + 9) & 15]));
                }
    } else if (role == 8) {
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
        // operand g of 8 rotating registers: KB (g & 7) + lane chunk, every
        // address a multiple of 16 below 8 KB
        auto rd = [&](int g) { return base + (uint32_t)(((g & 7) * 1024 + lane * 16) & 8191); };
#pragma unroll
        for (int g = 0; g < 4; ++g) asm volatile("ds_read_b128 %0, %1" : "=v"(r[g]) : "v"(rd(g)) : "memory");
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                f32x16_t& c = (g & 3) == 0 ? c0 : (g & 3) == 1 ? c1 : (g & 3) == 2 ? c2 : c3;
                asm volatile("s_waitcnt lgkmcnt(3)" ::: "memory");
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(r[g]), "v"(b));
                asm volatile("ds_read_b128 %0, %1" : "=v"(r[(g + 4) & 7]) : "v"(rd(g + 4)) : "memory");
                const int j = 2 * g;
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j]));
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 1]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 8) & 15]) : "v"(x[16]), "v"(x[17]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 9) & 15]) : "v"(x[16]), "v"(x[17]));
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else if (role == 9) {
        float e[16], sum = 0.f;
        uint32_t pk[8];
        const uint32_t ones = 0x3f803f80u;
#pragma unroll
        for (int j = 0; j < 16; ++j) e[j] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) pk[j] = 0u;
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                f32x16_t& c = (g & 3) == 0 ? c0 : (g & 3) == 1 ? c1 : (g & 3) == 2 ? c2 : c3;
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
                const int j = 2 * g;
                float t0, t1;
                asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(t0) : "v"(x[j]), "v"(x[16]), "v"(x[17]));
                asm volatile("v_exp_f32 %0, %1" : "=v"(e[j]) : "v"(t0));
                asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(t1) : "v"(x[j + 1]), "v"(x[16]), "v"(x[17]));
                asm volatile("v_exp_f32 %0, %1" : "=v"(e[j + 1]) : "v"(t1));
                const int pj = (j + 14) & 15;   // the previous pair
                asm volatile("s_nop 0\n\tv_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(pk[g]) : "v"(e[pj]), "v"(e[pj + 1]));
                asm volatile("v_dot2c_f32_bf16 %0, %1, %2" : "+v"(sum) : "v"(ones), "v"(pk[(g + 7) & 7]));
            }
        x[0] += sum;
    } else if (role == 10 || role == 11) {
        // source: 1 KB of this block's sink (lane chunk lane * 16); LDS
        // destination rotates over 8 KB of the buffer
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
        const uint32_t voff = (uint32_t)lane * 16u;
        auto dma = [&](int slot) {
            asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(src),
                         "{m0}"(base + (uint32_t)(slot & 7) * 1024u) : "memory");
        };
        if (role == 10) {
            for (int i = 0; i < iters; ++i) {
#pragma unroll
                for (int j = 0; j < 8; ++j) dma(j);
                asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            }
        } else {
            for (int i = 0; i < iters; ++i) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
                    dma(2 * u);
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
                }
                asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (role == 12) {
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
        auto rd = [&](int g) { return base + (uint32_t)(((g & 7) * 1024 + lane * 16) & 8191); };
#pragma unroll
        for (int g = 0; g < 4; ++g) asm volatile("ds_read_b128 %0, %1" : "=v"(r[g]) : "v"(rd(g)) : "memory");
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // operand r[g] feeds two MFMAs (two independent chains each)
                asm volatile("s_waitcnt lgkmcnt(3)" ::: "memory");
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(g & 1 ? c2 : c0) : "v"(r[g]), "v"(b));
                asm volatile("ds_read_b128 %0, %1" : "=v"(r[(g + 4) & 7]) : "v"(rd(g + 4)) : "memory");
                const int j = 4 * g;
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j]));
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 1]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 8) & 15]) : "v"(x[16]), "v"(x[17]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 9) & 15]) : "v"(x[16]), "v"(x[17]));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(g & 1 ? c3 : c1) : "v"(r[g]), "v"(a));
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 2]));
                asm volatile("v_exp_f32 %0, %0" : "+v"(x[j + 3]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 10) & 15]) : "v"(x[16]), "v"(x[17]));
                asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(x[(j + 11) & 15]) : "v"(x[16]), "v"(x[17]));
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else if (role == 5) {
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds;
        for (int i = 0; i < iters; ++i) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                // 16-byte chunk of lane `lane` in KB j of the 32 KB buffer: every
                // address is a multiple of 16 below 32768 - 16 + 16
                const uint32_t addr = base + (uint32_t)((lane * 16 + j * 1024 + i * 2048) & 32767);
                asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(addr) : "memory");
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int j = 0; j < 16; ++j) x[j & 15] += __uint_as_float(r[j][0] & 0x3fffffffu);
        }
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");   // MFMA results settle before the reads below
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += x[j] + c0[j] + c1[j] + c2[j] + c3[j];
    return sum;
}

__global__ __launch_bounds__(512, 1) void calib_rates_kernel(int ra, int rb, int iters, float* sink,
                                                             unsigned long long* cyc) {
    __shared__ __attribute__((aligned(1024))) char lds[32768];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < 32768 / 4; i += 512) reinterpret_cast<uint32_t*>(lds)[i] = (uint32_t)i * 0x9e3779b9u;
    __syncthreads();
    const int role = __builtin_amdgcn_readfirstlane(w < 4 ? ra : rb);   // wave-uniform
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    const float s = role ? rate_role(role, iters, lane, lds, sink + blockIdx.x * 512) : 0.f;
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (s == 1.2345f) sink[blockIdx.x * 512 + threadIdx.x] = s;   // keeps the streams live
    if (lane == 0) {
        cyc[(blockIdx.x * 8 + w) * 2] = t1 - t0;
        cyc[(blockIdx.x * 8 + w) * 2 + 1] = r1 - r0;
    }
}

}  // namespace

extern "C" {

// blocks x 8 waves x iters x 8 MFMAs of 32x32x16 (32768 FLOP each).
// sink: blocks * 512 floats; clk: 2 u64. Returns a hipError_t code.
int mtlattn_calib_mfma(int blocks, int iters, float* sink, unsigned long long* clk, void* stream) {
    if (blocks < 1 || iters < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(calib_mfma_kernel, dim3(blocks), dim3(512), 0, (hipStream_t)stream, iters, sink, clk);
    return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of blocks * 32 KiB) from src. sink: blocks * 4 words.
int mtlattn_calib_read(const void* src, int64_t bytes, int blocks, uint32_t* sink, unsigned long long* clk,
                       void* stream) {
    const int64_t span = (int64_t)kReadUnroll * 256 * 16;
    if (blocks < 1 || bytes < span || bytes % (span * blocks) != 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(calib_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4_t*)src, bytes / 16 / blocks, sink, clk);
    return (int)hipGetLastError();
}

// Issue-rate probe (see calib_rates_kernel): roles ra (waves 0-3) and rb
// (waves 4-7), `iters` iterations, one block per CU (`blocks` = CU count).
// sink: blocks * 512 floats; cyc: blocks * 8 * 2 u64 (per wave: shader
// cycles, 100 MHz ticks). Operations per iteration of role r: ops_per_iter.
int mtlattn_calib_rates(int ra, int rb, int iters, int blocks, float* sink, unsigned long long* cyc, void* stream) {
    if (ra < 0 || ra > 12 || rb < 0 || rb > 12 || iters < 1 || blocks < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(calib_rates_kernel, dim3(blocks), dim3(512), 0, (hipStream_t)stream, ra, rb, iters, sink, cyc);
    return (int)hipGetLastError();
}
int mtlattn_calib_rate_ops(int role) { return role >= 0 && role <= 12 ? kRateOps[role] : 0; }

}  // extern "C"
