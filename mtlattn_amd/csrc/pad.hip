// Key-padding pack / unpack for the SDPA adapter, on the device.
//
// The reference's adapter (mtlattn/__init__.py:202-249) turns a dense
// [B, H, N, D] self-attention call with a key-padding mask into a varlen call
// by copying each batch's valid prefix in a Python loop, after pulling the
// lengths to the host. Here the prefix sums and both copies run on the
// device: a batch's first lens[b] tokens go to packed rows cu[b] + n, the
// padded tokens after all valid ones (so the packed tensor keeps B * N rows
// and no host ever needs the total), and the unpack writes the dense output
// with zeros for padded query rows.
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels.h"

namespace mtlattn {

namespace {

// cu[0] = 0, cu[b + 1] = cu[b] + clamp(lens[b], 0, n): one workgroup, a
// chunked scan (B is a batch size).
__global__ void pad_prefix_kernel(const int* __restrict__ lens, int* __restrict__ cu, int B, int N) {
    __shared__ int part[256];
    const int t = threadIdx.x;
    const int per = (B + 255) / 256;
    const int b0 = t * per, b1 = min(B, b0 + per);
    int s = 0;
    for (int b = b0; b < b1; ++b) s += min(max(lens[b], 0), N);
    part[t] = s;
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int i = 0; i < 256; ++i) {
            const int x = part[i];
            part[i] = run;
            run += x;
        }
        cu[B] = run;
    }
    __syncthreads();
    int run = part[t];
    for (int b = b0; b < b1; ++b) {
        cu[b] = run;
        run += min(max(lens[b], 0), N);
    }
}

// One thread per (token, head, 16-byte chunk) when U = 16-byte vectors, per
// element otherwise. PACK: dense -> packed rows; else packed -> dense (zeros
// for padded tokens).
template <typename U, bool PACK>
__global__ __launch_bounds__(256) void pad_copy_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                                       const int* __restrict__ lens, const int* __restrict__ cu,
                                                       int B, int N, int H, int units, int64_t sb, int64_t sh,
                                                       int64_t sn) {
    const int64_t total = (int64_t)B * N * H * units;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int u = (int)(i % units);
        const int64_t r = i / units;
        const int h = (int)(r % H);
        const int64_t tok = r / H;
        const int n = (int)(tok % N), b = (int)(tok / N);
        const int len = min(max(lens[b], 0), N);
        // dense element offset (in units) and packed row
        const int64_t dense = (int64_t)b * sb + (int64_t)h * sh + (int64_t)n * sn + u;
        int64_t row = n < len ? (int64_t)cu[b] + n : (int64_t)cu[B] + (int64_t)b * N - cu[b] + n - len;
        // (cu from the matching pack keeps rows in range; any other cu is
        // clamped to the tensor instead of addressing outside it)
        row = row < 0 ? 0 : (row >= (int64_t)B * N ? (int64_t)B * N - 1 : row);
        const int64_t packed = (row * H + h) * units + u;
        const U* s = reinterpret_cast<const U*>(src);
        U* d = reinterpret_cast<U*>(dst);
        if (PACK) {
            d[packed] = s[dense];
        } else {
            d[dense] = n < len ? s[packed] : U{};
        }
    }
}

template <bool PACK>
hipError_t launch_copy(int esize, int B, int N, int H, int D, const void* src, void* dst, const int* lens,
                       const int* cu, int64_t sb, int64_t sh, int64_t sn, hipStream_t st) {
    const int64_t bytes_row = (int64_t)D * esize;
    const bool vec = bytes_row % 16 == 0 && ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0) &&
                     (sb * esize) % 16 == 0 && (sh * esize) % 16 == 0 && (sn * esize) % 16 == 0;
    const int64_t items = (int64_t)B * N * H * (vec ? bytes_row / 16 : D);
    if (items == 0) return hipSuccess;
    const int64_t blocks = (items + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
    if (vec) {
        const int k = 16 / esize;   // elements per vector
        hipLaunchKernelGGL((pad_copy_kernel<u32x4_t, PACK>), dim3(grid), dim3(256), 0, st, (const char*)src,
                           (char*)dst, lens, cu, B, N, H, (int)(bytes_row / 16), sb / k, sh / k, sn / k);
    } else if (esize == 4) {
        hipLaunchKernelGGL((pad_copy_kernel<uint32_t, PACK>), dim3(grid), dim3(256), 0, st, (const char*)src,
                           (char*)dst, lens, cu, B, N, H, D, sb, sh, sn);
    } else {
        hipLaunchKernelGGL((pad_copy_kernel<uint16_t, PACK>), dim3(grid), dim3(256), 0, st, (const char*)src,
                           (char*)dst, lens, cu, B, N, H, D, sb, sh, sn);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_pad_pack(int esize, int B, int N, int H, int D, const void* src, int64_t sb, int64_t sh,
                           int64_t sn, const int* lens, int* cu, void* dst, hipStream_t st) {
    hipLaunchKernelGGL(pad_prefix_kernel, dim3(1), dim3(256), 0, st, lens, cu, B, N);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_copy<true>(esize, B, N, H, D, src, dst, lens, cu, sb, sh, sn, st);
}

hipError_t launch_pad_unpack(int esize, int B, int N, int H, int D, const void* src, const int* lens, const int* cu,
                             void* dst, int64_t sb, int64_t sh, int64_t sn, hipStream_t st) {
    return launch_copy<false>(esize, B, N, H, D, src, dst, lens, cu, sb, sh, sn, st);
}

}  // namespace mtlattn
