// Device-side synthetic initialisation (the workload's seeded random-init weights/state).
//
// Stream definition (shared with the test oracle, which restates it independently):
//   mix(x)       = splitmix64 finaliser of (x + 0x9E3779B97F4A7C15)
//   key          = mix(mix(seed) + fnv1a64(tensor name))
//   r_j(i)       = mix(key + 3 i + j), j = 0, 1, 2
//   normal(i)    = (float)(sum of the 12 16-bit halves of r_0..r_2 - 393210) * (float)(std / 65536)
// Integer-exact up to one correctly rounded f32 multiply, so host, numpy and device
// agree bit for bit; values are rounded to bf16 with round-to-nearest-even.
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

__device__ __forceinline__ uint64_t dmix(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i, float scale) {
    int32_t s = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        uint64_t r = dmix(key + 3 * i + (uint64_t)j);
        s += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
             (int32_t)(r >> 48);
    }
    return __fmul_rn((float)(s - 393210), scale);
}

// Logical tensor [N][K] (row-major stream index n*K + k) written into a tiled matrix at
// row offset row_off of a combined weight with Kdst == K.
__global__ void gen_normal_tiled(uint64_t key, float scale, int N, int K, int row_off, uint16_t* dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * K;
    for (; i < total; i += (long long)gridDim.x * blockDim.x) {
        int n = (int)(i / K), k = (int)(i % K);
        dst[tiled_offset(n + row_off, k, K)] = f2bf(normal_at(key, (uint64_t)i, scale));
    }
}

__global__ void gen_normal_plain(uint64_t key, float scale, long long n, uint16_t* dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (long long)gridDim.x * blockDim.x) dst[i] = f2bf(normal_at(key, (uint64_t)i, scale));
}

__global__ void gen_normal_f32(uint64_t key, float scale, long long n, float* dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (long long)gridDim.x * blockDim.x) dst[i] = normal_at(key, (uint64_t)i, scale);
}

hipError_t launch_gen_normal_tiled(uint64_t key, float scale, int N, int K, int row_off_dst,
                                   uint16_t* dst, int Kdst, hipStream_t st) {
    if (K != Kdst || K % 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gen_normal_tiled, dim3(4096), dim3(256), 0, st, key, scale, N, K, row_off_dst, dst);
    return hipGetLastError();
}
// K cache seeding: element i = slot * 256 + d of the stream (the same values as a row-major
// fill) stored at the tiled position of (slot, d).
__global__ void gen_normal_kv_tiled(uint64_t key, float scale, long long n, uint16_t* dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (long long)gridDim.x * blockDim.x)
        dst[kv_tiled_offset((int)(i >> 8), (int)(i & 255))] = f2bf(normal_at(key, (uint64_t)i, scale));
}

// V cache rows of the plain stream's values (element i = slot * 256 + d) in the 8-slot layout
__global__ void gen_normal_kv_v8(uint64_t key, float scale, long long n, uint16_t* dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (long long)gridDim.x * blockDim.x)
        dst[kv_v8_offset((int)(i >> 8), (int)(i & 255))] = f2bf(normal_at(key, (uint64_t)i, scale));
}

hipError_t launch_gen_normal_kv_v8(uint64_t key, float scale, int n_slots, uint16_t* dst, hipStream_t st) {
    if (n_slots <= 0) return hipSuccess;
    hipLaunchKernelGGL(gen_normal_kv_v8, dim3(4096), dim3(256), 0, st, key, scale, (long long)n_slots * 256, dst);
    return hipGetLastError();
}

hipError_t launch_gen_normal_kv_tiled(uint64_t key, float scale, int n_slots, uint16_t* dst, hipStream_t st) {
    if (n_slots <= 0) return hipSuccess;
    hipLaunchKernelGGL(gen_normal_kv_tiled, dim3(4096), dim3(256), 0, st, key, scale, (long long)n_slots * 256, dst);
    return hipGetLastError();
}

hipError_t launch_gen_normal_plain(uint64_t key, float scale, long long n, uint16_t* dst, hipStream_t st) {
    hipLaunchKernelGGL(gen_normal_plain, dim3(4096), dim3(256), 0, st, key, scale, n, dst);
    return hipGetLastError();
}
hipError_t launch_gen_normal_f32(uint64_t key, float scale, long long n, float* dst, hipStream_t st) {
    hipLaunchKernelGGL(gen_normal_f32, dim3(4096), dim3(256), 0, st, key, scale, n, dst);
    return hipGetLastError();
}

}  // namespace q35

namespace q35 {

// Checkpoint row-major [N][K] <-> tiled layout (loader and test read-back).
__global__ void tile_kernel(const uint16_t* src, int N, int K, uint16_t* dst, int row_off, int inverse) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * K;
    for (; i < total; i += (long long)gridDim.x * blockDim.x) {
        int n = (int)(i / K), k = (int)(i % K);
        size_t t = tiled_offset(n + row_off, k, K);
        if (inverse) dst[i] = src[t];
        else dst[t] = src[i];
    }
}

hipError_t launch_tile(const uint16_t* src, int N, int K, uint16_t* dst, int row_off, int inverse,
                       hipStream_t st) {
    if (K % 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(tile_kernel, dim3(2048), dim3(256), 0, st, src, N, K, dst, row_off, inverse);
    return hipGetLastError();
}

// Copies row src_rows[i] of a [*][width] bf16 matrix to row dst_rows[i] of another.
__global__ void copy_rows_kernel(const uint16_t* src, const int* src_rows, uint16_t* dst,
                                 const int* dst_rows, int width) {
    const int i = blockIdx.x;
    const uint16_t* s = src + (size_t)src_rows[i] * width;
    uint16_t* d = dst + (size_t)dst_rows[i] * width;
    for (int k = threadIdx.x; k < width; k += blockDim.x) d[k] = s[k];
}

// copy_rows_kernel plus the decode step's metadata advance for row i (one row per lane): the
// row's position and slot move to the next one and its lane's state slot index turns over,
// so that the next decode step of the same lanes finds its metadata on the device (the
// sampled token is already in place: the argmax writes it to the token row)
__global__ void copy_rows_advance_kernel(const uint16_t* src, const int* src_rows, uint16_t* dst,
                                         const int* dst_rows, int width, int* pos, int* slot,
                                         int* cur, int* wcur, int* pend, int nslots, int defer) {
    const int i = blockIdx.x;
    const uint16_t* s = src + (size_t)src_rows[i] * width;
    uint16_t* d = dst + (size_t)dst_rows[i] * width;
    for (int k = threadIdx.x; k < width; k += blockDim.x) d[k] = s[k];
    if (threadIdx.x == 0) {
        pos[i] += 1;
        slot[i] += 1;
        const int p = pend[i];
        if ((p & 15) < defer) {
            pend[i] = p + 1;
        } else {
            cur[i] = (cur[i] + 1) % nslots;
            pend[i] = p & 16;
        }
        wcur[i] = (wcur[i] + 1) % nslots;
    }
}

hipError_t launch_copy_rows_advance(const uint16_t* src, const int* src_rows, uint16_t* dst, const int* dst_rows,
                                    int n, int width, int* pos, int* slot, int* cur, int* wcur, int* pend, int nslots,
                                    int defer, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(copy_rows_advance_kernel, dim3(n), dim3(256), 0, st, src, src_rows, dst, dst_rows, width,
                       pos, slot, cur, wcur, pend, nslots, defer);
    return hipGetLastError();
}

hipError_t launch_copy_rows(const uint16_t* src, const int* src_rows, uint16_t* dst, const int* dst_rows,
                            int n, int width, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(copy_rows_kernel, dim3(n), dim3(256), 0, st, src, src_rows, dst, dst_rows, width);
    return hipGetLastError();
}

}  // namespace q35
