// Row glue: embedding gather, residual add and zero-centred RMSNorm, MTP fc input.
//
// rmsnorm_zc follows speccheck/specimpl.py:135-139 (f32 math, (x * rsqrt(mean(x^2)+eps))
// rounded to f32, times (1+w), one bf16 rounding); the residual pairing follows
// specimpl.py:426-451 (bf16 adds). Replaces engine/kernels_glue.cpp:13-60 and
// engine/kernels_embed.cpp:65-80 of the reference.
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One row per block, 256 threads x 4 elements.
// The mode is a template argument: with a run-time mode the compiler waited for the residual
// row's load at the mode branch, before issuing the chain loads (two round trips instead of one).
// TILED: h in the weights' tiled fragment layout (tiled_offset with the row as n), the A operand
// of the many-row K = 1024 GEMM; a thread's 4 elements stay contiguous there.
template <int mode, bool TILED = false>
__global__ void __launch_bounds__(256) addnorm_kernel(const int* tok, const uint16_t* E,
                                                      uint16_t* x, const uint16_t* delta,
                                                      const float* kpart, int kblocks,
                                                      const uint16_t* w, uint16_t* h) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const int k = threadIdx.x * 4;
    // every load first: the GEMM k-block chains, then the residual row, then the norm weight
    float4 d[16];
    if (mode == 3 || mode == 4) {
        const size_t stride = (size_t)gridDim.x * kHidden;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb)
            if (kb < kblocks) d[kb] = *(const float4*)(kpart + kb * stride + (size_t)r * kHidden + k);
    }
    const uint2 wv = h ? *(const uint2*)(w + k) : make_uint2(0u, 0u);
    float xv[4];
    uint16_t* xr = x + (size_t)r * kHidden + k;
    if (mode == 0) {
        const uint16_t* er = E + tiled_offset(tok[r], k, kHidden);
        uint2 e = *(const uint2*)er;
        *(uint2*)xr = e;
        xv[0] = __uint_as_float(e.x << 16); xv[1] = __uint_as_float(e.x & 0xffff0000u);
        xv[2] = __uint_as_float(e.y << 16); xv[3] = __uint_as_float(e.y & 0xffff0000u);
    } else {
        uint2 a = *(const uint2*)xr;
        xv[0] = __uint_as_float(a.x << 16); xv[1] = __uint_as_float(a.x & 0xffff0000u);
        xv[2] = __uint_as_float(a.y << 16); xv[3] = __uint_as_float(a.y & 0xffff0000u);
        if (mode == 1 || mode == 3 || mode == 4) {
            float dv[4];
            if (mode == 1) {
                uint2 d = *(const uint2*)(delta + (size_t)r * kHidden + k);
                dv[0] = __uint_as_float(d.x << 16); dv[1] = __uint_as_float(d.x & 0xffff0000u);
                dv[2] = __uint_as_float(d.y << 16); dv[3] = __uint_as_float(d.y & 0xffff0000u);
            } else {
                // GEMM k-block chains summed in k-block order, rounded once to bf16
                float4 c = d[0];
#pragma unroll
                for (int kb = 1; kb < 16; ++kb)
                    if (kb < kblocks) { c.x = c.x + d[kb].x; c.y = c.y + d[kb].y; c.z = c.z + d[kb].z; c.w = c.w + d[kb].w; }
                dv[0] = rbf(c.x); dv[1] = rbf(c.y); dv[2] = rbf(c.z); dv[3] = rbf(c.w);
                if (mode == 4) { xv[0] = 0.f; xv[1] = 0.f; xv[2] = 0.f; xv[3] = 0.f; }
            }
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { o[i] = f2bf(xv[i] + dv[i]); xv[i] = bf2f(o[i]); }
            uint2 st;
            st.x = o[0] | ((uint32_t)o[1] << 16);
            st.y = o[2] | ((uint32_t)o[3] << 16);
            *(uint2*)xr = st;
        }
    }
    if (!h) return;
    float ss = quad_ss(xv[0], xv[1], xv[2], xv[3]);
    ss = block_sum256(ss, red);
    const float rs = hidden_rsqrt(ss);
    float wf[4] = {__uint_as_float(wv.x << 16), __uint_as_float(wv.x & 0xffff0000u),
                   __uint_as_float(wv.y << 16), __uint_as_float(wv.y & 0xffff0000u)};
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2bf(norm_elem(xv[i], rs, wf[i]));
    uint2 st;
    st.x = o[0] | ((uint32_t)o[1] << 16);
    st.y = o[2] | ((uint32_t)o[3] << 16);
    *(uint2*)(h + (TILED ? tiled_offset(r, k, kHidden) : (size_t)r * kHidden + k)) = st;
}

// MTP fc input (speccheck/mtp.py:64-69): [rmsnorm_zc(E[y], w_e) | rmsnorm_zc(h, w_h)].
__global__ void __launch_bounds__(256) mtp_concat_kernel(const int* tok, const uint16_t* E,
                                                         const uint16_t* hin, int ldh,
                                                         const uint16_t* we, const uint16_t* wh,
                                                         uint16_t* out) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const int k = threadIdx.x * 4;
#pragma unroll 1
    for (int part = 0; part < 2; ++part) {
        uint2 a = part == 0 ? *(const uint2*)(E + tiled_offset(tok[r], k, kHidden))
                            : *(const uint2*)(hin + (size_t)r * ldh + k);
        float xv[4] = {__uint_as_float(a.x << 16), __uint_as_float(a.x & 0xffff0000u),
                       __uint_as_float(a.y << 16), __uint_as_float(a.y & 0xffff0000u)};
        float ss = quad_ss(xv[0], xv[1], xv[2], xv[3]);
        ss = block_sum256(ss, red);
        const float rs = hidden_rsqrt(ss);
        const uint16_t* w = part == 0 ? we : wh;
        uint2 wv = *(const uint2*)(w + k);
        float wf[4] = {__uint_as_float(wv.x << 16), __uint_as_float(wv.x & 0xffff0000u),
                       __uint_as_float(wv.y << 16), __uint_as_float(wv.y & 0xffff0000u)};
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f2bf(norm_elem(xv[i], rs, wf[i]));
        uint2 st;
        st.x = o[0] | ((uint32_t)o[1] << 16);
        st.y = o[2] | ((uint32_t)o[3] << 16);
        *(uint2*)(out + (size_t)r * 2 * kHidden + part * kHidden + k) = st;
    }
}

hipError_t launch_addnorm(int mode, const int* tok, const uint16_t* E, uint16_t* x,
                          const uint16_t* delta, const float* kpart, int kblocks,
                          const uint16_t* w, uint16_t* h, int rows, hipStream_t st, int h_tiled) {
    if (rows <= 0) return hipErrorInvalidValue;
    if (h_tiled) {
        if (!h) return hipErrorInvalidValue;
#define Q35_ADDNORM_T(M) hipLaunchKernelGGL((addnorm_kernel<M, true>), dim3(rows), dim3(256), 0, st, tok, E, x, delta, kpart, kblocks, w, h)
        switch (mode) {
            case 0: Q35_ADDNORM_T(0); break;
            case 3: Q35_ADDNORM_T(3); break;
            case 4: Q35_ADDNORM_T(4); break;
            default: return hipErrorInvalidValue;
        }
#undef Q35_ADDNORM_T
        return hipGetLastError();
    }
#define Q35_ADDNORM(M) hipLaunchKernelGGL(addnorm_kernel<M>, dim3(rows), dim3(256), 0, st, tok, E, x, delta, kpart, kblocks, w, h)
    switch (mode) {
        case 0: Q35_ADDNORM(0); break;
        case 1: Q35_ADDNORM(1); break;
        case 2: Q35_ADDNORM(2); break;
        case 3: Q35_ADDNORM(3); break;
        case 4: Q35_ADDNORM(4); break;
        default: return hipErrorInvalidValue;
    }
#undef Q35_ADDNORM
    return hipGetLastError();
}

hipError_t launch_mtp_concat(const int* tok, const uint16_t* E, const uint16_t* hin, int ldh,
                             const uint16_t* we, const uint16_t* wh, uint16_t* out, int rows,
                             hipStream_t st) {
    if (rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mtp_concat_kernel, dim3(rows), dim3(256), 0, st, tok, E, hin, ldh, we, wh, out);
    return hipGetLastError();
}

}  // namespace q35
