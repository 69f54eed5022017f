// bf16 GEMM family for every projection, the MLP and the tied lm_head (gfx950, wave64).
//
// Y[m][n] = sum_k A[m][k] * W[n][k] with W pre-tiled (q35_common.h tiled_offset), f32
// accumulate, one bf16 rounding -- the projection policy of speccheck/specimpl.py:247-250,
// 327-333, 400-407, 475 (torch bf16 matmul). Replaces the reference's GEMV launchers
// engine/kernels_proj.cpp:128-260, engine/kernels_mlp.cpp:192-347 and
// engine/kernels_lmhead.cpp:28-191.
//
// Canonical reduction (shared by every kernel in this file, for any M): for each 256-wide
// k-block kb, one chain of 8 v_mfma_f32_16x16x32_bf16 starting from zero gives c_kb; the
// output is ((c_0 + c_1) + c_2) + ... in k-block order. Each output element therefore
// depends only on its own row of A, never on M or on the other rows, so batched lanes, the
// MTP verify rows and a batch-1 decode produce identical bits for the same row.
//
// A operand "producers" fuse the elementwise work of the consumer's input:
//   kAPlain     bf16 rows
//   kASiluMul   act = bf16(bf16(silu(g)) * u)          (specimpl.py:404-407)
//   kAGatedNorm y = bf16(w * (o * rsqrt(mean_head(o^2)+eps)) * silu(z)), per 128-wide
//               head, o f32, z bf16                    (specimpl.py:142-147, 304-305)
// Epilogues: kEStore (bf16 rows) and kEArgmax (bf16-rounded logits, per-tile max with
// the lowest index, optional f32 copy of the logits).
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

template <int AM>
__device__ __forceinline__ q35_bf16x8 load_a_frag(const GemmArgs& a, int m, int k0,
                                                  const float* rs) {
    if (AM == kAPlain) {
        const uint16_t* p = (const uint16_t*)a.X + (size_t)m * a.ldx + k0;
        return *(const q35_bf16x8*)p;
    } else if (AM == kASiluMul) {
        const uint16_t* pg = (const uint16_t*)a.X + (size_t)m * a.ldx + k0;
        const uint16_t* pu = (const uint16_t*)a.X2 + (size_t)m * a.ldx2 + k0;
        q35_u32x4 g = *(const q35_u32x4*)pg, u = *(const q35_u32x4*)pu;
        q35_u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float g0 = __uint_as_float(g[i] << 16), g1 = __uint_as_float(g[i] & 0xffff0000u);
            float u0 = __uint_as_float(u[i] << 16), u1 = __uint_as_float(u[i] & 0xffff0000u);
            uint32_t lo = f2bf(rbf(silu_f(g0)) * u0), hi = f2bf(rbf(silu_f(g1)) * u1);
            r[i] = lo | (hi << 16);
        }
        return *(q35_bf16x8*)&r;
    } else {  // kAGatedNorm: rs[0] = rsqrt for this lane's head, handled by caller
        const float* po = (const float*)a.X + (size_t)m * a.ldx + k0;
        const uint16_t* pz = (const uint16_t*)a.X2 + (size_t)m * a.ldx2 + k0;
        const uint16_t* pw = a.aux_w + (k0 & 127);
        q35_u32x4 zz = *(const q35_u32x4*)pz, ww = *(const q35_u32x4*)pw;
        float4 o0 = *(const float4*)po, o1 = *(const float4*)(po + 4);
        float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
        q35_u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t out2[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float z = h ? __uint_as_float(zz[i] & 0xffff0000u) : __uint_as_float(zz[i] << 16);
                float w = h ? __uint_as_float(ww[i] & 0xffff0000u) : __uint_as_float(ww[i] << 16);
                float n = __fmul_rn(ov[2 * i + h], rs[0]);
                out2[h] = f2bf(__fmul_rn(__fmul_rn(w, n), silu_f(z)));
            }
            r[i] = out2[0] | (out2[1] << 16);
        }
        return *(q35_bf16x8*)&r;
    }
}

// Small-M kernel: one block = one 16-column tile x one 16-row tile; wave w owns k-block w.
template <int AM, int EM>
__global__ void __launch_bounds__(1024) gemm_small_m(GemmArgs a) {
    const int nt = blockIdx.x;
    const int mt = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int kb = threadIdx.x >> 6;
    const int KB = a.K >> 8;
    const int m = mt * 16 + (lane & 15);
    const int g = lane >> 4;
    const bool mvalid = m < a.M;

    // W fragments: 8 contiguous 1 KiB wave loads.
    const q35_bf16x8* wp = (const q35_bf16x8*)(a.W + ((size_t)nt * KB + kb) * 4096) + lane;
    q35_bf16x8 wf[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) wf[s] = __builtin_nontemporal_load(wp + s * 64);

    float rs = 0.f;
    const int kbase = kb * 256 + g * 64;
    if (AM == kAGatedNorm && mvalid) {
        const float* po = (const float*)a.X + (size_t)m * a.ldx + kbase;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 64; i += 4) {
            float4 v = *(const float4*)(po + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss += __shfl_xor(ss, 16, 64);     // the other half of the 128-wide head
        rs = rsqrtf(ss * (1.0f / 128.0f) + kEps);
    }
    q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        q35_bf16x8 af;
        if (mvalid) af = load_a_frag<AM>(a, m, kbase + s * 8, &rs);
        else af = (q35_bf16x8){};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc, 0, 0, 0);
    }

    __shared__ q35_f32x4 part[16][64];
    part[kb][lane] = acc;
    __syncthreads();
    if (kb != 0) return;
    q35_f32x4 sum = part[0][lane];
    for (int w = 1; w < KB; ++w) {
        q35_f32x4 p = part[w][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] = sum[r] + p[r];
    }
    // lane holds D[row = 4*(lane/16) + r][col = lane%16]
    const int col = nt * 16 + (lane & 15);
    if (EM == kEStore) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = mt * 16 + 4 * g + r;
            if (row < a.M) a.Y[(size_t)row * a.ldy + col] = f2bf(sum[r]);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = mt * 16 + 4 * g + r;
            float v = rbf(sum[r]);
            if (row < a.M && a.logits) a.logits[(size_t)row * a.ldl + col] = v;
            int idx = col;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                float v2 = __shfl_xor(v, o, 64);
                int i2 = __shfl_xor(idx, o, 64);
                if (v2 > v || (v2 == v && i2 < idx)) { v = v2; idx = i2; }
            }
            if ((lane & 15) == 0 && row < a.M) {
                a.part_val[(size_t)row * a.ldp + nt] = v;
                a.part_idx[(size_t)row * a.ldp + nt] = idx;
            }
        }
    }
}

// Final argmax over the per-tile partials of each row: lowest id among the maxima.
__global__ void __launch_bounds__(256) argmax_rows(const float* pv, const int* pi, int ldp, int n,
                                                   int* out_tok, float* out_val) {
    const int row = blockIdx.x;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = pv[(size_t)row * ldp + i];
        int id = pi[(size_t)row * ldp + i];
        if (v > best || (v == best && id < bi)) { best = v; bi = id; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = __shfl_xor(best, o, 64);
        int i2 = __shfl_xor(bi, o, 64);
        if (v2 > best || (v2 == best && i2 < bi)) { best = v2; bi = i2; }
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
        for (int w = 1; w < 4; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) { best = sv[w]; bi = si[w]; }
        out_tok[row] = bi;
        if (out_val) out_val[row] = best;
    }
}

hipError_t launch_gemm(const GemmArgs& a, int amode, int emode, hipStream_t st) {
    if (a.K % 256 || a.N % 16 || a.K > 4096 || a.M <= 0) return hipErrorInvalidValue;
    dim3 grid(a.N / 16, (a.M + 15) / 16);
    dim3 block(64 * (a.K / 256));
#define Q35_L(AMV, EMV) hipLaunchKernelGGL((gemm_small_m<AMV, EMV>), grid, block, 0, st, a)
    if (emode == kEStore) {
        if (amode == kAPlain) Q35_L(kAPlain, kEStore);
        else if (amode == kASiluMul) Q35_L(kASiluMul, kEStore);
        else if (amode == kAGatedNorm) Q35_L(kAGatedNorm, kEStore);
        else return hipErrorInvalidValue;
    } else if (emode == kEArgmax && amode == kAPlain) {
        Q35_L(kAPlain, kEArgmax);
    } else {
        return hipErrorInvalidValue;
    }
#undef Q35_L
    return hipGetLastError();
}

hipError_t launch_argmax(const float* pv, const int* pi, int ldp, int n, int rows, int* tok,
                         float* val, hipStream_t st) {
    hipLaunchKernelGGL(argmax_rows, dim3(rows), dim3(256), 0, st, pv, pi, ldp, n, tok, val);
    return hipGetLastError();
}

}  // namespace q35
