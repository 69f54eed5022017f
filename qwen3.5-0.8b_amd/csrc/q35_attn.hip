// Gated GQA decode attention over a bf16 KV cache, split over 256-slot chunks.
//
// Math (speccheck/specimpl.py:320-397): de-interleave [q | gate] per head; zero-centred
// RMSNorm on q and k per head; rope on dims 0..63 (pairs i, i+32, theta 1e7) in f32;
// append k (post-rope) and v at the row's cache slot; scores q.K / 16 in f32; softmax in
// f32; weights rounded to bf16; P.V with f32 accumulation rounded to bf16; times
// bf16(sigmoid(gate)). GQA: query head i reads kv head i / 4.
// Replaces engine/kernels_attn.cpp:415-1108 (prep, core, combine) of the reference.
//
// Four launches per layer:
//   attn_prep   (row, head)         q norm+rope -> f32 scratch; k norm+rope, v -> cache
//   attn_scores (row, kv head, chunk) f32 scores -> scratch, per-chunk (max, sum e^(s-max))
//   attn_pv     (row, kv head, 64-slot part) global (max, sum) from the chunk stats,
//               p = bf16(e/l), partial P.V per part
//   attn_combine (row, q head)      sum of the parts in order, bf16, times bf16(sigmoid(gate))
// The k cache holds bf16(k post-rope); the reference's torch path keeps it in f32, so
// k's rotated dims carry one extra bf16 rounding here (the cache layout is bf16 by design).
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

constexpr int kChunk = 256;

__device__ __forceinline__ float block_sum256a(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ void __launch_bounds__(256) attn_prep(AttnArgs a) {
    __shared__ float red[4];
    __shared__ float nv[256];
    const int r = blockIdx.x, hh = blockIdx.y, d = threadIdx.x;
    const int lane = a.rm.lane[r], pos = a.rm.pos[r], slot = a.rm.slot[r];
    const uint16_t* pr = a.proj + (size_t)r * kAttnInRows;
    const bool isq = hh < kNq;
    const int j = hh - kNq;
    float x = bf2f(isq ? pr[hh * 512 + d] : pr[kAttnKOff + j * 256 + d]);
    const float ss = block_sum256a(x * x, red);
    const float rs = rsqrtf(ss * (1.0f / 256.0f) + kEps);
    const float w = bf2f((isq ? a.q_norm : a.k_norm)[d]);
    const float n = rbf(__fmul_rn(__fmul_rn(x, rs), 1.0f + w));
    nv[d] = n;
    __syncthreads();
    float out = n;
    if (d < kRotDim) {
        const int i = d & 31;
        const float ang = __fmul_rn((float)pos, a.inv_freq[i]);
        const float c = cosf(ang), s = sinf(ang);
        const float rot = d < 32 ? -nv[d + 32] : nv[d - 32];
        out = __fadd_rn(__fmul_rn(n, c), __fmul_rn(rot, s));
    }
    if (isq) {
        a.q[((size_t)r * kNq + hh) * 256 + d] = out;
    } else {
        const size_t off = lane * a.kv_lane + a.kv_layer_off + ((size_t)j * a.cap + slot) * 256 + d;
        a.kc[off] = f2bf(out);
        a.vc[off] = pr[kAttnVOff + j * 256 + d];
    }
}

// Thread = one cache slot of the chunk; 4 query heads of the kv group.
__global__ void __launch_bounds__(256) attn_scores(AttnArgs a) {
    __shared__ float4 qv[256];          // qv[d] = (q0[d], q1[d], q2[d], q3[d])
    __shared__ float red[4][4];
    const int r = blockIdx.x, j = blockIdx.y, c = blockIdx.z, tid = threadIdx.x;
    const int slot = a.rm.slot[r];
    if (c * kChunk > slot) return;
    const int lane = a.rm.lane[r];
    {
        const float* q = a.q + ((size_t)r * kNq + 4 * j) * 256;
        qv[tid] = make_float4(q[tid], q[256 + tid], q[512 + tid], q[768 + tid]);
    }
    __syncthreads();
    const int t = c * kChunk + tid;
    const bool valid = t <= slot;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (valid) {
        const uint16_t* kr = a.kc + lane * a.kv_lane + a.kv_layer_off + ((size_t)j * a.cap + t) * 256;
#pragma unroll 4
        for (int dd = 0; dd < 256; dd += 8) {
            q35_u32x4 kk = *(const q35_u32x4*)(kr + dd);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float kf = (e & 1) ? __uint_as_float(kk[e >> 1] & 0xffff0000u) : __uint_as_float(kk[e >> 1] << 16);
                float4 q = qv[dd + e];
                s0 = fmaf(q.x, kf, s0); s1 = fmaf(q.y, kf, s1);
                s2 = fmaf(q.z, kf, s2); s3 = fmaf(q.w, kf, s3);
            }
        }
    }
    float sv[4] = {s0 * 0.0625f, s1 * 0.0625f, s2 * 0.0625f, s3 * 0.0625f};
    float mx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (valid) a.sc[((size_t)r * kNq + 4 * j + i) * a.sc_ld + t] = sv[i];
        mx[i] = wave_max(valid ? sv[i] : -INFINITY);
        if ((tid & 63) == 0) red[i][tid >> 6] = mx[i];
    }
    __syncthreads();
    float m[4], e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = fmaxf(fmaxf(red[i][0], red[i][1]), fmaxf(red[i][2], red[i][3]));
        e[i] = valid ? expf(sv[i] - m[i]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float se = wave_sum(e[i]);
        if ((tid & 63) == 0) red[i][tid >> 6] = se;
    }
    __syncthreads();
    if (tid < 4) {
        float l = (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);
        float* st = a.stats + (((size_t)r * kNq + 4 * j + tid) * a.max_chunks + c) * 2;
        st[0] = m[tid];
        st[1] = l;
    }
}

// P.V over one 64-slot part: thread (dg, tg) owns dims dg*8..+8 for slots tg*8..+8 of the
// part (16-byte V loads), the 8 slot groups are summed in order through LDS.
constexpr int kPart = 64;

__global__ void __launch_bounds__(256) attn_pv(AttnArgs a) {
    __shared__ float p[4][kPart];
    __shared__ float ml[4][2];
    __shared__ float red[8][4][256];
    const int r = blockIdx.x, j = blockIdx.y, pc = blockIdx.z, tid = threadIdx.x;
    const int slot = a.rm.slot[r];
    const int nparts = slot / kPart + 1;
    if (pc >= nparts) return;
    const int nch = slot / kChunk + 1;
    const int lane = a.rm.lane[r];
    if (tid < 4) {
        const float* st = a.stats + ((size_t)r * kNq + 4 * j + tid) * a.max_chunks * 2;
        float m = -INFINITY;
        for (int i = 0; i < nch; ++i) m = fmaxf(m, st[2 * i]);
        float l = 0.f;
        for (int i = 0; i < nch; ++i) l += st[2 * i + 1] * expf(st[2 * i] - m);
        ml[tid][0] = m;
        ml[tid][1] = l;
    }
    __syncthreads();
    const int t0 = pc * kPart;
    const int n = min(kPart, slot + 1 - t0);
    {
        const int i = tid >> 6, t = tid & 63;
        float pv = 0.f;
        if (t < n) {
            float s = a.sc[((size_t)r * kNq + 4 * j + i) * a.sc_ld + t0 + t];
            pv = rbf(expf(s - ml[i][0]) / ml[i][1]);
        }
        p[i][t] = pv;
    }
    __syncthreads();
    const int dg = tid & 31, tg = tid >> 5;
    const uint16_t* vr = a.vc + lane * a.kv_lane + a.kv_layer_off + ((size_t)j * a.cap + t0) * 256 + dg * 8;
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
    q35_u32x4 vv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int t = tg * 8 + u;
        if (t < n) vv[u] = *(const q35_u32x4*)(vr + (size_t)t * 256);
        else vv[u] = (q35_u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int t = tg * 8 + u;
        float pp[4] = {p[0][t], p[1][t], p[2][t], p[3][t]};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = (e & 1) ? __uint_as_float(vv[u][e >> 1] & 0xffff0000u) : __uint_as_float(vv[u][e >> 1] << 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i][e] = fmaf(pp[i], v, acc[i][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[tg][i][dg * 8 + e] = acc[i][e];
    __syncthreads();
    float* pp = a.part + (((size_t)r * a.max_chunks * 4 + pc) * kNq + 4 * j) * 256 + tid;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float sum = red[0][i][tid];
#pragma unroll
        for (int g = 1; g < 8; ++g) sum += red[g][i][tid];
        pp[i * 256] = sum;
    }
}

// Sum of the 64-slot partials in part order, bf16, times bf16(sigmoid(gate)).
__global__ void __launch_bounds__(256) attn_combine(AttnArgs a) {
    const int r = blockIdx.x, qh = blockIdx.y, tid = threadIdx.x;
    const int nparts = a.rm.slot[r] / kPart + 1;
    const float* pp = a.part + ((size_t)r * a.max_chunks * 4 * kNq + qh) * 256 + tid;
    float acc = 0.f;
    for (int c0 = 0; c0 < nparts; c0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = c0 + u < nparts ? pp[(size_t)(c0 + u) * kNq * 256] : 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c0 + u < nparts) acc += v[u];
    }
    const uint16_t* pr = a.proj + (size_t)r * kAttnInRows;
    const float o = rbf(acc);
    const float g = rbf(sigmoid_f(bf2f(pr[qh * 512 + 256 + tid])));
    a.out[(size_t)r * 2048 + qh * 256 + tid] = f2bf(o * g);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (a.R <= 0 || a.max_chunks <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_prep, dim3(a.R, kNq + kNkv), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_scores, dim3(a.R, kNkv, a.max_chunks), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_pv, dim3(a.R, kNkv, a.max_chunks * 4), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_combine, dim3(a.R, kNq), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace q35
