// Gated GQA decode attention over a bf16 KV cache, split over 256-slot chunks.
//
// Math (speccheck/specimpl.py:320-397): de-interleave [q | gate] per head; zero-centred
// RMSNorm on q and k per head; rope on dims 0..63 (pairs i, i+32, theta 1e7) in f32;
// append k (post-rope) and v at the row's cache slot; scores q.K / 16 in f32; softmax in
// f32; weights rounded to bf16; P.V with f32 accumulation rounded to bf16; times
// bf16(sigmoid(gate)). GQA: query head i reads kv head i / 4.
// Replaces engine/kernels_attn.cpp:415-1108 (prep, core, combine) of the reference.
//
// Four launches per layer (batched lanes with short enough contexts: prep + one fused
// kernel, attn_fused):
//   attn_prep   (row, head)         q norm+rope -> f32 scratch; k norm+rope, v -> cache
//   attn_scores (row, kv head, chunk) scores on MFMA -> scratch, per-chunk (max, sum e^(s-max))
//   attn_pv     (row, kv head, 128-slot part) global (max, sum) from the chunk stats,
//               p = bf16(e/l), partial P.V per part on MFMA (V cache in 8-slot groups)
//   attn_combine (row, q head)      sum of the parts in order, bf16, times bf16(sigmoid(gate))
// plus attn_rows (MTP verify: a lane's rows in one block) and attn_prompt (prompt waves).
// The k cache holds bf16(k post-rope); the reference's torch path keeps it in f32, so
// k's rotated dims carry one extra bf16 rounding here (the cache layout is bf16 by design).
#include <algorithm>
#include <type_traits>

#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

constexpr int kChunk = 256;
// attn_rows<T, W>: the top parts (128 slots) whose scores fit the block's dynamic LDS beside
// the slice stats keep them there -- W = 4: two blocks per CU (80 KiB each, less the static q
// staging and ml), at most 8 parts; W = 8: one block per CU, at most 24 parts
constexpr int kRowsLdsDyn4 = 80 * 1024 - 16480, kRowsLdsDyn8 = 160 * 1024 - 16480;
__host__ __device__ constexpr int rows_lds_parts(int T, int max_chunks, int W) {
    return max(0, min(W == 8 ? 24 : 8, ((W == 8 ? kRowsLdsDyn8 : kRowsLdsDyn4) - T * 4 * 8 * max_chunks * 4) /
                                           (T * 4 * 128 * 4)));
}
__host__ __device__ constexpr size_t rows_lds_bytes(int T, int max_chunks, int W) {
    return (size_t)T * 4 * (8 * max_chunks + 128 * rows_lds_parts(T, max_chunks, W)) * 4;
}
// attn_fused<*, 2>: dynamic LDS of its two items, the CU's 160 KiB less both halves' static
// arrays (ubuf, ml, nparts)
constexpr int kFused2MaxLds = 160 * 1024 - 16464;

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
        const size_t base = lane * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256;
        a.kc[base + kv_tiled_offset(slot, d)] = f2bf(out);
        a.vc[base + kv_v8_offset(slot, d)] = pr[kAttnVOff + j * 256 + d];
    }
}

// Scores on MFMA: a wave takes 16 cache slots per v_mfma_f32_16x16x32_bf16 chain with the
// K rows as the A operand (step s of lane (slot t, group g) carries dims s*32 + g*8 .. +8;
// the K cache is stored in exactly that order, q35_common.h kv_tiled_offset, so each load
// instruction reads one contiguous KiB) and B = [q_hi(4 heads) |
// q_lo(4 heads) | 0], q_hi = bf16(q), q_lo = bf16(q - q_hi), so s = C[t][h] + C[t][h+4]
// carries q to ~2^-16 relative. A chunk = 4 waves x 64 slots.
//
// The chunk score pass, the part P.V pass and the part sum are device functions shared by
// the split kernels (any batch, any context) and the fused per-lane kernel (batched lanes,
// contexts that fit LDS), so both give the same bits.

// q fragments of kv group j for row r (all 256 threads; contains a barrier).
__device__ __forceinline__ void load_q_frags(const AttnArgs& a, int r, int j, uint16_t (*qb)[256],
                                             q35_u32x4* qf) {
    const int tid = threadIdx.x & 255, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const float* q = a.q + ((size_t)r * kNq + 4 * j) * 256;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const float qv = q[h * 256 + tid];
        const uint16_t hi = f2bf(qv);
        qb[h][tid] = hi;
        qb[4 + h][tid] = f2bf(qv - bf2f(hi));
        qb[8 + h][tid] = 0;
        qb[12 + h][tid] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const q35_u32x4*)&qb[n][s * 32 + g * 8];
}

// Scores of chunk c (slots c*256 .. +256, masked beyond `slot`) -> dst[h * dst_stride + t],
// chunk stats (max, sum e^(s - max)) -> stats[h * stats_stride + 2c .. +1]. Contains barriers.
// K fragments of sub-tile st of 64-slot slice q for this lane: K tile 4q + st of the tiled
// cache, step s = one contiguous KiB (the tile index is clamped to `slot`'s tile; slots past
// `slot` are masked later).
// NT: nontemporal loads (streamed once: one row per lane); cached when the lane's several rows
// (MTP verify rows) read the same K/V from L2 in consecutive blocks.
template <bool NT = true>
__device__ __forceinline__ void load_k_sub(const AttnArgs& a, int lrow, int j, int q, int st, int slot,
                                           q35_u32x4* kf) {
    const int lane = threadIdx.x & 63;
    const int tile = max(min(q * 4 + st, slot >> 4), 0);
    const uint16_t* kp = a.kc + lrow * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256 + (size_t)tile * 4096 + lane * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s)
        kf[s] = NT ? __builtin_nontemporal_load((const q35_u32x4*)(kp + s * 512)) : *(const q35_u32x4*)(kp + s * 512);
}

template <bool NT = true>
__device__ __forceinline__ void load_k_slice(const AttnArgs& a, int lrow, int j, int q, int slot,
                                             q35_u32x4 (*kf)[8]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) load_k_sub<NT>(a, lrow, j, q, st, slot, kf[st]);
}

// Scores of the 64-slot slice q (slots q*64 .. +64, masked beyond `slot`) by one wave.
// Scores -> dst[h * dst_stride + t]; slice stats (max, sum e^(s - max)) ->
// stats[h * stats_stride + 2q .. +1]. No barriers: waves run independently.
// kf holds slice q's K fragments on entry; with REFILL each sub-tile's registers are
// refilled with slice qnext's as soon as its MFMA chain has consumed them (unconditionally:
// past the end every lane reloads row `slot`, so the wait counts stay exact and the loads
// stay in flight across iterations).
template <bool REFILL, bool NT = true>
__device__ __forceinline__ void score_slice(const AttnArgs& a, int lrow, int j, int q, int slot,
                                            const q35_u32x4* qf, q35_u32x4 (*kf)[8], int qnext,
                                            float* dst, size_t dst_stride, float* stats, size_t stats_stride) {
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    const int t0 = q * 64;
    float sv[4][4];      // [sub-tile][r] for this lane's head (lanes n < 4)
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&kf[st][s], *(const q35_bf16x8*)&qf[s], acc, 0, 0, 0);
        if (REFILL) load_k_sub<NT>(a, lrow, j, qnext, st, slot, kf[st]);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float lo = row_down4(acc[rr]);   // lanes n < 4 add the q_lo column n + 4
            const float sc = (acc[rr] + lo) * 0.0625f;
            const int t = t0 + st * 16 + 4 * g + rr;
            const bool ok = n < 4 && t <= slot;
            sv[st][rr] = ok ? sc : -INFINITY;
            if (ok) dst[n * dst_stride + t] = sc;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) m = fmaxf(m, sv[st][rr]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, xor32(m));
    float e = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) e += sv[st][rr] > -INFINITY ? expf(sv[st][rr] - m) : 0.f;
    e += __shfl_xor(e, 16, 64);
    e += xor32(e);
    if (lane < 4 && t0 <= slot) {
        float* sp = stats + lane * stats_stride + 2 * q;
        sp[0] = m;
        sp[1] = e;
    }
}

// q fragments for a one-wave block: lane L converts dims 4L .. 4L+3 of the 4 heads.
__device__ __forceinline__ void load_q_frags_wave(const AttnArgs& a, int r, int j, uint16_t (*qb)[256],
                                                  q35_u32x4* qf) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const float* q = a.q + ((size_t)r * kNq + 4 * j) * 256;
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = 4 * lane + e;
            const float qv = q[h * 256 + d];
            const uint16_t hi = f2bf(qv);
            qb[h][d] = hi;
            qb[4 + h][d] = f2bf(qv - bf2f(hi));
            qb[8 + h][d] = 0;
            qb[12 + h][d] = 0;
        }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const q35_u32x4*)&qb[n][s * 32 + g * 8];
}

// One wave per (row, kv head, 64-slot slice): many small blocks, so a single row's scores
// spread over the CUs.
__global__ void __launch_bounds__(64) attn_scores(AttnArgs a) {
    __shared__ uint16_t qb[16][256];
    const int r = blockIdx.x, j = blockIdx.y, q = blockIdx.z;
    const int slot = a.rm.slot[r];
    if (q * 64 > slot) return;
    q35_u32x4 qf[8], kf[4][8];
    load_k_slice(a, a.rm.lane[r], j, q, slot, kf);
    load_q_frags_wave(a, r, j, qb, qf);
    score_slice<false>(a, a.rm.lane[r], j, q, slot, qf, kf, 0, a.sc + ((size_t)r * kNq + 4 * j) * a.sc_ld, a.sc_ld,
                       a.stats + ((size_t)r * kNq + 4 * j) * a.max_chunks * 8, (size_t)a.max_chunks * 8);
}

// attn_prep's per-head arithmetic for one wave: lane holds d = lane + 64 w (w = 0..3); the
// sum of squares folds each 64-element quarter with a wave sum and then (q0 + q1) + (q2 + q3),
// block_sum256a's tree, so the result is bit-identical to the 256-thread kernel.
__device__ __forceinline__ void head_norm_rope_wave(const AttnArgs& a, const uint16_t* src,
                                                    const uint16_t* normw, int pos, float* out) {
    const int lane = threadIdx.x & 63;
    float x[4], ssq[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) x[w] = bf2f(src[lane + 64 * w]);
#pragma unroll
    for (int w = 0; w < 4; ++w) ssq[w] = wave_sum(x[w] * x[w]);
    const float rs = rsqrtf(((ssq[0] + ssq[1]) + (ssq[2] + ssq[3])) * (1.0f / 256.0f) + kEps);
#pragma unroll
    for (int w = 0; w < 4; ++w) out[w] = rbf(__fmul_rn(__fmul_rn(x[w], rs), 1.0f + bf2f(normw[lane + 64 * w])));
    // rope on dims 0..63 (pairs d, d +- 32): quarter 0 holds them, the partner is lane ^ 32
    const float partner = xor32(out[0]);
    const int i = lane & 31;
    const float ang = __fmul_rn((float)pos, a.inv_freq[i]);
    const float c = cosf(ang), sn = sinf(ang);
    const float rot = lane < 32 ? -partner : partner;
    out[0] = __fadd_rn(__fmul_rn(out[0], c), __fmul_rn(rot, sn));
}

// The split path with one row per lane (batch-1 decode): attn_prep folded into the slice
// score kernel. Every block makes its 4 q heads itself; the block whose slice holds the new
// slot also makes the new K row, appends K and V to the cache and patches its own K fragments
// for that slot (its global load may still hold the previous contents).
__global__ void __launch_bounds__(64) attn_scores_prep(AttnArgs a) {
    __shared__ uint16_t qb[16][256];
    __shared__ uint16_t knew[256];
    const int r = blockIdx.x, j = blockIdx.y, q = blockIdx.z;
    const int slot = a.rm.slot[r];
    if (q * 64 > slot) return;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int lrow = a.rm.lane[r], pos = a.rm.pos[r];
    q35_u32x4 qf[8], kf[4][8];
    load_k_slice(a, lrow, j, q, slot, kf);
    const uint16_t* pr = a.proj + (size_t)r * kAttnInRows;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float o[4];
        head_norm_rope_wave(a, pr + (4 * j + i) * 512, a.q_norm, pos, o);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int d = lane + 64 * w;
            const uint16_t hi = f2bf(o[w]);
            qb[i][d] = hi;
            qb[4 + i][d] = f2bf(o[w] - bf2f(hi));
            qb[8 + i][d] = 0;
            qb[12 + i][d] = 0;
        }
    }
    const bool own = q == (slot >> 6);
    if (own) {
        float o[4];
        head_norm_rope_wave(a, pr + kAttnKOff + j * 256, a.k_norm, pos, o);
        const size_t base = lrow * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int d = lane + 64 * w;
            const uint16_t kb = f2bf(o[w]);
            knew[d] = kb;
            a.kc[base + kv_tiled_offset(slot, d)] = kb;
            a.vc[base + kv_v8_offset(slot, d)] = pr[kAttnVOff + j * 256 + d];
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const q35_u32x4*)&qb[n][s * 32 + g * 8];
    if (own && n == (slot & 15)) {
        const int st = (slot >> 4) - q * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (t == st) {
#pragma unroll
                for (int s = 0; s < 8; ++s) kf[t][s] = *(const q35_u32x4*)&knew[s * 32 + g * 8];
            }
    }
    score_slice<false>(a, lrow, j, q, slot, qf, kf, 0, a.sc + ((size_t)r * kNq + 4 * j) * a.sc_ld, a.sc_ld,
                       a.stats + ((size_t)r * kNq + 4 * j) * a.max_chunks * 8, (size_t)a.max_chunks * 8);
}

// P.V over one 128-slot part on MFMA (v_mfma_f32_16x16x32_bf16, k = slots): D = P V with
// A = P (16 query columns x 32 slots: the normalised weights rounded to bf16, from LDS) and
// B = V (32 slots x 16 dims: one 16-byte load of the 8-slot V layout per lane), one chain of
// the part's four 32-slot steps from zero per 16-dim tile; the parts are summed in order.
// Lane (n, g) of D holds query column 4g + r, dim n. A query column's result depends only on
// its own row of P, so one row, a lane's several rows and the split path give the same bits.
// A wave takes 4 dim tiles (64 dims): 16 V fragments per part.
constexpr int kPart = 128;
constexpr int kPlStride = kPart + 8;          // bf16 row stride of P in LDS (conflict-free reads)

// Softmax (max, sum) of the row's 4 heads from the nsl slice stats -> ml[h][0..1]: wave h
// takes head h, lane i folds slices i, i + 64, ... in order, then a fixed xor butterfly.
// Needs 4 waves.
__device__ __forceinline__ void softmax_ml(const float* stats, size_t stats_stride, int nsl, float (*ml)[2]) {
    const int lane = threadIdx.x & 63, h = (threadIdx.x >> 6) & 3;
    const float* st = stats + h * stats_stride;
    float m = -INFINITY;
    for (int i = lane; i < nsl; i += 64) m = fmaxf(m, st[2 * i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float l = 0.f;
    for (int i = lane; i < nsl; i += 64) l += st[2 * i + 1] * expf(st[2 * i] - m);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) {
        ml[h][0] = m;
        ml[h][1] = l;
    }
}

// V fragments of part pc for dim tiles dt0 .. dt0 + NTL - 1: vf[ks][i] = slots pc*128 + 32 ks +
// 8 g .. +8 of dim 16 (dt0 + i) + n. Unconditional loads with the 8-slot group clamped to slot's
// (past the end every lane re-reads that group, so the wait counts stay exact); slots past
// `slot` are zeroed by mask_vf before use.
template <bool NT = true, int NTL = 4>
__device__ __forceinline__ void load_vf(const AttnArgs& a, int lrow, int j, int pc, int slot, int dt0,
                                        q35_u32x4 (*vf)[NTL]) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const uint16_t* vb = a.vc + lrow * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int sg = min(pc * 16 + 4 * ks + g, slot >> 3);
#pragma unroll
        for (int i = 0; i < NTL; ++i) {
            const q35_u32x4* p = (const q35_u32x4*)(vb + (size_t)sg * 2048 + (16 * (dt0 + i) + n) * 8);
            vf[ks][i] = NT ? __builtin_nontemporal_load(p) : *p;
        }
    }
}

// Zero the V values of slots past `slot` in part pc's fragments (its last part only: V memory
// past the written slots is not initialised, and a zero weight times a NaN would be NaN).
template <int NTL = 4>
__device__ __forceinline__ void mask_vf(int pc, int slot, q35_u32x4 (*vf)[NTL]) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int cnt = slot + 1 - (pc * 128 + 32 * ks + 8 * g);   // valid slots of the group
        uint32_t mk[4];
#pragma unroll
        for (int w = 0; w < 4; ++w)
            mk[w] = (cnt > 2 * w ? 0xffffu : 0u) | (cnt > 2 * w + 1 ? 0xffff0000u : 0u);
#pragma unroll
        for (int i = 0; i < NTL; ++i)
            vf[ks][i] = (q35_u32x4){vf[ks][i][0] & mk[0], vf[ks][i][1] & mk[1], vf[ks][i][2] & mk[2], vf[ks][i][3] & mk[3]};
    }
}

// The part's four 32-slot steps for the wave's NTL dim tiles: out[i] = D of tile dt0 + i.
// pl: P in LDS, [16][kPlStride] bf16 (query column rows); rows >= nq are taken as zero.
template <int NTL = 4>
__device__ __forceinline__ void pv_mfma(const uint16_t* pl, int nq, q35_u32x4 (*vf)[NTL], q35_f32x4* out) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    q35_u32x4 af[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const q35_u32x4 v = *(const q35_u32x4*)(pl + n * kPlStride + 32 * ks + 8 * g);
        af[ks] = n < nq ? v : (q35_u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < NTL; ++i) {
        q35_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&af[ks], *(q35_bf16x8*)&vf[ks][i], d, 0, 0, 0);
        out[i] = d;
    }
}

// The weights of part pc for query columns c0 .. c0 + 3 (the 4 heads of one row) into P rows
// c0 .. c0 + 3: p = bf16(e^(s - m) / l), zero past `slot`; `scores` -> head 0's scores of the
// row (head stride s_stride), 256 threads, two weights each.
__device__ __forceinline__ void part_weights(const float* scores, size_t s_stride, const float (*ml)[2], int pc,
                                             int slot, uint16_t* pl, int c0) {
    const int tid = threadIdx.x & 255, t0 = pc * kPart;
    const int nn = min(kPart, slot + 1 - t0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int idx = tid + q * 256, i = idx >> 7, t = idx & 127;
        const float s = t < nn ? scores[i * s_stride + t0 + t] : 0.f;
        pl[(c0 + i) * kPlStride + t] = t < nn ? f2bf(expf(s - ml[i][0]) / ml[i][1]) : (uint16_t)0;
    }
}

// The softmax (max, sum) of a row's 4 heads from its nsl slice stats, in one wave, with
// softmax_ml's arithmetic per head (lane i folds slices i, i + 64, ... in order, then the xor
// butterfly), the heads interleaved so that their loads are in flight together. Every lane
// ends with all four (m, l).
__device__ __forceinline__ void wave_ml(const float* stats, size_t sst, int nsl, float* m, float* l) {
    const int tid = threadIdx.x & 63;
    // slices tid and tid + 64 held in registers (up to 128 slices, an 8,192-slot context),
    // the rest re-read in the second pass; unconditional clamped loads, masked values
#pragma unroll
    for (int h = 0; h < 4; ++h) m[h] = -INFINITY;
    float sm0[4][2], se0[4][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = min(tid + 64 * u, nsl - 1);
        const bool ok = tid + 64 * u < nsl;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float2 v = *(const float2*)(stats + h * sst + 2 * i);
            sm0[h][u] = ok ? v.x : -INFINITY;
            se0[h][u] = v.y;
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int h = 0; h < 4; ++h) m[h] = fmaxf(m[h], sm0[h][u]);
    for (int i = tid + 128; i < nsl; i += 64) {
#pragma unroll
        for (int h = 0; h < 4; ++h) m[h] = fmaxf(m[h], stats[h * sst + 2 * i]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int h = 0; h < 4; ++h) m[h] = fmaxf(m[h], __shfl_xor(m[h], o, 64));
#pragma unroll
    for (int h = 0; h < 4; ++h) l[h] = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
        if (tid + 64 * u < nsl) {
#pragma unroll
            for (int h = 0; h < 4; ++h) l[h] += se0[h][u] * expf(sm0[h][u] - m[h]);
        }
    for (int i = tid + 128; i < nsl; i += 64) {
        float sm[4], se[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) { sm[h] = stats[h * sst + 2 * i]; se[h] = stats[h * sst + 2 * i + 1]; }
#pragma unroll
        for (int h = 0; h < 4; ++h) l[h] += se[h] * expf(sm[h] - m[h]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int h = 0; h < 4; ++h) l[h] += __shfl_xor(l[h], o, 64);
}

// attention output element: bf16(bf16(sum of parts) * bf16(sigmoid(gate)))
__device__ __forceinline__ uint16_t gated_out(const AttnArgs& a, int r, int qh, int d, float acc) {
    const uint16_t* pr = a.proj + (size_t)r * kAttnInRows;
    const float o = rbf(acc);
    const float g = rbf(sigmoid_f(bf2f(pr[qh * 512 + 256 + d])));
    return f2bf(o * g);
}

// Split path, one block per (row, kv head, part): wave w takes dims 64w .. +64.
__global__ void __launch_bounds__(256) attn_pv(AttnArgs a) {
    __shared__ uint16_t pl[16 * kPlStride];
    __shared__ float ml[4][2];
    const int r = blockIdx.x, j = blockIdx.y, pc = blockIdx.z;
    const int slot = a.rm.slot[r];
    if (pc >= slot / kPart + 1) return;
    const int lrow = a.rm.lane[r], wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    q35_u32x4 vf[4][4];
    load_vf(a, lrow, j, pc, slot, 4 * wv, vf);
    softmax_ml(a.stats + ((size_t)r * kNq + 4 * j) * a.max_chunks * 8, (size_t)a.max_chunks * 8, slot / 64 + 1, ml);
    __syncthreads();
    part_weights(a.sc + ((size_t)r * kNq + 4 * j) * a.sc_ld, a.sc_ld, ml, pc, slot, pl, 0);
    __syncthreads();
    if (pc == slot / kPart) mask_vf(pc, slot, vf);
    q35_f32x4 out[4];
    pv_mfma(pl, 4, vf, out);
    if (lane < 16) {
        float* pp = a.part + (((size_t)r * a.max_chunks * 2 + pc) * kNq + 4 * j) * 256 + 64 * wv + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int h = 0; h < 4; ++h) pp[h * 256 + 16 * i] = out[i][h];
    }
}

// Sum of the 128-slot partials in part order, bf16, times bf16(sigmoid(gate)).
__global__ void __launch_bounds__(256) attn_combine(AttnArgs a) {
    const int r = blockIdx.x, qh = blockIdx.y, tid = threadIdx.x;
    const int nparts = a.rm.slot[r] / kPart + 1;
    const float* pp = a.part + ((size_t)r * a.max_chunks * 2 * kNq + qh) * 256 + tid;
    const uint16_t graw = a.proj[(size_t)r * kAttnInRows + qh * 512 + 256 + tid];
    float acc = 0.f;
    // 40 parts per round (a 5,120-slot context in one), all loads issued before the adds:
    // unconditional from clamped part indices, so no branch makes the compiler wait per load
    for (int c0 = 0; c0 < nparts; c0 += 40) {
        float v[40];
#pragma unroll
        for (int u = 0; u < 40; ++u) v[u] = pp[(size_t)min(c0 + u, nparts - 1) * kNq * 256];
#pragma unroll
        for (int u = 0; u < 40; ++u)
            if (c0 + u < nparts) acc += v[u];
    }
    const float o = rbf(acc);
    const float g = rbf(sigmoid_f(bf2f(graw)));
    a.out[(size_t)r * 2048 + qh * 256 + tid] = f2bf(o * g);
}

// ---------------------------------------------------------------- split path, 4-wave blocks
// The split path's kernels with more waves per block and the same arithmetic, so a row's
// K/V streams over 4x the waves (batch 1 uses a quarter of the CUs otherwise):
//   attn_scores4   (row, kv head, 64-slot slice): wave w scores 16-slot sub-tile w (8 KiB of
//                  K) and, with PREP, makes q head 4j + w (wave 0 also the new K row); wave 0
//                  then forms the slice stats from all four sub-tiles' values in score_slice's
//                  order (max, then e summed sub-tile-major)
//   attn_pv4       (row, kv head, 128-slot part, 64-dim quarter): one wave, the part's P.V
//                  for its 4 dim tiles on MFMA (pv_mfma), the weights made in the wave
template <bool PREP>
__global__ void __launch_bounds__(256) attn_scores4(AttnArgs a) {
    __shared__ uint16_t qb[16][256];
    __shared__ uint16_t knew[256];
    __shared__ float svl[4][4][64];          // [sub-tile][r][lane]
    const int r = blockIdx.x, j = blockIdx.y, q = blockIdx.z;
    const int slot = a.rm.slot[r];
    if (q * 64 > slot) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, n = lane & 15, g = lane >> 4;
    const int lrow = a.rm.lane[r];
    q35_u32x4 qf[8], kf[8];
    load_k_sub(a, lrow, j, q, wv, slot, kf);
    const bool own = PREP && q == (slot >> 6);
    if (PREP) {
        const int pos = a.rm.pos[r];
        const uint16_t* pr = a.proj + (size_t)r * kAttnInRows;
        float o[4];
        head_norm_rope_wave(a, pr + (4 * j + wv) * 512, a.q_norm, pos, o);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int d = lane + 64 * w;
            const uint16_t hi = f2bf(o[w]);
            qb[wv][d] = hi;
            qb[4 + wv][d] = f2bf(o[w] - bf2f(hi));
            qb[8 + wv][d] = 0;
            qb[12 + wv][d] = 0;
        }
        if (own && wv == 0) {
            head_norm_rope_wave(a, pr + kAttnKOff + j * 256, a.k_norm, pos, o);
            const size_t base = lrow * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int d = lane + 64 * w;
                const uint16_t kb = f2bf(o[w]);
                knew[d] = kb;
                a.kc[base + kv_tiled_offset(slot, d)] = kb;
                a.vc[base + kv_v8_offset(slot, d)] = pr[kAttnVOff + j * 256 + d];
            }
        }
    } else {
        const float* qp = a.q + ((size_t)r * kNq + 4 * j + wv) * 256;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int d = lane + 64 * w;
            const float qv = qp[d];
            const uint16_t hi = f2bf(qv);
            qb[wv][d] = hi;
            qb[4 + wv][d] = f2bf(qv - bf2f(hi));
            qb[8 + wv][d] = 0;
            qb[12 + wv][d] = 0;
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const q35_u32x4*)&qb[n][s * 32 + g * 8];
    if (own && n == (slot & 15) && wv == (slot >> 4) - q * 4) {
#pragma unroll
        for (int s = 0; s < 8; ++s) kf[s] = *(const q35_u32x4*)&knew[s * 32 + g * 8];
    }
    float* dst = a.sc + ((size_t)r * kNq + 4 * j) * a.sc_ld;
    const int t0 = q * 64;
    {
        q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&kf[s], *(const q35_bf16x8*)&qf[s], acc, 0, 0, 0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float lo = row_down4(acc[rr]);   // lanes n < 4 add the q_lo column n + 4
            const float sc = (acc[rr] + lo) * 0.0625f;
            const int t = t0 + wv * 16 + 4 * g + rr;
            const bool ok = n < 4 && t <= slot;
            svl[wv][rr][lane] = ok ? sc : -INFINITY;
            if (ok) dst[n * a.sc_ld + t] = sc;
        }
    }
    __syncthreads();
    if (wv != 0) return;
    float sv[4][4];
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sv[st][rr] = svl[st][rr][lane];
    float m = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) m = fmaxf(m, sv[st][rr]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, xor32(m));
    float e = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) e += sv[st][rr] > -INFINITY ? expf(sv[st][rr] - m) : 0.f;
    e += __shfl_xor(e, 16, 64);
    e += xor32(e);
    if (lane < 4) {
        float* sp = a.stats + ((size_t)r * kNq + 4 * j + lane) * a.max_chunks * 8 + 2 * q;
        sp[0] = m;
        sp[1] = e;
    }
}

__global__ void __launch_bounds__(64) attn_pv4(AttnArgs a) {
    __shared__ uint16_t pl[16 * kPlStride];
    const int r = blockIdx.x, j = blockIdx.y, pc = blockIdx.z >> 2, dq = blockIdx.z & 3;
    const int slot = a.rm.slot[r];
    if (pc >= slot / kPart + 1) return;
    const int tid = threadIdx.x;
    const int lrow = a.rm.lane[r];
    const int t0 = pc * kPart;
    // V fragments first (unconditional clamped loads), as load_vf does
    q35_u32x4 vf[4][4];
    load_vf(a, lrow, j, pc, slot, 4 * dq, vf);
    // this part's raw scores (independent of the softmax statistics: loaded early)
    const int n = min(kPart, slot + 1 - t0);
    const float* scores = a.sc + ((size_t)r * kNq + 4 * j) * a.sc_ld;
    float sraw[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int idx = tid + k * 64, i = idx >> 7, t = idx & 127;
        sraw[k] = scores[i * a.sc_ld + t0 + min(t, n - 1)];
    }
    float m[4], l[4];
    wave_ml(a.stats + ((size_t)r * kNq + 4 * j) * a.max_chunks * 8, (size_t)a.max_chunks * 8, slot / 64 + 1, m, l);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int idx = tid + k * 64, i = idx >> 7, t = idx & 127;
        const float mi = i == 0 ? m[0] : i == 1 ? m[1] : i == 2 ? m[2] : m[3];
        const float li = i == 0 ? l[0] : i == 1 ? l[1] : i == 2 ? l[2] : l[3];
        pl[i * kPlStride + t] = t < n ? f2bf(expf(sraw[k] - mi) / li) : (uint16_t)0;
    }
    __syncthreads();
    if (pc == slot / kPart) mask_vf(pc, slot, vf);
    q35_f32x4 out[4];
    pv_mfma(pl, 4, vf, out);
    if (tid < 16) {
        float* pp = a.part + (((size_t)r * a.max_chunks * 2 + pc) * kNq + 4 * j) * 256 + dq * 64 + tid;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int h = 0; h < 4; ++h) pp[h * 256 + 16 * i] = out[i][h];
    }
}

// Batched lanes: one block per (row, kv head) runs every chunk's scores into LDS, the
// softmax, every part's P.V and the gated sum -- the same device functions and orders as the
// split kernels, without the score / stats / partial round trips through HBM.
// NI = 2 (one row per lane): a block of 512 threads runs two (row, kv head) items, one per
// 256-thread half, with their own LDS. Two one-item blocks sharing a CU do not progress
// evenly (the older block's waves win the issue arbitration: at 256 lanes and ctx 4096 the
// first-dispatched half of the grid finished at ~260 us and the other at ~330 us, the CUs
// half idle in between); the halves of one block meet at every barrier, so both items end
// together. A half with fewer parts runs idle parts (its loads clamped, its sums not added)
// to keep the barrier count equal.
template <bool NT, int NI>
__global__ void __launch_bounds__(256 * NI) attn_fused(AttnArgs a, int lds_slots) {
    extern __shared__ float fl[];
    const int half = NI == 1 ? 0 : (int)(threadIdx.x >> 8);
    const size_t item_lds = (size_t)4 * lds_slots + (size_t)4 * 8 * a.max_chunks;
    float* scl = fl + half * item_lds;                  // [4][lds_slots]
    float* stl = scl + 4 * lds_slots;                   // [4][8 * max_chunks]
    __shared__ float ubuf_all[NI][2048];                // q staging, then the part's weights
    __shared__ float ml_all[NI][4][2];
    __shared__ int nparts_all[NI];
    uint16_t(*qb)[256] = (uint16_t(*)[256])ubuf_all[half];
    float(*ml)[2] = ml_all[half];
    // Block order: the T rows of one lane read the same K/V, so they run as consecutive
    // blocks of one XCD (blocks go round-robin to the 8 XCDs) and share its L2 stream. With
    // fewer (lane, kv head) pairs than XCDs (a prompt wave of one lane) each pair's rows are
    // cut into `nseg` contiguous segments of `seg` rows so that every XCD gets a segment:
    // virtual pair v -> XCD v % 8, blocks 8 ((v / 8) seg + i) + v % 8. With NI = 2 the
    // virtual blocks 16 (b / 8) + b % 8 and that + 8 run in block b (same XCD).
    const int T = a.T, tid = threadIdx.x & 255;
    const int npairs = (a.R / T) * kNkv;
    const int nseg = max(1, 8 / npairs), seg = (T + nseg - 1) / nseg;
    const int vb = NI == 1 ? (int)blockIdx.x : (int)(blockIdx.x >> 3) * 16 + half * 8 + (int)(blockIdx.x & 7);
    const int xcd = vb & 7, kk = vb >> 3;
    const int v = (kk / seg) * 8 + xcd;
    const int pr = v / nseg, t = (v % nseg) * seg + kk % seg;
    const bool active = v < npairs * nseg && t < T;
    if (NI == 1 && !active) return;
    const int j = pr % kNkv, r = active ? (pr / kNkv) * T + t : 0;
    const int slot = active ? a.rm.slot[r] : 0;
    const int lrow = a.rm.lane[r];
    const int nch = active ? slot / kChunk + 1 : 0, nparts = active ? slot / kPart + 1 : 0;
    const size_t sst = (size_t)a.max_chunks * 8;
    q35_u32x4 qf[8];
    {
        const int wv = tid >> 6;
        q35_u32x4 kf[4][8];
        load_k_slice<NT>(a, lrow, j, wv, slot, kf);
        load_q_frags(a, r, j, qb, qf);
        // wave wv takes slices 4c + wv; the last one refills nothing (no loads past the end
        // ahead of the V stream's first loads)
        for (int c = 0; c + 1 < nch; ++c)
            score_slice<true, NT>(a, lrow, j, 4 * c + wv, slot, qf, kf, 4 * (c + 1) + wv, scl, lds_slots, stl, sst);
        if (nch > 0) score_slice<false, NT>(a, lrow, j, 4 * (nch - 1) + wv, slot, qf, kf, 0, scl, lds_slots, stl, sst);
    }
    if (NI > 1 && tid == 0) nparts_all[half] = nparts;
    __syncthreads();
    int np = nparts;
    if (NI > 1) np = max(nparts_all[0], nparts_all[NI - 1]);
    // P.V: wave wv takes dims 64 wv .. +64 (pv_mfma); each part's V fragments are refilled
    // with the next part's right after their MFMAs and stay in flight across the LDS-only
    // barriers. The q staging holds the part's weights.
    const int wv = tid >> 6, lane = tid & 63;
    uint16_t* pl = (uint16_t*)ubuf_all[half];
    // V two parts ahead (the K registers of the score pass are free here): parts alternate
    // between vfa and vfb, each refilled with the part after next once used; a part at np
    // (np odd) is idle like a short half's parts: zero weights, its sum not added
    q35_u32x4 vfa[4][4], vfb[4][4];
    load_vf<NT>(a, lrow, j, 0, slot, 4 * wv, vfa);
    load_vf<NT>(a, lrow, j, 1, slot, 4 * wv, vfb);
    softmax_ml(stl, sst, slot / 64 + 1, ml);
    q35_f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
    auto part = [&](int pc, q35_u32x4 (&vf)[4][4]) {
        lds_barrier();          // ml is in; every wave is done with the previous part's weights
        part_weights(scl, lds_slots, ml, pc, slot, pl, 0);
        lds_barrier();
        if (pc == nparts - 1) mask_vf(pc, slot, vf);
        q35_f32x4 out[4];
        pv_mfma(pl, 4, vf, out);
        load_vf<NT>(a, lrow, j, pc + 2, slot, 4 * wv, vf);
        if (pc < nparts) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += out[i];
        }
    };
    for (int pc = 0; pc < np; pc += 2) {
        part(pc, vfa);
        part(pc + 1, vfb);
    }
    if (!active || lane >= 16) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int d = 64 * wv + 16 * i + lane;
            a.out[(size_t)r * 2048 + (4 * j + h) * 256 + d] = gated_out(a, r, 4 * j + h, d, acc[i][h]);
        }
}

// MTP verify rows at many lanes (T = 2 or 3 rows per lane at consecutive slots): one block
// per (lane, kv head) for all T rows, so the lane's K/V stream from HBM once and through the
// block once (one block per row re-read each line from L2 three times: ~45 GB/s per CU of
// L2 -> CU traffic for the same HBM rate). Every K fragment feeds the score MFMAs of all T
// rows: B tile u holds rows 2u and 2u + 1 as columns 8 (t % 2) + h (q hi) and + 4 (q lo), and
// an MFMA output column depends only on its own B column, so a row's scores and slice stats
// are the one-row kernel's bits. Each V part, loaded once into registers, feeds the P.V of
// every row at once (the rows' weights are rows of P). T rows x 4 heads x cap f32 scores do
// not fit LDS beside two blocks per CU: the last kRowsLdsParts parts' scores stay in LDS (the
// first written, the last read), the rest go to the global scratch; the block reads back only
// what it wrote, after a block barrier.
// W = 8 (engine option attn_rows 2): one block of 8 waves per CU -- the memory parallelism of
// two 4-wave blocks, and three times the LDS tail; P.V then takes 2 dim tiles per wave.
template <int T, int W = 4>
__global__ void __launch_bounds__(64 * W) attn_rows(AttnArgs a) {
    extern __shared__ float stl_all[];                  // [T][4][8 * max_chunks] slice stats, then
                                                        // the LDS tail [T][4][lpn * 128]
    __shared__ uint16_t qbuf[2][16][256];               // q staging (tiles), then the part's weights
    __shared__ float ml_all[T][4][2];
    constexpr int NU = (T + 1) / 2;                     // q tiles
    constexpr int NTL = 16 / W;                         // P.V dim tiles per wave
    constexpr int WPT = 8 / W;                          // weights per thread and row of a part
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, n = lane & 15, g = lane >> 4;
    const int pr = blockIdx.x, j = pr % kNkv, r0 = (pr / kNkv) * T;
    int slot_t[T];
#pragma unroll
    for (int t = 0; t < T; ++t) slot_t[t] = a.rm.slot[r0 + t];
    int slot = slot_t[0];
#pragma unroll
    for (int t = 1; t < T; ++t) slot = max(slot, slot_t[t]);
    const int lrow = a.rm.lane[r0];
    const size_t sst = (size_t)a.max_chunks * 8;
    float* tl = stl_all + (size_t)T * 4 * sst;
    const int lpn = rows_lds_parts(T, a.max_chunks, W), lsl = 128 * lpn;
    const int p0 = max(slot / kPart + 1 - lpn, 0);     // first part in the LDS tail
    // q fragments: tile u, column 8 (t % 2) + h = bf16(q) of row t = 2u + t % 2, head h, and
    // + 4 its low part (zero columns for a missing row), as load_q_frags makes them
    if (tid < 256) {
#pragma unroll
        for (int t = 0; t < 2 * NU; ++t)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int c = 8 * (t & 1) + h;
                if (t < T) {
                    const float qv = a.q[((size_t)(r0 + t) * kNq + 4 * j + h) * 256 + tid];
                    const uint16_t hi = f2bf(qv);
                    qbuf[t >> 1][c][tid] = hi;
                    qbuf[t >> 1][c + 4][tid] = f2bf(qv - bf2f(hi));
                } else {
                    qbuf[t >> 1][c][tid] = 0;
                    qbuf[t >> 1][c + 4][tid] = 0;
                }
            }
    }
    __syncthreads();
    // scores: wave wv takes slices W c + wv (score_slice's arithmetic, one MFMA chain per tile)
    {
        // q fragments in registers, K two sub-tiles ahead (kf[st % 2] holds sub-tile st; the
        // registers of sub-tile st are refilled with sub-tile st + 2, then the next slice's)
        q35_u32x4 qf[NU][8];
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int s = 0; s < 8; ++s) qf[u][s] = *(const q35_u32x4*)&qbuf[u][n][s * 32 + g * 8];
        q35_u32x4 kf[2][8];
        // the first slice's sub-tile 0 strictly before its sub-tile 1: the loop head's wait for
        // sub-tile 0 must hold on entry too, and with sub-tile 0 loaded last it would drain the
        // whole prefetch (and the previous slice's score stores) at every slice
        const int nch = (slot / 64 + W) / W;             // rounds of W slices
        load_k_sub<true>(a, lrow, j, W * (nch - 1) + wv, 0, slot, kf[0]);
        __builtin_amdgcn_sched_barrier(0);
        load_k_sub<true>(a, lrow, j, W * (nch - 1) + wv, 1, slot, kf[1]);
        // this block's rows of the score scratch as a buffer resource (byte offsets)
        const __amdgpu_buffer_rsrc_t scres = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.sc + (size_t)r0 * kNq * a.sc_ld), 0, T * kNq * a.sc_ld * 4, 0x00020000);
        const int tr = n >> 3;                           // this lane's row within a tile: 2u + tr
        int lslot[NU];                                   // that row's slot (-1: no such row)
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int ta = 2 * u, tb = 2 * u + 1 < T ? 2 * u + 1 : 2 * u;
            lslot[u] = tr == 0 ? slot_t[ta] : 2 * u + 1 < T ? slot_t[tb] : -1;
        }
        // chunks from the last down (a slice's scores and stats do not depend on the order):
        // the top parts, written first, stay in the LDS tail, and the P.V pass starts on the
        // scores written last, still in L2
        for (int c = nch - 1; c >= 0; --c) {
            const int q = W * c + wv, qnext = W * (c - 1) + wv, t0 = q * 64;
            const bool inl = q >= 2 * p0;                // this slice's scores go to the LDS tail
            float sv[NU][4][4];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                q35_f32x4 acc[NU];
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    acc[u] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < 8; ++s)
                        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&kf[st & 1][s], *(const q35_bf16x8*)&qf[u][s], acc[u], 0, 0, 0);
                }
                if (st < 2) load_k_sub<true>(a, lrow, j, q, st + 2, slot, kf[st & 1]);
                else load_k_sub<true>(a, lrow, j, qnext, st - 2, slot, kf[st & 1]);
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    // the lane's 4 consecutive slots go out as one 16-byte store (slots past the
                    // row's last are never read: the P.V pass gives them zero weight)
                    q35_f32x4 scv;
                    const int t = 2 * u + tr, tt0 = t0 + st * 16 + 4 * g;
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const float lo = row_down4(acc[u][rr]);   // lanes with n % 8 < 4 add the q_lo column
                        const float sc = (acc[u][rr] + lo) * 0.0625f;
                        const bool ok = (n & 7) < 4 && tt0 + rr <= lslot[u];
                        sv[u][st][rr] = ok ? sc : -INFINITY;
                        scv[rr] = sc;
                    }
                    // slices below the LDS tail: an unconditional buffer store (lanes without a
                    // score get an offset past the range, which the hardware drops; a store
                    // under a branch would make the compiler drain outstanding loads at the join)
                    const bool okst = (n & 7) < 4 && tt0 <= lslot[u] && !inl;
                    const int off = okst ? ((t * kNq + 4 * j + (n & 3)) * a.sc_ld + tt0) * 4 : 0x7ffffff0;
                    __builtin_amdgcn_raw_buffer_store_b128(
                        (q35_u32x4){__float_as_uint(scv[0]), __float_as_uint(scv[1]), __float_as_uint(scv[2]), __float_as_uint(scv[3])},
                        scres, off, 0, 0);
                    if (inl && (n & 7) < 4 && tt0 <= lslot[u])
                        *(q35_f32x4*)(tl + (t * 4 + (n & 3)) * lsl + (tt0 - 128 * p0)) = scv;
                }
                // sub-tiles stay in order: with the next sub-tile's MFMAs hoisted into this one
                // their K wait also drained this slice's earlier score stores
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                float m = -INFINITY;
#pragma unroll
                for (int st = 0; st < 4; ++st)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) m = fmaxf(m, sv[u][st][rr]);
                m = fmaxf(m, __shfl_xor(m, 16, 64));
                m = fmaxf(m, xor32(m));
                float e = 0.f;
#pragma unroll
                for (int st = 0; st < 4; ++st)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) e += sv[u][st][rr] > -INFINITY ? expf(sv[u][st][rr] - m) : 0.f;
                e += __shfl_xor(e, 16, 64);
                e += xor32(e);
                const int t = 2 * u + tr;
                if (g == 0 && (n & 7) < 4 && t0 <= lslot[u]) {
                    float* sp = stl_all + ((size_t)t * 4 + (n & 3)) * sst + 2 * q;
                    sp[0] = m;
                    sp[1] = e;
                }
            }
        }
    }
    __syncthreads();          // scores (global scratch) and stats (LDS) of every wave are in
#pragma unroll
    for (int t = 0; t < T; ++t) softmax_ml(stl_all + (size_t)t * 4 * sst, sst, slot_t[t] / 64 + 1, ml_all[t]);
    // P.V: P rows 4t + h hold row t's weights, so one pv_mfma per part serves every row (a
    // query column's result depends only on its own weights: the one-row kernel's bits);
    // the q staging holds the weights
    uint16_t* pl = &qbuf[0][0][0];
    // V two parts ahead (the K and q registers of the score pass are free here): parts
    // alternate between vfa and vfb, each refilled with the part after next once used
    q35_f32x4 acc[NTL];
#pragma unroll
    for (int i = 0; i < NTL; ++i) acc[i] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
    const int np = slot / kPart + 1;
    // the thread's scores (head i = idx / 128, slot idx % 128 of the part, idx = tid + 64 W q)
    // of every row, loaded two parts ahead like V and issued just before that part's V
    // (clamped to the last slot: unconditional). The vector-memory counter completes in
    // order, so waiting for a part's scores then never waits for V loads issued later.
    auto load_scores = [&](int pc, float (&sr)[T][WPT]) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int q = 0; q < WPT; ++q) {
                const int idx = tid + q * 64 * W, i = idx >> 7, tt = idx & 127;
                // both sources without a branch: a part in the LDS tail reads slot 0 of the
                // scratch (one line for every lane) and takes the LDS value
                const int ts = min(pc * kPart + tt, slot);
                const bool lp = pc >= p0 && lpn > 0;
                const float gv = a.sc[((size_t)(r0 + t) * kNq + 4 * j + i) * a.sc_ld + (lp ? 0 : ts)];
                const float lv = *(lp ? tl + (t * 4 + i) * lsl + max(ts - 128 * p0, 0) : stl_all);
                sr[t][q] = lp ? lv : gv;
            }
    };
    q35_u32x4 vfa[4][NTL], vfb[4][NTL];
    float sra[T][WPT], srb[T][WPT];
    // in this order (the loop's waits must hold on entry as well: with a part's scores issued
    // after its V, the first wait of every part would drain the whole V prefetch)
    load_scores(0, sra);
    __builtin_amdgcn_sched_barrier(0);
    load_vf<true, NTL>(a, lrow, j, 0, slot, NTL * wv, vfa);
    __builtin_amdgcn_sched_barrier(0);
    load_scores(1, srb);
    __builtin_amdgcn_sched_barrier(0);
    load_vf<true, NTL>(a, lrow, j, 1, slot, NTL * wv, vfb);
    __builtin_amdgcn_sched_barrier(0);
    const int tg = lane >> 4;
    const int myslot = tg == 0 ? slot_t[0] : tg == 1 ? slot_t[T > 1 ? 1 : 0] : slot_t[T > 2 ? 2 : 0];
    // one part (a part at np, when np is odd, is idle: zero weights, its sum not added)
    auto part = [&](int pc, q35_u32x4 (&vf)[4][NTL], float (&sr)[T][WPT]) {
        lds_barrier();          // ml is in; every wave is done with the previous part's weights
        // part_weights' arithmetic, from the scores in registers
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int nn = min(kPart, slot_t[t] + 1 - pc * kPart);
#pragma unroll
            for (int q = 0; q < WPT; ++q) {
                const int idx = tid + q * 64 * W, i = idx >> 7, tt = idx & 127;
                pl[(4 * t + i) * kPlStride + tt] = tt < nn ? f2bf(expf(sr[t][q] - ml_all[t][i][0]) / ml_all[t][i][1]) : (uint16_t)0;
            }
        }
        lds_barrier();
        if (pc == np - 1) mask_vf<NTL>(pc, slot, vf);
        q35_f32x4 out[NTL];
        pv_mfma<NTL>(pl, 4 * T, vf, out);
        load_scores(pc + 2, sr);
        load_vf<true, NTL>(a, lrow, j, pc + 2, slot, NTL * wv, vf);
        // lane (n, g) holds row g's heads: add this part where it is one of that row's parts
        if (tg < T && pc < myslot / kPart + 1) {
#pragma unroll
            for (int i = 0; i < NTL; ++i) acc[i] += out[i];
        }
    };
    for (int pc = 0; pc < np; pc += 2) {
        part(pc, vfa, sra);
        part(pc + 1, vfb, srb);
    }
    if (tg < T) {
#pragma unroll
        for (int i = 0; i < NTL; ++i)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int d = 16 * (NTL * wv + i) + (lane & 15);
                a.out[(size_t)(r0 + tg) * 2048 + (4 * j + h) * 256 + d] = gated_out(a, r0 + tg, 4 * j + h, d, acc[i][h]);
            }
    }
}

// ---------------------------------------------------------------- prompt waves (flash form)
// A prompt wave of one lane (T >= 64 rows at consecutive slots): all of its rows read the
// same K/V, so a block takes 16 rows x the 4 q heads of one kv head (64 query columns) and
// streams the lane's K/V once for all of them, with both products on MFMA:
//   S^T = K Q^T   A = the K cache's fragments (16 slots x 32 dims per step), B = q as bf16 hi
//                 (8 steps) plus its lo part on the rotated dims 0..63 (2 steps): the
//                 decode path's split of the f32 post-rope q; wave w owns columns
//                 (row 4w + n/4, head n%4) and streams every K tile itself
//   online softmax per column over 64-slot tiles (running max and sum in f32, e^(s - m)
//                 rounded to bf16 as the P.V operand)
//   O = P V       A = P straight from the S^T accumulators (lane (column, g) holds slots
//                 4g + r of each 16-slot sub-tile: the MFMA's k index is taken in that order),
//                 B = V from LDS, staged by all 4 waves in the cache's 8-slot layout, where a
//                 lane's 4 slots of one dim are one 8-byte read
// The softmax normalisation comes last (O / l), so the bf16 rounding of the weights happens
// before it rather than after as on the decode path (speccheck/specimpl.py:385-392 rounds
// the normalised weights): same math, different rounding point -- prompt logits stay within
// the engine-vs-oracle tolerance, not bit-equal to the one-row kernels.
constexpr int kPrRows = 16;
typedef short q35_s16x4 __attribute__((ext_vector_type(4)));

// V tile in LDS: the cache's 8-slot layout (kv_v8_offset) as it stands, 8 groups x 256 dims x
// 8 slots (32 KiB); a lane's 4 slots of one dim are one 8-byte read, every read address one
// lane base plus an immediate offset
constexpr int kPrVBuf = 64 * 256 * 2;                       // bytes per V tile


constexpr int kPrLds = 2 * 64 * 256 * 2 + 2 * kPrVBuf;   // K and V tiles, double-buffered: 128 KiB

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 q35_bf16x2;
// two f32 -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
    const q35_bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__global__ void __launch_bounds__(256) attn_prompt(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t pr_lds[];
    uint16_t(*kt)[64 * 256] = (uint16_t(*)[64 * 256])pr_lds;
    uint16_t* vt = pr_lds + 2 * 64 * 256;                          // [2][8 groups][256 dims][8 slots]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int T = a.T, ngrp = (T + kPrRows - 1) / kPrRows;
    // XCDs 0-3 take kv head 0 and 4-7 kv head 1: each XCD's L2 holds one head's K/V stream
    const int xcd = blockIdx.x & 7, j = xcd >> 2;
    const int grp = (blockIdx.x >> 3) * 4 + (xcd & 3);
    if (grp >= ngrp) return;
    const int r0 = grp * kPrRows;
    const int lrow = a.rm.lane[0];
    const int smax = a.rm.slot[min(r0 + kPrRows, T) - 1];
    const int qrow = min(r0 + 4 * wv + (n >> 2), T - 1);
    const int qslot = a.rm.slot[qrow];
    const int wslot = a.rm.slot[min(r0 + 4 * wv, T - 1)];     // the wave's smallest slot
    const size_t kvbase = lrow * a.kv_lane + a.kv_layer_off + (size_t)j * a.cap * 256;

    // q fragments of column n: dims s*32 + g*8 .. +8
    q35_u32x4 qhi[8], qlo[2];
    {
        const float* qp = a.q + ((size_t)qrow * kNq + 4 * j + (n & 3)) * 256 + g * 8;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float4 x0 = *(const float4*)(qp + s * 32), x1 = *(const float4*)(qp + s * 32 + 4);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            uint16_t h[8], l[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h[e] = f2bf(xs[e]);
                l[e] = f2bf(xs[e] - bf2f(h[e]));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) qhi[s][e] = (uint32_t)h[2 * e] | ((uint32_t)h[2 * e + 1] << 16);
            if (s < 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) qlo[s][e] = (uint32_t)l[2 * e] | ((uint32_t)l[2 * e + 1] << 16);
            }
        }
    }
    const int ntiles = smax / 64 + 1;
    // K and V tiles (64 slots) reach LDS by direct-to-LDS loads (global_load_lds: lane i of
    // an instruction fills the 16-byte slot i of a 1 KiB run), issued one tile ahead: K in its
    // cache layout (four 16-slot MFMA tiles, 32 KiB contiguous), V in its 8-slot layout (eight
    // 4 KiB groups, contiguous). Cached loads: the 12 blocks of a kv head on one XCD read
    // the same tiles and all but the first hit that XCD's L2. Tiles and groups past the group's
    // last slot are clamped to it (K: scores masked; V: weights zero, and the values of slots
    // past the last are zeroed where they are read, in the last tile). The wave's 8 K and 8 V
    // runs per tile are its only vector-memory loads in the loop, so "s_waitcnt vmcnt(0)"
    // at the top of a tile waits for exactly that tile's data; every LDS read below is
    // inline asm, which keeps the compiler from waiting on the prefetch in flight.
    auto issue_tiles = [&](int it, int buf) {
        const int t0 = it * 64;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int run = wv * 8 + i;                   // 1 KiB run of the 32 KiB tile
            const int tile = min(it * 4 + (run >> 3), smax >> 4);
            __builtin_amdgcn_global_load_lds(
                (const void*)(a.kc + kvbase + (size_t)tile * 4096 + (run & 7) * 512 + lane * 8),
                (__attribute__((address_space(3))) void*)&kt[buf][run * 512], 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int run = wv * 8 + i;                   // 1 KiB run: group run / 4, dims 64 (run % 4) ..
            const int grp = min(t0 / 8 + (run >> 2), smax >> 3);
            __builtin_amdgcn_global_load_lds(
                (const void*)(a.vc + kvbase + (size_t)grp * 2048 + (run & 3) * 512 + lane * 8),
                (__attribute__((address_space(3))) void*)(vt + buf * (kPrVBuf / 2) + run * 512), 16, 0, 0);
        }
    };
    issue_tiles(0, 0);

    float m_run = -INFINITY, l_run = 0.f;
    q35_f32x4 o[16];
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) o[dt] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
    // LDS byte offsets: K fragment (sub-tile st, step s) at st*8192 + s*1024 + lane*16; V:
    // lane (n, g) reads slots 32ks + 16c + 4g .. +4 of dim 16 dt + n, i.e. group 4ks + 2c + g/2,
    // slots 4 (g % 2) .. +4: the lane's base plus the immediate (4ks + 2c) * 4096 + 256 dt
    const unsigned kb0 = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&kt[0][0] + lane * 16;
    const unsigned vlane = (unsigned)(size_t)(__attribute__((address_space(3))) void*)vt +
                           (unsigned)(((g >> 1) * 2048 + n * 8 + 4 * (g & 1)) * 2);

    for (int it = 0; it < ntiles; ++it) {
        const int t0 = it * 64, buf = it & 1;
        // this tile's loads have landed (the only ones in flight), and every wave is done
        // with the other buffer (tile it - 1) before it is refilled
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (it + 1 < ntiles) issue_tiles(it + 1, buf ^ 1);
        const unsigned kbase = kb0 + (unsigned)(buf * 64 * 256 * 2);
        float sv[4][4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            q35_u32x4 kf[8];
#pragma unroll
            for (int s = 0; s < 8; ++s)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kf[s]) : "v"(kbase), "n"(st * 8192 + s * 1024) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]), "+v"(kf[7]));
            q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&kf[s], *(q35_bf16x8*)&qhi[s], acc, 0, 0, 0);
#pragma unroll
            for (int s = 0; s < 2; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&kf[s], *(q35_bf16x8*)&qlo[s], acc, 0, 0, 0);
            // scores in the log2 domain: s / 16 * log2(e)
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[st][r] = acc[r] * (0.0625f * 1.4426950408889634f);
        }
        if (t0 + 63 > wslot) {            // a tile crossing the diagonal of some column of the wave
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (t0 + st * 16 + 4 * g + r > qslot) sv[st][r] = -INFINITY;
        }
        // online softmax of column n over this tile
        float mt = -INFINITY;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sv[st][r]);
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, xor32(mt));
        const float mnew = fmaxf(m_run, mt);      // finite: slot 0 is in every column's first tile
        const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);   // exp2(-inf) = 0 on the first tile
        // P as the A operand, bf16 (k = g*8 + e <-> slot 32 ks + 16 (e / 4) + 4g + e % 4); the
        // running sum adds the rounded weights that P.V uses
        q35_u32x4 pa[2];
        float ps = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            float pv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) pv[r] = __builtin_amdgcn_exp2f(sv[st][r] - mnew);   // masked: 0
            const uint32_t w0 = pk_bf16(pv[0], pv[1]), w1 = pk_bf16(pv[2], pv[3]);
            pa[st >> 1][2 * (st & 1)] = w0;
            pa[st >> 1][2 * (st & 1) + 1] = w1;
            ps += (__uint_as_float(w0 << 16) + __uint_as_float(w0 & 0xffff0000u)) +
                  (__uint_as_float(w1 << 16) + __uint_as_float(w1 & 0xffff0000u));
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += xor32(ps);
        l_run = l_run * alpha + ps;
        m_run = mnew;
        // rescale O rows 4g + r by their columns' alpha -- only when some column's max moved
        if (__any(alpha != 1.f)) {
            float ar[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
            for (int dt = 0; dt < 16; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dt][r] *= ar[r];
        }
        // P.V: V fragments 8 d-tiles at a time (16 reads, one wait, 8 MFMAs); in the last tile
        // the values of slots past the group's last are zeroed (their memory is not initialised)
        const unsigned vb = vlane + (unsigned)(buf * kPrVBuf);
        const bool last = it == ntiles - 1;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            uint2 mk[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int cnt = last ? smax + 1 - (t0 + 32 * ks + 16 * c + 4 * g) : 4;   // valid slots of the 4
                mk[c] = (uint2){(cnt > 0 ? 0xffffu : 0u) | (cnt > 1 ? 0xffff0000u : 0u),
                                (cnt > 2 ? 0xffffu : 0u) | (cnt > 3 ? 0xffff0000u : 0u)};
            }
#pragma unroll
            for (int dh = 0; dh < 2; ++dh) {
                uint2 v0[8], v1[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v0[u])
                                 : "v"(vb), "n"((4 * ks) * 4096 + 256 * (8 * dh + u)) : "memory");
                    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v1[u])
                                 : "v"(vb), "n"((4 * ks + 2) * 4096 + 256 * (8 * dh + u)) : "memory");
                }
                asm volatile("s_waitcnt lgkmcnt(0)"
                             : "+v"(v0[0]), "+v"(v0[1]), "+v"(v0[2]), "+v"(v0[3]), "+v"(v0[4]), "+v"(v0[5]), "+v"(v0[6]), "+v"(v0[7]),
                               "+v"(v1[0]), "+v"(v1[1]), "+v"(v1[2]), "+v"(v1[3]), "+v"(v1[4]), "+v"(v1[5]), "+v"(v1[6]), "+v"(v1[7]));
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    q35_u32x4 b = {v0[u].x & mk[0].x, v0[u].y & mk[0].y, v1[u].x & mk[1].x, v1[u].y & mk[1].y};
                    o[8 * dh + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&pa[ks], *(q35_bf16x8*)&b,
                                                                           o[8 * dh + u], 0, 0, 0);
                }
            }
        }
    }
    // O / l, bf16, times bf16(sigmoid(gate)): lane (n, g) holds row 4 wv + g, head r, dims 16 dt + n
    const int row = r0 + 4 * wv + g;
    float lr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) lr[r] = __shfl(l_run, 4 * g + r, 64);
    if (row < T) {
        // every gate value loaded before the first store (a store to out could alias proj,
        // which would otherwise serialize each load behind the previous store)
        const uint16_t* pr = a.proj + (size_t)row * kAttnInRows + 256 + n;
        uint16_t gv[4][16];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) gv[r][dt] = pr[(4 * j + r) * 512 + 16 * dt];
        uint16_t* po = a.out + (size_t)row * 2048 + 4 * j * 256 + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                const float ov = rbf(o[dt][r] / lr[r]);
                const float gt = rbf(sigmoid_f(bf2f(gv[r][dt])));
                const int col = (4 * j + r) * 256 + 16 * dt + n;
                if (a.out_tiled) a.out[tiled_offset(row, col, 2048)] = f2bf(ov * gt);
                else po[r * 256 + 16 * dt] = f2bf(ov * gt);
            }
        }
    }
}

hipError_t attn_init() {
    hipError_t e = hipFuncSetAttribute((const void*)attn_fused<true, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)attn_fused<false, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)attn_fused<true, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, kFused2MaxLds);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)attn_rows<2, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, kRowsLdsDyn8);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)attn_rows<3, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, kRowsLdsDyn8);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void*)attn_prompt, hipFuncAttributeMaxDynamicSharedMemorySize, kPrLds);
}

static size_t fused_lds(const AttnArgs& a) {
    return (size_t)(4 * ((a.cap + 63) / 64 * 64) + 4 * 8 * a.max_chunks) * 4;
}
static bool fused_fits(const AttnArgs& a) { return fused_lds(a) <= 96 * 1024; }
static bool use_fused(const AttnArgs& a) {
    if (a.force == kAttnFused || a.force == kAttnFusedPair) return fused_fits(a);
    if (a.force != kAttnAuto) return false;
    return a.R >= 64 && fused_fits(a);
}
// two items per block (one row per lane) when both items' LDS fits the CU
static bool use_fused2(const AttnArgs& a) {
    if (a.force == kAttnFused) return false;
    return a.T == 1 && (a.fused_pair || a.force == kAttnFusedPair) && 2 * fused_lds(a) <= (size_t)kFused2MaxLds;
}
// one row per lane on the split path: the prep runs inside the slice score kernel
static bool prep_in_scores(const AttnArgs& a) { return !use_fused(a) && a.T == 1; }
// a lane's 2-3 verify rows in one block when the (lane, kv head) blocks fill the CUs
static int rows_w(const AttnArgs& a) { return a.rows_form == 2 ? 8 : 4; }
static bool use_rows(const AttnArgs& a) {
    // the slice stats (and the tail) fit the block's dynamic LDS
    const bool shape = (a.T == 2 || a.T == 3) && a.R % a.T == 0 &&
                       rows_lds_bytes(a.T, a.max_chunks, rows_w(a)) <= (rows_w(a) == 8 ? (size_t)kRowsLdsDyn8 : 65536);
    if (a.force == kAttnRows) return shape;
    if (a.force != kAttnAuto) return false;
    return a.rows_form && shape && a.R / a.T * kNkv >= 256;
}
static bool use_prompt(const AttnArgs& a) {
    const bool shape = a.T >= 64 && a.R == a.T;
    if (a.force == kAttnPrompt) return shape;
    if (a.force != kAttnAuto) return false;
    return a.prompt_flash && shape;
}

bool attn_prompt_form(const AttnArgs& a) { return use_prompt(a); }

// Whether the forced form can run this shape (kAttnAuto always can).
bool attn_form_ok(const AttnArgs& a) {
    switch (a.force) {
    case kAttnAuto: case kAttnSplit: case kAttnSplit4: return true;
    case kAttnFused: return use_fused(a) && a.R % a.T == 0;
    case kAttnFusedPair: return use_fused(a) && use_fused2(a);
    case kAttnRows: return use_rows(a);
    case kAttnPrompt: return use_prompt(a);
    default: return false;
    }
}

hipError_t launch_attn_prep(const AttnArgs& a, hipStream_t st) {
    if (a.R <= 0 || a.max_chunks <= 0) return hipErrorInvalidValue;
    if (prep_in_scores(a)) return hipSuccess;
    hipLaunchKernelGGL(attn_prep, dim3(a.R, kNq + kNkv), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_attn_core(const AttnArgs& a, hipStream_t st) {
    if (a.R <= 0 || a.max_chunks <= 0) return hipErrorInvalidValue;
    const int lds_slots = (a.cap + 63) / 64 * 64;
    const size_t lds = fused_lds(a);
    if (!attn_form_ok(a)) return hipErrorInvalidValue;
    if (use_prompt(a)) {
        // one lane's prompt wave: 16 rows per block, kv head by XCD half
        const int ngrp = (a.T + kPrRows - 1) / kPrRows;
        hipLaunchKernelGGL(attn_prompt, dim3((ngrp + 3) / 4 * 8), dim3(256), kPrLds, st, a);
    } else if (use_rows(a)) {
        const int W = rows_w(a);
        const size_t lds = rows_lds_bytes(a.T, a.max_chunks, W);
        if (W == 8) {
            if (a.T == 2) hipLaunchKernelGGL((attn_rows<2, 8>), dim3(a.R / 2 * kNkv), dim3(512), lds, st, a);
            else hipLaunchKernelGGL((attn_rows<3, 8>), dim3(a.R / 3 * kNkv), dim3(512), lds, st, a);
        } else if (a.T == 2) hipLaunchKernelGGL((attn_rows<2, 4>), dim3(a.R / 2 * kNkv), dim3(256), lds, st, a);
        else hipLaunchKernelGGL((attn_rows<3, 4>), dim3(a.R / 3 * kNkv), dim3(256), lds, st, a);
    } else if (use_fused(a)) {
        if (a.T < 1 || a.R % a.T) return hipErrorInvalidValue;
        const int pairs = a.R / a.T * kNkv;
        const int nseg = std::max(1, 8 / pairs), seg = (a.T + nseg - 1) / nseg;
        const dim3 grid((pairs * nseg + 7) / 8 * seg * 8);
        if (use_fused2(a))
            hipLaunchKernelGGL((attn_fused<true, 2>), dim3((grid.x + 15) / 16 * 8), dim3(512), 2 * lds, st, a, lds_slots);
        else if (a.T == 1)
            hipLaunchKernelGGL((attn_fused<true, 1>), grid, dim3(256), lds, st, a, lds_slots);
        else
            hipLaunchKernelGGL((attn_fused<false, 1>), grid, dim3(256), lds, st, a, lds_slots);
    } else {
        if (a.force == kAttnSplit4 || (a.force != kAttnSplit && a.split4)) {
            if (prep_in_scores(a))
                hipLaunchKernelGGL(attn_scores4<true>, dim3(a.R, kNkv, a.max_chunks * 4), dim3(256), 0, st, a);
            else
                hipLaunchKernelGGL(attn_scores4<false>, dim3(a.R, kNkv, a.max_chunks * 4), dim3(256), 0, st, a);
            hipLaunchKernelGGL(attn_pv4, dim3(a.R, kNkv, a.max_chunks * 8), dim3(64), 0, st, a);
        } else {
            if (prep_in_scores(a))
                hipLaunchKernelGGL(attn_scores_prep, dim3(a.R, kNkv, a.max_chunks * 4), dim3(64), 0, st, a);
            else
                hipLaunchKernelGGL(attn_scores, dim3(a.R, kNkv, a.max_chunks * 4), dim3(64), 0, st, a);
            hipLaunchKernelGGL(attn_pv, dim3(a.R, kNkv, a.max_chunks * 2), dim3(256), 0, st, a);
        }
        hipLaunchKernelGGL(attn_combine, dim3(a.R, kNq), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace q35
