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
// output is ((c_0 + c_1) + c_2) + ... in k-block order. Within a chain, step s of lane
// (row or column i, group g) carries k = kb*256 + g*64 + s*8 .. +8. Each output element
// therefore depends only on its own row of A, never on M or on the other rows, so batched
// lanes, the MTP verify rows and a batch-1 decode produce identical bits for the same row.
//
// Kernels (all follow the order above):
//   gemm_small_m   one 16-row tile; wave w of a block owns k-block w (M <= 16, batch 1);
//                  with a producer the wave builds its A tile cooperatively in LDS
//   gemm_pre       K = 1024 at M > 16: 32 x 64 (or 64 x 128) blocks, every load issued up front
//                  (A by LDS-DMA)
//   gemm_lmhead3   tied lm_head at M > 16: persistent, A in registers, the weights through an
//                  LDS ring, a running argmax per column stream (gemm_lmhead: A resident in LDS)
//   gemm_large_m   4 waves x 16 columns, 64 rows per block; the A tile of each k-block is
//                  staged once in LDS in MFMA fragment order, the next k-block's loads in
//                  flight meanwhile (batched lanes);
//                  a non-plain producer runs first as its own elementwise kernel
// kEPartial (N = 1024 outputs feeding the residual add): each block computes ONE k-block
// chain and stores it to kpart[kb][M][N]; the following add+norm kernel sums the chains in
// k-block order. That keeps ~KB x more blocks in flight without cross-block atomics.
//
// A operand "producers" fuse the elementwise work of the consumer's input:
//   kAPlain     bf16 rows
//   kASiluMul   act = bf16(bf16(silu(g)) * u)          (specimpl.py:404-407)
//   kAGatedNorm y = bf16(w * (o * rsqrt(mean_head(o^2)+eps)) * silu(z)), per 128-wide
//               head, o f32, z bf16                    (specimpl.py:142-147, 304-305)
//   kANormX     h = rmsnorm_zc(x) of the residual row (specimpl.py:135-139), batch-1 only
//   kANormXP    one row: x' = bf16(x + bf16(sum of the producing GEMM's k-block chains in
//               k-block order)) -- the residual add of specimpl.py:445-448 -- then h =
//               rmsnorm_zc(x'); block 0 writes x' to xres (the next residual row)
// Epilogues: kEStore (bf16 rows), kEPartial (one f32 k-block chain), kEResidual (batch-1:
// x <- bf16(x + bf16(sum)), the residual add of specimpl.py:445-448) and kEArgmax
// (bf16-rounded logits, per-tile max with the lowest index, optional f32 logits copy).
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

// ---------------------------------------------------------------- shared producers
// 8 A elements of row m at k0 (k0 % 8 == 0); rs = rsqrt of the head holding k0 (gated norm).
template <int AM>
__device__ __forceinline__ q35_u32x4 produce_a(const GemmArgs& a, int m, int k0, float rs) {
    if (AM == kAPlain) {
        return *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + k0);
    } else if (AM == kASiluMul) {
        q35_u32x4 g = *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + k0);
        q35_u32x4 u = *(const q35_u32x4*)((const uint16_t*)a.X2 + (size_t)m * a.ldx2 + k0);
        return silu_mul8(g, u);
    } else if (AM == kANormXP) {          // one row only: produced in the direct path
        return (q35_u32x4){0u, 0u, 0u, 0u};
    } else if (AM == kANormX) {
        q35_u32x4 x = *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + k0);
        q35_u32x4 w = *(const q35_u32x4*)(a.aux_w + k0);
        q35_u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo = f2bf(norm_elem(__uint_as_float(x[i] << 16), rs, __uint_as_float(w[i] << 16)));
            uint32_t hi = f2bf(norm_elem(__uint_as_float(x[i] & 0xffff0000u), rs, __uint_as_float(w[i] & 0xffff0000u)));
            r[i] = lo | (hi << 16);
        }
        return r;
    } else {
        const float* po = (const float*)a.X + (size_t)m * a.ldx + k0;
        q35_u32x4 zz = *(const q35_u32x4*)((const uint16_t*)a.X2 + (size_t)m * a.ldx2 + k0);
        q35_u32x4 ww = *(const q35_u32x4*)(a.aux_w + (k0 & 127));
        float ov[8];
        *(float4*)&ov[0] = *(const float4*)po;
        *(float4*)&ov[4] = *(const float4*)(po + 4);
        return gated8(ov, zz, ww, rs);
    }
}

__device__ __forceinline__ q35_bf16x8 as_bf(q35_u32x4 v) { return *(q35_bf16x8*)&v; }

// (max, lowest index) over the 16 lanes of a DPP row; every lane ends with the result. The
// combine is exact and commutative, so the pairing order (quad swaps, then the half-row and
// row mirrors) gives the same winner as any other reduction order.
__device__ __forceinline__ void argmax16_step(float& v, int& idx, int ctrl) {
    float v2;
    int i2;
    if (ctrl == 0xB1) {
        v2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
        i2 = __builtin_amdgcn_update_dpp(0, idx, 0xB1, 0xf, 0xf, false);
    } else if (ctrl == 0x4E) {
        v2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
        i2 = __builtin_amdgcn_update_dpp(0, idx, 0x4E, 0xf, 0xf, false);
    } else if (ctrl == 0x141) {
        v2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
        i2 = __builtin_amdgcn_update_dpp(0, idx, 0x141, 0xf, 0xf, false);
    } else {
        v2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
        i2 = __builtin_amdgcn_update_dpp(0, idx, 0x140, 0xf, 0xf, false);
    }
    if (v2 > v || (v2 == v && i2 < idx)) { v = v2; idx = i2; }
}
__device__ __forceinline__ void argmax16(float& v, int& idx) {
    argmax16_step(v, idx, 0xB1);    // quad_perm [1,0,3,2]
    argmax16_step(v, idx, 0x4E);    // quad_perm [2,3,0,1]
    argmax16_step(v, idx, 0x141);   // row_half_mirror: quad 0 <-> quad 1, 2 <-> 3
    argmax16_step(v, idx, 0x140);   // row_mirror: half 0 <-> half 1
}

// Epilogue of one 16x16 tile: lane holds D[row0 + 4*(lane/16) + r][col0 + lane%16].
template <int EM>
__device__ __forceinline__ void epilogue(const GemmArgs& a, q35_f32x4 sum, int nt, int row0, int lane,
                                         int kchain = -1) {
    const int col = nt * 16 + (lane & 15);
    const int g = lane >> 4;
    if (EM == kEPartial) {      // sum is the chain of k-block kchain (default: blockIdx.z)
        const int kc = kchain >= 0 ? kchain : (int)blockIdx.z;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = row0 + 4 * g + r;
            if (row < a.M) a.kpart[((size_t)kc * a.M + row) * a.N + col] = sum[r];
        }
    } else if (EM == kEStore) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = row0 + 4 * g + r;
            if (row < a.M) a.Y[(size_t)row * a.ldy + col] = f2bf(sum[r]);
        }
    } else if (EM == kEResidual) {   // the same add as the add+norm kernel's partial mode
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = row0 + 4 * g + r;
            if (row < a.M) {
                uint16_t* px = a.xres + (size_t)row * kHidden + col;
                *px = f2bf(bf2f(*px) + rbf(sum[r]));
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 4 * g + r;
            float v = rbf(sum[r]);
            // 32-bit element offsets (logits < 2^31 elements): no 64-bit products to keep live
            if (row < a.M && a.logits) a.logits[(unsigned)(row * a.ldl + col)] = v;
            int idx = col;
            argmax16(v, idx);
            if ((lane & 15) == 0 && row < a.M) {
                a.part_val[(unsigned)(row * a.ldp + nt)] = v;
                a.part_idx[(unsigned)(row * a.ldp + nt)] = idx;
            }
        }
    }
}

// ---------------------------------------------------------------- small M
// kEStore / kEArgmax: grid (N/16, ceil(M/16)); block = KB waves, wave w owns k-block w.
// kEPartial: grid (N/16, ceil(M/16), KB); one wave per block, storing its k-block chain.
// TPB > 1 (one row with a norm producer, kEStore): each block takes TPB adjacent column tiles,
// so the producer's per-block work (the norm, or the fold of the residual's k-block chains --
// 57 KiB of chain reads per block, more than its weight tile) is shared by TPB tiles; every
// wave runs TPB MFMA chains on the same A fragments. Used with TPB = 2 for N >= 4096
// (batch 1: 1,171 -> 1,209 tok/s; TPB = 4, a quarter of the blocks: 1,168).
// KP: chain loads of the kANormXP fold (16, or 8 when the producing GEMM left at most 8)
// XT (TPB = 2): the grid covers the first 2 x gridDim.x column tiles and block b also takes
// tile 2 x gridDim.x + b if it exists, so a width of 514 tiles (the GDN in_proj) runs as 256
// blocks instead of a 257th one doubling up on a CU
template <int AM, int EM, int TPB = 1, int KP = 16, bool XT = false>
__global__ void __launch_bounds__(TPB > 1 ? 256 : 1024) gemm_small_m(GemmArgs a) {   // TPB > 1: K = 1024, 4 waves
    const int nt = blockIdx.x * TPB;
    const int ntx = TPB * gridDim.x + blockIdx.x;       // XT: the extra tile
    const bool hx = XT && ntx < a.N / 16;              // block-uniform
    const int mt = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int KB = a.K >> 8;
    const int kb = EM == kEPartial ? blockIdx.z : wv;
    const int m = mt * 16 + (lane & 15);
    const int g = lane >> 4;
    const bool mvalid = m < a.M;

    const q35_bf16x8* wp = (const q35_bf16x8*)(a.W + ((size_t)nt * KB + kb) * 4096) + lane;
    q35_bf16x8 wf[TPB][8], wx[8];
    auto load_w = [&] {
#pragma unroll
        for (int t = 0; t < TPB; ++t)
#pragma unroll
            for (int s = 0; s < 8; ++s) wf[t][s] = __builtin_nontemporal_load(wp + (size_t)t * KB * 512 + s * 64);
        if (hx) {
            const q35_bf16x8* wq = (const q35_bf16x8*)(a.W + ((size_t)ntx * KB + kb) * 4096) + lane;
#pragma unroll
            for (int s = 0; s < 8; ++s) wx[s] = __builtin_nontemporal_load(wq + s * 64);
        }
    };
    // batch 1 with a producer: the producer's own loads go first (the vector-memory counter
    // completes in order, so its arithmetic then overlaps the weight stream instead of
    // waiting behind it)
    const bool direct = AM != kAPlain && a.M == 1;
    if (!direct) load_w();
    // residual rows of the epilogue, loaded now so their latency overlaps the k-block work
    // (unconditional loads from clamped rows: a branch per load would make the compiler wait
    // for every outstanding load at the join)
    uint16_t xr[4] = {0, 0, 0, 0};      // raw bits: converted only in the epilogue (every wave
    if (EM == kEResidual) {              // loads them: no branch, so no wait at a join)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = min(mt * 16 + 4 * g + r, a.M - 1);
            xr[r] = a.xres[(size_t)row * kHidden + nt * 16 + (lane & 15)];
        }
    }

    const int kbase = kb * 256 + g * 64;
    q35_u32x4 af[8];
    if (AM == kAPlain) {
        // all 8 fragment loads issued before the MFMAs
#pragma unroll
        for (int s = 0; s < 8; ++s)
            af[s] = mvalid ? *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + kbase + s * 8)
                           : (q35_u32x4){0u, 0u, 0u, 0u};
    } else if (a.M == 1) {
        // Batch 1: lane c < 32 produces chunk c (k-block elements c*8 .. +8) with the same
        // produce_a arithmetic and row factors as the cooperative form below; the fragments
        // of the row-0 lanes (g, s) = chunk 8g + s are gathered with wave shuffles -- no LDS
        // round trip, no block barrier.
        const int c = lane & 31;
        const int k0 = kb * 256 + c * 8;
        q35_u32x4 mine;
        if (AM == kANormX) {
            const uint16_t* xr0 = (const uint16_t*)a.X;
            uint2 v[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) v[w] = *(const uint2*)(xr0 + 4 * (64 * w + lane));
            const q35_u32x4 xc = *(const q35_u32x4*)(xr0 + k0);
            const q35_u32x4 wc = *(const q35_u32x4*)(a.aux_w + k0);
            asm volatile("" ::: "memory");     // keep the producer's loads ahead of W
            load_w();
            __builtin_amdgcn_sched_barrier(0);   // ... and its arithmetic behind W's issue
            float wsum[4];
#pragma unroll
            for (int w = 0; w < 4; ++w)
                wsum[w] = wave_sum(quad_ss(__uint_as_float(v[w].x << 16), __uint_as_float(v[w].x & 0xffff0000u),
                                           __uint_as_float(v[w].y << 16), __uint_as_float(v[w].y & 0xffff0000u)));
            const float rs = hidden_rsqrt((wsum[0] + wsum[1]) + (wsum[2] + wsum[3]));
#pragma unroll
            for (int i = 0; i < 4; ++i) {      // produce_a<kANormX> on the preloaded chunk
                const uint32_t lo = f2bf(norm_elem(__uint_as_float(xc[i] << 16), rs, __uint_as_float(wc[i] << 16)));
                const uint32_t hi = f2bf(norm_elem(__uint_as_float(xc[i] & 0xffff0000u), rs, __uint_as_float(wc[i] & 0xffff0000u)));
                mine[i] = lo | (hi << 16);
            }
        } else if (AM == kANormXP) {
            // this GEMM has K = 1024, so wave kb owns columns 256 kb .. +255: lane L folds the
            // quad q = 64 kb + L (columns 4q .. 4q+3) -- the add+norm kernel's quad -- and the
            // four waves exchange their square sums (same reduction tree)
            const uint16_t* xr0 = (const uint16_t*)a.X;
            const int q0 = 256 * kb + 4 * lane;
            const uint2 xq = *(const uint2*)(xr0 + q0);
            float4 d[KP];
#pragma unroll
            for (int j = 0; j < KP; ++j)     // unconditional clamped loads: no wait at a join
                d[j] = *(const float4*)(a.kpart + (size_t)min(j, a.kpb - 1) * kHidden + q0);
            const q35_u32x4 wc = *(const q35_u32x4*)(a.aux_w + k0);
            asm volatile("" ::: "memory");     // keep the producer's loads ahead of W
            load_w();
            __builtin_amdgcn_sched_barrier(0);   // ... and its arithmetic behind W's issue
            float4 dsum = d[0];
#pragma unroll
            for (int j = 1; j < KP; ++j)
                if (j < a.kpb) { dsum.x = dsum.x + d[j].x; dsum.y = dsum.y + d[j].y; dsum.z = dsum.z + d[j].z; dsum.w = dsum.w + d[j].w; }
            const float xv0[4] = {__uint_as_float(xq.x << 16), __uint_as_float(xq.x & 0xffff0000u),
                                  __uint_as_float(xq.y << 16), __uint_as_float(xq.y & 0xffff0000u)};
            const float cv[4] = {dsum.x, dsum.y, dsum.z, dsum.w};
            uint32_t o[4];
            float xn[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { o[i] = f2bf(xv0[i] + rbf(cv[i])); xn[i] = bf2f((uint16_t)o[i]); }
            const uint2 pk = {o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
            if (blockIdx.x == 0) *(uint2*)(a.xres + q0) = pk;
            __shared__ float wred[16];
            const float ws = wave_sum(quad_ss(xn[0], xn[1], xn[2], xn[3]));
            if (lane == 0) wred[kb] = ws;
            __syncthreads();
            const float rs = hidden_rsqrt((wred[0] + wred[1]) + (wred[2] + wred[3]));
            // chunk c = columns 256 kb + 8c .. +7 = the quads of lanes 2c and 2c + 1
            q35_u32x4 xc;
            xc[0] = (uint32_t)__shfl((int)pk.x, 2 * c, 64);
            xc[1] = (uint32_t)__shfl((int)pk.y, 2 * c, 64);
            xc[2] = (uint32_t)__shfl((int)pk.x, 2 * c + 1, 64);
            xc[3] = (uint32_t)__shfl((int)pk.y, 2 * c + 1, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) {      // produce_a<kANormX> on x'
                const uint32_t lo = f2bf(norm_elem(__uint_as_float(xc[i] << 16), rs, __uint_as_float(wc[i] << 16)));
                const uint32_t hi = f2bf(norm_elem(__uint_as_float(xc[i] & 0xffff0000u), rs, __uint_as_float(wc[i] & 0xffff0000u)));
                mine[i] = lo | (hi << 16);
            }
        } else if (AM == kASiluMul) {         // produce_a<kASiluMul> on preloaded g, u
            const q35_u32x4 gq = *(const q35_u32x4*)((const uint16_t*)a.X + k0);
            const q35_u32x4 uq = *(const q35_u32x4*)((const uint16_t*)a.X2 + k0);
            asm volatile("" ::: "memory");     // keep the producer's loads ahead of W
            load_w();
            __builtin_amdgcn_sched_barrier(0);   // ... and its arithmetic behind W's issue
            mine = silu_mul8(gq, uq);
        } else {                               // kAGatedNorm: produce_a on preloaded o, z, w
            // lane L sums quarter L/16 (64 contiguous o values); chunk c is in head c/16,
            // whose quarters are 2(c/16) and 2(c/16)+1
            const float* po = (const float*)a.X;
            float qv[64];
#pragma unroll
            for (int i = 0; i < 16; ++i) *(float4*)&qv[4 * i] = *(const float4*)(po + kb * 256 + (lane >> 4) * 64 + 4 * i);
            float ov[8];
            *(float4*)&ov[0] = *(const float4*)(po + k0);
            *(float4*)&ov[4] = *(const float4*)(po + k0 + 4);
            const q35_u32x4 zz = *(const q35_u32x4*)((const uint16_t*)a.X2 + k0);
            const q35_u32x4 ww = *(const q35_u32x4*)(a.aux_w + (k0 & 127));
            asm volatile("" ::: "memory");     // keep the producer's loads ahead of W
            load_w();
            __builtin_amdgcn_sched_barrier(0);   // ... and its arithmetic behind W's issue
            const float q = half_head_ss_regs(qv);
            const int h2 = (c >> 4) * 32;
            const float rs = head_rsqrt(__shfl(q, h2, 64), __shfl(q, h2 + 16, 64));
            mine = gated8(ov, zz, ww, rs);
        }
        if (AM == kANormX && a.hout && blockIdx.x == 0 && lane < 32)
            *(q35_u32x4*)(a.hout + k0) = mine;
        const bool row0 = (lane & 15) == 0;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int src = 8 * g + s;
            q35_u32x4 f;
#pragma unroll
            for (int i = 0; i < 4; ++i) f[i] = (uint32_t)__shfl((int)mine[i], src, 64);
            af[s] = row0 ? f : (q35_u32x4){0u, 0u, 0u, 0u};
        }
    } else {
        // Producer modes: each wave builds its 16 x 256 A tile cooperatively -- only the M
        // valid rows, 8 elements per (lane, chunk) -- into its own LDS region in fragment
        // order, so the per-element work is spread over all 64 lanes.
        extern __shared__ q35_u32x4 dyn_lds[];
        q35_u32x4(*As)[64] = (q35_u32x4(*)[64])(dyn_lds + wv * 512);
        float* rowv = (float*)(dyn_lds + (EM == kEPartial ? 1 : KB) * 512) + wv * 64;   // [16][4]
        const int M = min(a.M - mt * 16, 16);
#pragma unroll
        for (int s = 0; s < 8; ++s) As[s][lane] = (q35_u32x4){0u, 0u, 0u, 0u};
        if (AM == kAGatedNorm) {
            for (int c = lane; c < M * 4; c += 64) {
                const int row = c >> 2, q = c & 3;
                rowv[row * 4 + q] = half_head_ss((const float*)a.X + (size_t)(mt * 16 + row) * a.ldx + kb * 256 + q * 64);
            }
        } else if (AM == kANormX) {
            // row rsqrt with the add+norm kernel's reduction tree (quad t = 64w + lane)
            for (int row = 0; row < M; ++row) {
                const uint16_t* xr = (const uint16_t*)a.X + (size_t)(mt * 16 + row) * a.ldx;
                float wsum[4];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    uint2 v = *(const uint2*)(xr + 4 * (64 * w + lane));
                    wsum[w] = wave_sum(quad_ss(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                                               __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)));
                }
                if (lane == 0) rowv[row * 4] = hidden_rsqrt((wsum[0] + wsum[1]) + (wsum[2] + wsum[3]));
            }
        }
        __syncthreads();
        for (int c = lane; c < M * 32; c += 64) {
            const int row = c >> 5, kc = c & 31;
            const int k0 = kb * 256 + kc * 8;
            float rs = 0.f;
            if (AM == kAGatedNorm) rs = head_rsqrt(rowv[row * 4 + (kc >> 4) * 2], rowv[row * 4 + (kc >> 4) * 2 + 1]);
            if (AM == kANormX) rs = rowv[row * 4];
            const q35_u32x4 v = produce_a<AM>(a, mt * 16 + row, k0, rs);
            As[kc & 7][(kc >> 3) * 16 + row] = v;
            if (AM == kANormX && a.hout && blockIdx.x == 0)
                *(q35_u32x4*)(a.hout + (size_t)(mt * 16 + row) * kHidden + k0) = v;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 8; ++s) af[s] = As[s][lane];
    }
    q35_f32x4 acc[TPB];
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        acc[t] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(af[s]), wf[t][s], acc[t], 0, 0, 0);
    }
    if (EM == kEPartial) {
        epilogue<EM>(a, acc[0], nt, mt * 16, lane);
        return;
    }
    __shared__ q35_f32x4 part[TPB + XT][16][64];
#pragma unroll
    for (int t = 0; t < TPB; ++t) part[t][wv][lane] = acc[t];
    if (hx) {
        q35_f32x4 ax = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) ax = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(af[s]), wx[s], ax, 0, 0, 0);
        part[TPB][wv][lane] = ax;
    }
    __syncthreads();
    if (wv >= TPB + (hx ? 1 : 0)) return;  // wave t sums tile t's k-block chains in order
    q35_f32x4 sum = part[wv][0][lane];
    for (int w = 1; w < KB; ++w) {
        q35_f32x4 p = part[wv][w][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] = sum[r] + p[r];
    }
    if (EM == kEResidual) {     // x <- bf16(x + bf16(sum)), as the epilogue below
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = mt * 16 + 4 * g + r;
            if (row < a.M) a.xres[(size_t)row * kHidden + nt * 16 + (lane & 15)] = f2bf(bf2f(xr[r]) + rbf(sum[r]));
        }
        return;
    }
    epilogue<EM>(a, sum, wv < TPB ? nt + wv : ntx, mt * 16, lane);
}

// Elementwise A producer for batched launches: Y[m][k] = produce_a(m, k) (bf16), so the
// GEMM that follows reads plain bf16 and each element is produced once.
template <int AM>
__global__ void __launch_bounds__(256) produce_kernel(GemmArgs a) {
    const int m = blockIdx.x;
    for (int c = threadIdx.x; c < a.K / 8; c += 256) {
        const int k0 = c * 8;
        float rs = 0.f;
        if (AM == kAGatedNorm) {
            const int hq = (k0 / 128) * 128;    // head start
            const float* po = (const float*)a.X + (size_t)m * a.ldx;
            rs = head_rsqrt(half_head_ss(po + hq), half_head_ss(po + hq + 64));
        }
        *(q35_u32x4*)(a.Y + (size_t)m * a.ldy + k0) = produce_a<AM>(a, m, k0, rs);
    }
}

// The same producer writing Y in the tiled fragment layout (K = a.K): block (16-row tile, 16
// chunks of 8 k), the row fastest across threads, so the 16 rows' pieces of one (k-block, step,
// quarter) -- one contiguous 256-byte run of the layout -- are written together (one row per
// block would leave each 16-byte piece alone in its line).
// Made row-major (16 threads per row share its reads) and transposed through LDS.
template <int AM>
__global__ void __launch_bounds__(256) produce_tiled_kernel(GemmArgs a) {
    __shared__ q35_u32x4 t[16][16];                     // [chunk][row]
    const int tid = threadIdx.x;
    {
        const int r = tid >> 4, c = tid & 15, m = min(blockIdx.x * 16 + r, a.M - 1);
        const int k0 = (blockIdx.y * 16 + c) * 8;
        float rs = 0.f;
        if (AM == kAGatedNorm) {
            const int hq = (k0 / 128) * 128;    // head start
            const float* po = (const float*)a.X + (size_t)m * a.ldx;
            rs = head_rsqrt(half_head_ss(po + hq), half_head_ss(po + hq + 64));
        }
        t[c][r] = produce_a<AM>(a, m, k0, rs);
    }
    __syncthreads();
    const int r = tid & 15, c = tid >> 4, m = blockIdx.x * 16 + r;
    if (m < a.M) *(q35_u32x4*)(a.Y + tiled_offset(m, (blockIdx.y * 16 + c) * 8, a.K)) = t[c][r];
}

// ---------------------------------------------------------------- large M
// Plain bf16 A. grid (8 * ceil(N/(16*NW) / 8) * ceil(M/(16*MT)), 1, kEPartial ? KB : 1); NW waves,
// wave w -> column tile NW*(column block) + w; the block's A rows of one k-block are staged in LDS in
// MFMA fragment order (As[m-tile][step][lane]).
// LDS slot of fragment lane (g, r16) at step s: an XOR swizzle that keeps the MFMA reads
// (fixed s, 64 lanes) a permutation of 64 consecutive slots and spreads the staging writes
// (one row: s = 0..7, g = 0..3) over 16 bank groups.
__device__ __forceinline__ int lds_swz(int s, int g, int r16) {
    return g * 16 + (r16 ^ ((s + 8 * (g & 1)) & 15));
}

template <int EM, int MT, int NW, bool FULLK = false>
__global__ void __launch_bounds__(64 * NW) gemm_large_m(GemmArgs a) {
    __shared__ q35_u32x4 As[MT][8][64];
    constexpr int NT = 64 * NW;                    // threads
    constexpr int CPT = MT * 512 / NT;             // 16-byte A chunks per thread per k-block
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // XCD-aware block order: consecutive blocks go round-robin to the 8 XCDs, so block b
    // runs on XCD b % 8; give the M tiles of one column block consecutive slots on the
    // same XCD, so its weight tiles are fetched from HBM once and then hit that XCD's L2.
    const int mb = (a.M + MT * 16 - 1) / (MT * 16);
    const int KB = a.K >> 8;
    constexpr bool KXCD = EM == kEPartial && !FULLK;
    int nblk, rb, kbx = 0;
    if constexpr (KXCD) {
        // one k-block chain per block: XCD x takes k-blocks x, x + 8, ... of every tile, so each
        // slice of A and W is fetched from HBM by one XCD only (the column-block order below
        // fetches A once per XCD); the grid is 8 x tiles x ceil(KB / 8) blocks
        const int nb = (a.N / 16 + NW - 1) / NW, ntiles = nb * mb;
        const int xcd = blockIdx.x & 7, i = blockIdx.x >> 3;
        kbx = xcd + 8 * (i / ntiles);
        if (kbx >= KB) return;
        nblk = (i % ntiles) / mb;
        rb = (i % ntiles) % mb;
    } else {
        const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
        nblk = (idx / mb) * 8 + xcd;
        rb = idx % mb;
    }
    // kESiluMul: waves 0 .. NW/2-1 take gate tiles j, waves NW/2 .. take the up tiles j
    constexpr int HW = NW / 2;
    const int half = a.N / 32;                                  // gate tiles
    const int jg = nblk * HW + (wv % HW);
    if (EM == kESiluMul ? nblk * HW >= half : nblk * NW >= a.N / 16) return;
    const int nt = EM == kESiluMul ? (wv < HW ? jg : half + jg) : nblk * NW + wv;
    const bool nvalid = EM == kESiluMul ? jg < half : nt < a.N / 16;
    const int row0 = rb * MT * 16;
    // kEPartial: one k-block chain per block, or -- FULLK, enough row blocks to fill the
    // chip -- every chain summed in order in the block and stored as chain 0
    const int kb0 = KXCD ? kbx : 0;
    const int kb1 = KXCD ? kbx + 1 : KB;
    q35_f32x4 sum[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) sum[i] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};

    // register double buffer: the loads of k-block kb+1 are in flight while kb computes
    q35_bf16x8 wf[8];
    q35_u32x4 av[CPT];
    auto load_kb = [&](int kb, q35_bf16x8* w, q35_u32x4* x) {
        if (nvalid) {
            const q35_bf16x8* wp = (const q35_bf16x8*)(a.W + ((size_t)nt * KB + kb) * 4096) + lane;
#pragma unroll
            for (int s = 0; s < 8; ++s) w[s] = wp[s * 64];
        }
        // row-contiguous global reads: 32 consecutive threads cover one row's 512 bytes
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 5, kc = c & 31;
            const int m = row0 + row;
            x[i] = m < a.M ? *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + kb * 256 + kc * 8)
                           : (q35_u32x4){0u, 0u, 0u, 0u};
        }
    };
    load_kb(kb0, wf, av);
    for (int kb = kb0; kb < kb1; ++kb) {
        __syncthreads();   // previous k-block's fragments are consumed
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 5, kc = c & 31;
            As[row >> 4][kc & 7][lds_swz(kc & 7, kc >> 3, row & 15)] = av[i];
        }
        q35_bf16x8 wcur[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) wcur[s] = wf[s];
        __syncthreads();
        if (kb + 1 < kb1) load_kb(kb + 1, wf, av);
        if (nvalid) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                q35_f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 8; ++s)
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(As[mt][s][lds_swz(s, lane >> 4, lane & 15)]), wcur[s], c, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) sum[mt][r] = kb == kb0 ? c[r] : sum[mt][r] + c[r];
            }
        }
    }
    if (EM == kESiluMul) {
        // up waves hand bf16(u) to the gate waves through the (now free) A staging area
        float* ub = (float*)&As[0][0][0];                       // [HW][MT][4][64]
        __syncthreads();
        if (wv >= HW && nvalid) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) ub[(((wv - HW) * MT + mt) * 4 + r) * 64 + lane] = rbf(sum[mt][r]);
        }
        __syncthreads();
        if (wv >= HW || !nvalid) return;
        const int col = jg * 16 + (lane & 15);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + mt * 16 + 4 * (lane >> 4) + r;
                const float u = ub[((wv * MT + mt) * 4 + r) * 64 + lane];
                if (row < a.M) a.Y[(size_t)row * a.ldy + col] = f2bf(__fmul_rn(rbf(silu_f(rbf(sum[mt][r]))), u));
            }
        return;
    }
    if (!nvalid) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) epilogue<EM>(a, sum[mt], nt, row0 + mt * 16, lane, KXCD ? kbx : 0);
}

// ---------------------------------------------------------------- K = 1024, batched lanes
// Same column tiles, block order and epilogues as gemm_large_m<EM, MT, 4>, for K = 1024 (the
// hidden size: every input projection and gate|up), used with MT = 2 (32-row blocks). All of
// a block's loads are issued before its first MFMA: per k-block, the A fragments go straight
// into LDS with global_load_lds (layout below) and each wave's 8 weight fragments into
// registers. The k-blocks are then consumed in order, each after an explicit wait for its own
// loads (the vector-memory counter completes in order) and a raw barrier: one L2/HBM round
// trip per block instead of one per k-block. The LDS fragment reads and the weight loads are
// inline asm, so the compiler's wait insertion (which cannot order LDS-DMA against other
// loads) adds no wait for all loads; every wait is explicit and tied to the registers it
// guards. At 256 lanes: gate|up 17.1 us (pipelined kernel 18.2), attention qkv 11.9 (14.8).
constexpr int kPreKB = kHidden / 256;

template <int MT> constexpr int pre_lds_bytes() { return kPreKB * MT * 8 * 64 * 16; }

template <int EM, int MT, int NW = 4>
__global__ void __launch_bounds__(64 * NW) gemm_pre(GemmArgs a) {
    extern __shared__ q35_u32x4 dyn_lds[];
    q35_u32x4(*As)[MT][512] = (q35_u32x4(*)[MT][512])dyn_lds;          // [kb][mt][group * 64 + slot]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int HW = NW / 2;
    const int mb = (a.M + MT * 16 - 1) / (MT * 16);
    const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int nblk = (idx / mb) * 8 + xcd;
    const int half = a.N / 32;
    const int jg = nblk * HW + (wv % HW);
    if (EM == kESiluMul ? nblk * HW >= half : nblk * NW >= a.N / 16) return;   // whole block
    const int nt = EM == kESiluMul ? (wv < HW ? jg : half + jg) : nblk * NW + wv;
    const bool nvalid = EM == kESiluMul ? jg < half : nt < a.N / 16;
    const int ntc = nvalid ? nt : 0;          // invalid waves load a valid tile and store nothing
    const int row0 = (idx % mb) * MT * 16;

    // LDS layout per (k-block, m-tile): 8 KiB groups (g, h) = (k-group, row half), slot
    // row_lo * 8 + (s ^ row_lo) of a group holds A[row h*8 + row_lo][k-group g, step s]. One
    // DMA instruction fills one group: lane j = row_lo * 8 + sx reads chunk s = sx ^ row_lo of
    // its row, so the 64 lanes read 8 whole 128-byte lines; the XOR spreads the MFMA reads
    // (fixed s, rows row_lo = 0..7) over distinct bank groups.
    const int g = lane >> 4;
    const int jrow = lane >> 3, jchunk = (lane & 7) ^ (lane >> 3);
    // weight tile base (wave-uniform, scalar registers) and the lane's byte offset
    const uint16_t* wbase = a.W + (size_t)ntc * kPreKB * 4096;
    const unsigned wvoff = lane * 16;
    q35_u32x4 wf[kPreKB][8];
    constexpr int GPW = MT * 8 / NW;          // (mt, g, h) groups per wave per k-block
    // Load order: the row blocks of one column block (same XCD, same weight tile) start at
    // different k-blocks, k-block (q + rot) % 4 in issue slot q, so they do not all miss on the
    // same weight lines at once (cold weights: a 384 KiB-per-block microbenchmark loads in 7.4
    // instead of 9.1 us). The chains are computed in slot order and summed in k-block order.
    const int rot = (idx % mb) & (kPreKB - 1);
#pragma unroll
    for (int q = 0; q < kPreKB; ++q) {
        const int kb = (q + rot) & (kPreKB - 1);
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const int grp = wv * GPW + i, mt = grp >> 3, gg = (grp >> 1) & 3, h = grp & 1;
            const int m = min(row0 + mt * 16 + h * 8 + jrow, a.M - 1);   // rows >= M feed rows >= M only
            __builtin_amdgcn_global_load_lds(
                (const void*)((const uint16_t*)a.X + (size_t)m * a.ldx + kb * 256 + gg * 64 + jchunk * 8),
                (__attribute__((address_space(3))) void*)&As[q][mt][(gg * 2 + h) * 64], 16, 0, 0);
        }
        // weight fragments through inline asm as well (with LDS-DMA and ordinary loads both
        // pending the compiler treats the counter as out of order and waits for zero); cached
        // loads: the other row blocks of this column block re-read the tile from L2
        const uint16_t* wk0 = wbase + kb * 4096;
        const uint16_t* wk1 = wk0 + 2048;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(wf[q][s]) : "v"(wvoff), "s"(wk0), "n"(s * 1024) : "memory");
#pragma unroll
        for (int s = 4; s < 8; ++s)
            asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(wf[q][s]) : "v"(wvoff), "s"(wk1), "n"((s - 4) * 1024) : "memory");
        __builtin_amdgcn_sched_barrier(0);     // issue order = slot order (the waits below count it)
    }
    // LDS byte offsets of this lane's fragment (row r16 = lane & 15, k-group g) at each step s
    unsigned soff[8];
    {
        const int r16 = lane & 15, h = r16 >> 3, rl = r16 & 7;
#pragma unroll
        for (int s = 0; s < 8; ++s)
            soff[s] = (unsigned)(size_t)(__attribute__((address_space(3))) const void*)&As[0][0][(g * 2 + h) * 64 + rl * 8 + (s ^ rl)];
    }
    q35_f32x4 cq[kPreKB][MT];                 // the chain of slot q (k-block (q + rot) % 4)
#pragma unroll
    for (int q = 0; q < kPreKB; ++q) {
        // this slot's loads are the oldest (GPW + 8) * (kPreKB - q) still counted
        // (tied to this slot's weight registers, so no use of them moves above the wait)
#define Q35_PRE_WAIT(N)                                                                          \
    asm volatile("s_waitcnt vmcnt(%8)"                                                          \
                 : "+v"(wf[q][0]), "+v"(wf[q][1]), "+v"(wf[q][2]), "+v"(wf[q][3]),               \
                   "+v"(wf[q][4]), "+v"(wf[q][5]), "+v"(wf[q][6]), "+v"(wf[q][7])                \
                 : "n"(N) : "memory")
        if (q == 0) Q35_PRE_WAIT((GPW + 8) * 3);
        if (q == 1) Q35_PRE_WAIT((GPW + 8) * 2);
        if (q == 2) Q35_PRE_WAIT(GPW + 8);
        if (q == 3) Q35_PRE_WAIT(0);
#undef Q35_PRE_WAIT
        __builtin_amdgcn_s_barrier();          // every wave's share of the A groups has landed
        asm volatile("" ::: "memory");
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            // the fragment reads are inline asm: the compiler cannot tell which LDS-DMA they
            // depend on and would otherwise wait for every outstanding load (vmcnt(0)) first
            q35_u32x4 af[8];
#pragma unroll
            for (int s = 0; s < 8; ++s)
                asm volatile("ds_read_b128 %0, %1" : "=v"(af[s]) : "v"(soff[s] + (unsigned)((q * MT + mt) * 8192)) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(af[0]), "+v"(af[1]), "+v"(af[2]), "+v"(af[3]), "+v"(af[4]), "+v"(af[5]), "+v"(af[6]), "+v"(af[7]));
            q35_f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s)
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(af[s]), as_bf(wf[q][s]), c, 0, 0, 0);
            cq[q][mt] = c;
        }
    }
    // k-block kb's chain sits in slot (kb - rot) % 4: ((c0 + c1) + c2) + c3
    q35_f32x4 sum[MT];
    auto fold = [&](int s0, int s1, int s2, int s3) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[mt][r] = ((cq[s0][mt][r] + cq[s1][mt][r]) + cq[s2][mt][r]) + cq[s3][mt][r];
    };
    switch (rot) {
        case 0: fold(0, 1, 2, 3); break;
        case 1: fold(3, 0, 1, 2); break;
        case 2: fold(2, 3, 0, 1); break;
        default: fold(1, 2, 3, 0); break;
    }
    if (EM == kESiluMul) {
        // up waves hand bf16(u) to the gate waves through LDS (after every wave's last read)
        float* ub = (float*)dyn_lds;                             // [HW][MT][4][64]
        __syncthreads();
        if (wv >= HW && nvalid) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) ub[(((wv - HW) * MT + mt) * 4 + r) * 64 + lane] = rbf(sum[mt][r]);
        }
        __syncthreads();
        if (wv >= HW || !nvalid) return;
        const int col = jg * 16 + (lane & 15);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + mt * 16 + 4 * g + r;
                const float u = ub[((wv * MT + mt) * 4 + r) * 64 + lane];
                if (row < a.M) a.Y[(size_t)row * a.ldy + col] = f2bf(__fmul_rn(rbf(silu_f(rbf(sum[mt][r]))), u));
            }
        return;
    }
    if (!nvalid) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) epilogue<EM>(a, sum[mt], nt, row0 + mt * 16, lane);
}

// ---------------------------------------------------------------- K = 1024, many rows
// Prompt waves and MTP verify bodies (M >= 512 rows): 256-row x 128-column block tiles of 8 waves
// (one block per CU) and the K = 1024 stream through a six-stage LDS ring of one MFMA step each
// (24 KiB: 16 row tiles and 8 column tiles x 1 KiB), one barrier per stage. A comes in the weights'
// tiled fragment layout (tiled_offset with rows as n: the producing add+norm writes it so), so
// every DMA instruction moves one contiguous KiB that is already a fragment: ds_read_b128 at lane
// * 16 bytes, no swizzle. Wave (wm, wn) owns rows 64 wm .. +64 (4 row tiles) x columns 64 wn ..
// +64 (4 column tiles): 16 MFMAs per 8 fragment reads per step. Software pipelined: while a wave
// issues step j's MFMAs it reads step j + 1's fragments into its other register set (the LDS
// latency hides behind its own matrix work instead of adding to it), and the DMA runs four steps
// ahead of the reads. kESiluMul: wave wn takes gate tiles 2 wn, 2 wn + 1 and the matching up tiles,
// so the SwiGLU is lane-local (64 output columns per block). The steps of a k-block are unrolled, so a chain's first MFMA starts
// from a literal zero. Reduction: the canonical one (per k-block an MFMA chain over its 8 steps
// from zero, chains summed in k-block order), so rows equal the other GEMM forms bit for bit.
constexpr int kWideRing = 6;                        // stages (one MFMA step, 24 KiB each)
constexpr int kWideStage = 24 * 1024;
constexpr int kWideLds = kWideRing * kWideStage;    // 144 KiB

template <int EM>
__global__ void __launch_bounds__(512) gemm_wide(GemmArgs a) {
    extern __shared__ q35_u32x4 dyn_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv >> 1, wn = wv & 1;
    const int mb = (a.M + 255) / 256;
    const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int nblk = (idx / mb) * 8 + xcd, rb = idx % mb;
    const int ntiles = a.N / 16, mtiles = (a.M + 15) / 16;
    const int half = a.N / 32;                                   // kESiluMul: gate tiles
    if (EM == kESiluMul ? nblk * 4 >= half : nblk * 8 >= ntiles) return;
    // the 8 column tiles of this block (kESiluMul: 4 gate tiles, then the matching 4 up tiles)
    auto col_tile = [&](int c) {
        if (EM == kESiluMul) return c < 4 ? nblk * 4 + c : half + nblk * 4 + (c - 4);
        return nblk * 8 + c;
    };
    const int tr0 = rb * 16;                                      // first row tile
    // DMA pieces of a stage: 16 A pieces (row tile t), 8 W pieces (column tile c), piece pc at pc
    // KiB; wave wv issues pieces 3 wv .. 3 wv + 2 (pieces of tiles past the end re-read the last
    // valid tile: unconditional, so the wait counts stay exact)
    const char* pbase[3];
    unsigned ploff[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int pc = 3 * wv + i;
        if (pc < 16) {
            const int t = min(tr0 + pc, mtiles - 1);
            pbase[i] = (const char*)((const uint16_t*)a.X + (size_t)t * 4 * 8 * 512);
        } else {
            const int nt = min(col_tile(pc - 16), ntiles - 1);
            pbase[i] = (const char*)(a.W + (size_t)nt * 4 * 8 * 512);
        }
        ploff[i] = (unsigned)pc * 1024u;
    }
    // stage j = k-block j / 8, step j % 8: the j-th KiB of every tile's 32 KiB
    auto issue = [&](int j) {
        const unsigned koff = (unsigned)j * 1024u;
        char* lds = (char*)dyn_lds + (j % kWideRing) * kWideStage;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(uniform_ptr(pbase[i] + koff) + lane * 16),
                                             (__attribute__((address_space(3))) void*)(lds + ploff[i]), 16, 0, 0);
    };
    // this wave's fragments of a stage: its 4 row tiles' pieces (4 wm + i) and its 4 column
    // tiles' pieces (16 + 4 wn + i), 1 KiB each; the lane's 16 bytes at lane * 16
    const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) const void*)dyn_lds + lane * 16;
    // kESiluMul: wave wn takes gate tiles 2 wn, 2 wn + 1 (pieces 16 + 2 wn + h) and the matching up
    // tiles (pieces 20 + 2 wn + h), so each lane holds both operands of its outputs
    const unsigned abase = lds0 + (unsigned)(wm * 4) * 1024u;
    const unsigned bbase = lds0 + (unsigned)(16 + (EM == kESiluMul ? 2 : 4) * wn) * 1024u;
    constexpr int B2 = EM == kESiluMul ? 4096 : 2048, B3 = B2 + 1024;   // offsets of B tiles 2, 3
    q35_u32x4 fa[2][4], fb[2][4];                                 // two register sets: [set][tile]
    auto rd = [&](int j, q35_u32x4 (&af)[4], q35_u32x4 (&bw)[4]) {
        const unsigned so = (unsigned)((j % kWideRing) * kWideStage);
        const unsigned sa = abase + so, sbb = bbase + so;
#define Q35_WRD(dst, base, off) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "n"(off) : "memory")
        Q35_WRD(af[0], sa, 0); Q35_WRD(af[1], sa, 1024); Q35_WRD(af[2], sa, 2048); Q35_WRD(af[3], sa, 3072);
        Q35_WRD(bw[0], sbb, 0); Q35_WRD(bw[1], sbb, 1024); Q35_WRD(bw[2], sbb, B2); Q35_WRD(bw[3], sbb, B3);
#undef Q35_WRD
    };
    q35_f32x4 c[4][4], sum[4][4];
#pragma unroll
    for (int j = 0; j < kWideRing - 1; ++j) issue(j);
    asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");      // stage 0 landed
    rd(0, fa[0], fb[0]);
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const int j = kb * 8 + jj, cur = jj & 1;
        // stage j + 1 landed for every wave (stages j + 2 .. j + 4 may still be in flight), stage
        // j's fragments are in registers set cur; every wave is done with stage j's slot reads,
        // so the slot of stage j - 1 takes stage j + 5
        // (the last stages issue no DMA, so the count of later stages in flight shrinks to 0). The
        // vector-memory waits carry no register operands: a branch between asm statements that
        // name the fragment registers would let the compiler copy them before the LDS wait.
        if (kb < 3 || jj < 4) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");   // stages j + 2 .. j + 4 out, j <= 27
        else if (jj == 4) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");       // j = 28: stages 30, 31
        else if (jj == 5) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");       // j = 29: stage 31
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier"
                     : "+v"(fa[cur][0]), "+v"(fa[cur][1]), "+v"(fa[cur][2]), "+v"(fa[cur][3]),
                       "+v"(fb[cur][0]), "+v"(fb[cur][1]), "+v"(fb[cur][2]), "+v"(fb[cur][3])
                     :: "memory");
        if (kb < 3 || jj < 3) issue(j + kWideRing - 1);     // stages 5 .. 31
        if (j + 1 < 32) rd(j + 1, fa[cur ^ 1], fb[cur ^ 1]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jn = 0; jn < 4; ++jn)
                c[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(fa[cur][i]), as_bf(fb[cur][jn]),
                                                                    jj == 0 ? (q35_f32x4){0.f, 0.f, 0.f, 0.f} : c[i][jn], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (jj == 7) {                     // k-block kb done: ((c0 + c1) + c2) + c3
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jn = 0; jn < 4; ++jn)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sum[i][jn][r] = kb == 0 ? c[i][jn][r] : sum[i][jn][r] + c[i][jn][r];
        }
    }
    const int row0 = (tr0 + wm * 4) * 16;
    // Epilogue through the drained ring (no DMA is in flight): each wave leaves its bf16 outputs
    // in its own LDS region in row order and stores them back as 16-byte row pieces (the MFMA
    // layout would store 2 bytes per lane); a wave reads only what it wrote, so one block barrier
    // (the ring is drained by every wave) is all the epilogue needs.
    __syncthreads();
    uint16_t* wl = (uint16_t*)dyn_lds;
    if (EM == kESiluMul) {
        // lane holds gate (tiles h) and up (tiles 2 + h) of the same outputs: output tile
        // nblk * 4 + 2 wn + h = bf16(bf16(silu(bf16(g))) * bf16(u))
        uint16_t* ob = wl + (size_t)wv * 2048;                    // [64 rows][32 cols]
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ob[(i * 16 + 4 * (lane >> 4) + r) * 32 + h * 16 + (lane & 15)] =
                        f2bf(__fmul_rn(rbf(silu_f(rbf(sum[i][h][r]))), rbf(sum[i][2 + h][r])));
        wave_sync();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ch = lane + 64 * q, row = ch >> 2, piece = ch & 3;   // 4 pieces of 16 B per row
            const int jt = nblk * 4 + 2 * wn + (piece >> 1);
            const int grow = row0 + row;
            const int col = jt * 16 + (piece & 1) * 8;          // 8 consecutive k: one 16-byte piece
            if (grow < a.M && jt < half)                           // in either layout
                *(q35_u32x4*)(a.Y + (a.y_tiled ? tiled_offset(grow, col, a.ldy) : (size_t)grow * a.ldy + col)) =
                    *(const q35_u32x4*)(ob + row * 32 + piece * 8);
        }
        return;
    }
    uint16_t* ob = wl + (size_t)wv * 4096;                        // [64 rows][64 cols]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jn = 0; jn < 4; ++jn)
#pragma unroll
            for (int r = 0; r < 4; ++r) ob[(i * 16 + 4 * (lane >> 4) + r) * 64 + jn * 16 + (lane & 15)] = f2bf(sum[i][jn][r]);
    wave_sync();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int ch = lane + 64 * q, row = ch >> 3, piece = ch & 7;       // 8 pieces of 16 B per row
        const int nt = nblk * 8 + wn * 4 + (piece >> 1);
        const int grow = row0 + row;
        if (grow < a.M && nt < ntiles)
            *(q35_u32x4*)(a.Y + (size_t)grow * a.ldy + nt * 16 + (piece & 1) * 8) = *(const q35_u32x4*)(ob + row * 64 + piece * 8);
    }
}

// K = 1024 at batched lanes (M <= 511 rows, decode): gemm_wide's ring and pipeline with 64-row x
// 128-column block tiles (224 blocks for gate|up at 256 rows). kEPartial: any K (a multiple of
// 512), all of K in the block and the k-block chains summed in order into chain 0 -- the
// residual projections of prompt waves of >= partial_rows rows (256 blocks at 2,048 rows and
// N = 1024), bit-identical to gemm_large_m's full-K form. 8 waves of 32 x 32 (wave (wm, wn):
// row tiles 2 wm, 2 wm + 1; kEStore: column tiles 2 wn, 2 wn + 1; kESiluMul: gate tile wn and
// the matching up tile, so the SwiGLU is lane-local); stages of two MFMA steps (24 KiB: 4 row
// tiles and 8 column tiles x 2 steps x 1 KiB), a six-stage ring, DMA four stages ahead, the next
// stage's fragments read during the current stage's MFMAs. A in the tiled fragment layout, as
// for gemm_wide. Canonical reduction, bit-identical to the other forms.
template <int EM>
__global__ void __launch_bounds__(512) gemm_wide64(GemmArgs a) {
    extern __shared__ q35_u32x4 dyn_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv >> 2, wn = wv & 3;
    const int mb = (a.M + 63) / 64;
    const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int ntiles = a.N / 16, mtiles = (a.M + 15) / 16;
    const int half = a.N / 32;
    // column blocks by XCD (a weight slab stays in one XCD's L2); kEPartial (N = 1024: 8 column
    // blocks) row blocks by XCD instead, so an XCD fetches its quarter of the long A rows
    // once, not all of A
    const int ncb = (ntiles + 7) / 8;
    const int nblk = EM == kEPartial ? idx % ncb : (idx / mb) * 8 + xcd;
    const int rb = EM == kEPartial ? (idx / ncb) * 8 + xcd : idx % mb;
    if (EM == kEPartial && rb >= mb) return;
    if (EM == kESiluMul ? nblk * 4 >= half : nblk * 8 >= ntiles) return;
    auto col_tile = [&](int c) {
        if (EM == kESiluMul) return c < 4 ? nblk * 4 + c : half + nblk * 4 + (c - 4);
        return nblk * 8 + c;
    };
    const int tr0 = rb * 4;
    const int KB = a.K >> 8, NS = 4 * KB;                             // k-blocks, stages
    // DMA pieces of a stage: 8 A pieces (row tile pc / 2, step pc % 2), 16 W pieces (column tile
    // (pc - 8) / 2, step pc % 2); wave wv issues pieces 3 wv .. 3 wv + 2
    const char* pbase[3];
    unsigned ploff[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int pc = 3 * wv + i;
        if (pc < 8) {
            const int t = min(tr0 + (pc >> 1), mtiles - 1);
            pbase[i] = (const char*)((const uint16_t*)a.X + ((size_t)t * KB * 8 + (pc & 1)) * 512);
        } else {
            const int nt = min(col_tile((pc - 8) >> 1), ntiles - 1);
            pbase[i] = (const char*)(a.W + ((size_t)nt * KB * 8 + (pc & 1)) * 512);
        }
        ploff[i] = (unsigned)pc * 1024u;
    }
    auto issue = [&](int j) {          // stage j: k-block j / 4, steps 2 (j % 4), + 1
        const unsigned koff = (unsigned)((j >> 2) * 8 + (j & 3) * 2) * 1024u;
        char* lds = (char*)dyn_lds + (j % kWideRing) * kWideStage;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(uniform_ptr(pbase[i] + koff) + lane * 16),
                                             (__attribute__((address_space(3))) void*)(lds + ploff[i]), 16, 0, 0);
    };
    const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) const void*)dyn_lds + lane * 16;
    const unsigned abase = lds0 + (unsigned)(wm * 4) * 1024u;        // pieces 2 (2 wm + i) + u
    const unsigned bbase = lds0 + (unsigned)(8 + (EM == kESiluMul ? 2 : 4) * wn) * 1024u;
    constexpr int B1 = EM == kESiluMul ? 8192 : 2048;                 // offset of the second B tile
    q35_u32x4 fa[2][2][2], fb[2][2][2];                               // [set][step][tile]
    auto rd = [&](int j, q35_u32x4 (&af)[2][2], q35_u32x4 (&bw)[2][2]) {
        const unsigned so = (unsigned)((j % kWideRing) * kWideStage);
        const unsigned sa = abase + so, sbb = bbase + so;
#define Q35_WRD(dst, base, off) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "n"(off) : "memory")
        Q35_WRD(af[0][0], sa, 0); Q35_WRD(af[0][1], sa, 2048); Q35_WRD(bw[0][0], sbb, 0); Q35_WRD(bw[0][1], sbb, B1);
        Q35_WRD(af[1][0], sa, 1024); Q35_WRD(af[1][1], sa, 3072); Q35_WRD(bw[1][0], sbb, 1024); Q35_WRD(bw[1][1], sbb, B1 + 1024);
#undef Q35_WRD
    };
    q35_f32x4 c[2][2], sum[2][2];
#pragma unroll
    for (int j = 0; j < kWideRing - 1; ++j) issue(j);
    asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");      // stage 0 landed
    rd(0, fa[0], fb[0]);
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int j = kb * 4 + jj, cur = jj & 1, left = NS - 2 - j;    // stages issued after j + 1
        // stage j + 1 landed for every wave (stages j + 2 .. j + 4 may be in flight; none is
        // issued past the last stage); the vector-memory waits name no registers (see gemm_wide)
        if (left >= 3) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
        else if (left == 2) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else if (left == 1) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier"
                     : "+v"(fa[cur][0][0]), "+v"(fa[cur][0][1]), "+v"(fa[cur][1][0]), "+v"(fa[cur][1][1]),
                       "+v"(fb[cur][0][0]), "+v"(fb[cur][0][1]), "+v"(fb[cur][1][0]), "+v"(fb[cur][1][1])
                     :: "memory");
        if (j + kWideRing - 1 < NS) issue(j + kWideRing - 1);          // stages 5 .. NS - 1
        if (j + 1 < NS) rd(j + 1, fa[cur ^ 1], fb[cur ^ 1]);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn)
                    c[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(fa[cur][u][i]), as_bf(fb[cur][u][jn]),
                                                                        jj == 0 && u == 0 ? (q35_f32x4){0.f, 0.f, 0.f, 0.f} : c[i][jn], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (jj == 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sum[i][jn][r] = kb == 0 ? c[i][jn][r] : sum[i][jn][r] + c[i][jn][r];
        }
    }
    const int row0 = (tr0 + wm * 2) * 16;
    if (EM == kEPartial) {             // full K: the summed chains as chain 0
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {
                const int nt = nblk * 8 + wn * 2 + jn;
                if (nt < ntiles) epilogue<kEPartial>(a, sum[i][jn], nt, row0 + i * 16, lane, 0);
            }
        return;
    }
    __syncthreads();                   // the ring is drained by every wave: wave-private staging
    uint16_t* wl = (uint16_t*)dyn_lds;
    if (EM == kESiluMul) {
        uint16_t* ob = wl + (size_t)wv * 512;                        // [32 rows][16 cols]
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                ob[(i * 16 + 4 * (lane >> 4) + r) * 16 + (lane & 15)] =
                    f2bf(__fmul_rn(rbf(silu_f(rbf(sum[i][0][r]))), rbf(sum[i][1][r])));
        wave_sync();
        const int row = lane >> 1, piece = lane & 1, jt = nblk * 4 + wn, grow = row0 + row;
        if (grow < a.M && jt < half)
            *(q35_u32x4*)(a.Y + (size_t)grow * a.ldy + jt * 16 + piece * 8) = *(const q35_u32x4*)(ob + row * 16 + piece * 8);
        return;
    }
    uint16_t* ob = wl + (size_t)wv * 1024;                           // [32 rows][32 cols]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int r = 0; r < 4; ++r) ob[(i * 16 + 4 * (lane >> 4) + r) * 32 + jn * 16 + (lane & 15)] = f2bf(sum[i][jn][r]);
    wave_sync();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int ch = lane + 64 * q, row = ch >> 2, piece = ch & 3;
        const int nt = nblk * 8 + wn * 2 + (piece >> 1), grow = row0 + row;
        if (grow < a.M && nt < ntiles)
            *(q35_u32x4*)(a.Y + (size_t)grow * a.ldy + nt * 16 + (piece & 1) * 8) = *(const q35_u32x4*)(ob + row * 32 + piece * 8);
    }
}

// ---------------------------------------------------------------- tied lm_head, batched lanes
// K = 1024 (the hidden size), argmax epilogue, launches of M <= 512. Persistent blocks of NW waves,
// about one per CU: a block stages its 64 A rows (64 x 1024 bf16 = 128 KiB) in LDS once, in
// MFMA fragment order, and then walks a stream of column units; each wave computes a 64-row x
// (16 NTW)-column tile per unit, so each A fragment read from LDS feeds NTW MFMAs and each
// weight fragment feeds 4 (one per 16-row tile). The 8 NTW weight fragments of one k-block
// live in a rolling register buffer: the slot of (column tile n, step s) is refilled with
// the next k-block's (or the next unit's first k-block's) fragment right after its last
// use, so the weight stream stays one k-block ahead of the MFMAs without a second buffer.
// Used as <8, 2>: two waves per SIMD hide the weight-stream latency (275 us for M = 256 on
// MI355X against 400 us for the 64 x 256 tiled kernel, whose waves each re-read the whole A
// tile from LDS; <4, 4> at one wave per SIMD: 420 us). The row blocks of one column stream
// sit on one XCD and share each weight unit through its L2.
// Reduction order = the canonical one above (chain per k-block from zero, summed in order).
constexpr int kLmKB = kHidden / 256;
constexpr int kLmLds = 4 * kLmKB * 8 * 64 * 16;          // 128 KiB of A fragments

template <int NW, int NTW>
__global__ void __launch_bounds__(64 * NW) gemm_lmhead(GemmArgs a, int mb) {
    extern __shared__ q35_u32x4 dyn_lds[];
    q35_u32x4(*As)[kLmKB * 8][64] = (q35_u32x4(*)[kLmKB * 8][64])dyn_lds;   // [mt][kb*8+s][slot]
    constexpr int NT = 64 * NW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar addressing
    // blocks b, b + 8, ... run on XCD b % 8; the mb row blocks of one column stream take
    // consecutive slots there, so a weight unit is fetched from HBM once per XCD
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int rb = k % mb;
    const int streams = gridDim.x / mb;                      // a multiple of 8
    const int stream = (k / mb) * 8 + xcd;
    const int row0 = rb * 64;
    const int nunits = a.N / (16 * NTW);                     // wave units of NTW column tiles
    const int ustride = streams * NW;
    int u = stream * NW + wv;

    // weight fragment (unit, column tile n, k-block, step s): one lane-contiguous KiB, read
    // with buffer loads -- scalar resource + uniform scalar byte offset + the lane's 16-byte
    // offset, so no 64-bit address is held per fragment (the weight matrix is < 4 GiB)
    const __amdgpu_buffer_rsrc_t wres =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, 0, (int)((size_t)a.N * kHidden * 2), 0x00020000);
    const int voff = lane * 16;
    auto wload = [&](int unit, int n, int kb, int s) {
        const int so = (((unit * NTW + n) * kLmKB + kb) * 512 + s * 64) * 16;
        // cached: the other row blocks of this column stream on the XCD re-read it from L2
        q35_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wres, voff, so, 0);
        return *(q35_bf16x8*)&v;
    };
    const int u0 = min(u, nunits - 1);
    q35_bf16x8 wf[NTW][8];
#pragma unroll
    for (int n = 0; n < NTW; ++n)
#pragma unroll
        for (int s = 0; s < 8; ++s) wf[n][s] = wload(u0, n, 0, s);

    // stage A: chunk c = row * 32 + kk of a k-block (8 elements each); zero rows beyond M
#pragma unroll
    for (int kb = 0; kb < kLmKB; ++kb) {
        constexpr int CPT = 2048 / NT;
        q35_u32x4 v[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 5, kk = c & 31;
            const int m = min(row0 + row, a.M - 1);
            v[i] = *(const q35_u32x4*)((const uint16_t*)a.X + (size_t)m * a.ldx + kb * 256 + kk * 8);
        }
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 5, kk = c & 31;
            const q35_u32x4 z = {0u, 0u, 0u, 0u};
            As[row >> 4][kb * 8 + (kk & 7)][lds_swz(kk & 7, kk >> 3, row & 15)] = row0 + row < a.M ? v[i] : z;
        }
        __builtin_amdgcn_sched_barrier(0);     // one k-block of staging registers at a time
    }
    __syncthreads();

    int sw[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) sw[s] = lds_swz(s, lane >> 4, lane & 15);
    for (; u < nunits; u += ustride) {
        const int un = min(u + ustride, nunits - 1);         // next unit (clamped: a reload)
        q35_f32x4 sum[4][NTW];
        q35_u32x4 af[4], an[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) an[mt] = As[mt][0][sw[0]];
#pragma unroll
        for (int kb = 0; kb < kLmKB; ++kb) {
            q35_f32x4 c[4][NTW];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) af[mt] = an[mt];
                // the next step's A fragments are read while this step's MFMAs run
                const int kn = s < 7 ? kb : kb + 1, sn = (s + 1) & 7;
                if (kn < kLmKB) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) an[mt] = As[mt][kn * 8 + sn][sw[sn]];
                }
                __builtin_amdgcn_sched_barrier(0);   // those reads go out before the MFMAs
#pragma unroll
                for (int n = 0; n < NTW; ++n) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        c[mt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            as_bf(af[mt]), wf[n][s], s == 0 ? (q35_f32x4){0.f, 0.f, 0.f, 0.f} : c[mt][n], 0, 0, 0);
                    wf[n][s] = kb + 1 < kLmKB ? wload(u, n, kb + 1, s) : wload(un, n, 0, s);
                }
                // keep the refills where they are issued (the scheduler would otherwise sink
                // them next to their use a k-block later and wait on each)
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int n = 0; n < NTW; ++n) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) sum[mt][n][r] = kb == 0 ? c[mt][n][r] : sum[mt][n][r] + c[mt][n][r];
                    asm volatile("" : "+a"(sum[mt][n]));   // running sums wait in AGPRs: the
                }                                           // VGPRs hold the weight stream
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int n = 0; n < NTW; ++n) {
                // opaque per unit, so the row offsets are not hoisted out of the unit loop
                // (kept live across it they would spill, and a spill reload drains the stream)
                int r0 = row0 + mt * 16;
                asm volatile("" : "+s"(r0));
                epilogue<kEArgmax>(a, sum[mt][n], u * NTW + n, r0, lane);
                __builtin_amdgcn_sched_barrier(0);   // one tile's temporaries at a time
            }
    }
}

// Tied lm_head at batched lanes, second form: A in registers, the weight stream through an LDS
// ring. A block of 8 waves owns 128 rows; wave w holds all 32 A fragments of rows 16 w .. +16
// (128 VGPRs) and computes their full k-block chains in order, so each weight fragment read
// from LDS feeds the 8 row groups of the block and no chain crosses waves. Units are single
// 16-column tiles (all four k-blocks: 32 KiB, contiguous in the tiled layout); the ring holds
// four of them and the DMA runs three units ahead (global_load_lds by all 512 threads). The
// LDS fragment reads are inline asm (the compiler would make them wait for the in-flight DMA).
// Argmax epilogue: each lane keeps the running (max, index) of its column over the stream's
// tiles (their columns increase, so a strict > keeps the lowest index among equal values) and
// the 16 lanes of a row are reduced once at the end: one (max, index) partial per (row, stream)
// instead of one per (row, tile) -- the per-tile partial stores took half the kernel's time.
constexpr int kLm3Unit = kLmKB * 8 * 64 * 16;                     // 32 KiB
constexpr int kLm3Ring = 4;
constexpr int kLm3Lds = kLm3Ring * kLm3Unit;                       // 128 KiB

__global__ void __launch_bounds__(512) gemm_lmhead3(GemmArgs a, int mb) {
    extern __shared__ q35_u32x4 dyn_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int rb = k % mb;
    const int streams = gridDim.x / mb;
    const int stream = (k / mb) * 8 + xcd;
    const int row0 = rb * 128 + wv * 16;
    const int nunits = a.N / 16;

    q35_u32x4 af[kLmKB][8];
    {
        const int m = row0 + (lane & 15), g = lane >> 4;
        const uint16_t* xr = (const uint16_t*)a.X + (size_t)min(m, a.M - 1) * a.ldx;
#pragma unroll
        for (int kb = 0; kb < kLmKB; ++kb)
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const q35_u32x4 v = *(const q35_u32x4*)(xr + kb * 256 + g * 64 + s * 8);
                af[kb][s] = m < a.M ? v : (q35_u32x4){0u, 0u, 0u, 0u};
            }
    }
    // unit u's 32 KiB into ring slot r: 4 DMA instructions per thread, 16 bytes each
    auto fetch = [&](int u, int r) {
        const char* src = (const char*)(a.W + (size_t)u * kLmKB * 4096);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)(i * 512 + tid) * 16),
                                             (__attribute__((address_space(3))) void*)(dyn_lds + r * 2048 + i * 512 + wv * 64),
                                             16, 0, 0);
    };
    // the units of this stream: stream, stream + streams, ...; n-th unit in ring slot n % 4.
    // Issued: always 3 ahead (past the end, a clamped reload of the last unit, so the per-unit
    // DMA count -- and thus the wait count -- is constant)
    const int nmine = stream < nunits ? (nunits - 1 - stream) / streams + 1 : 0;
    auto unit_of = [&](int i) { return stream + min(i, nmine - 1) * streams; };
    if (nmine > 0) {
#pragma unroll
        for (int i = 0; i < kLm3Ring - 1; ++i) fetch(unit_of(i), i);
    }
    const unsigned lds_lane = (unsigned)(size_t)(__attribute__((address_space(3))) const void*)dyn_lds + lane * 16;
    float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    int bidx[4] = {0x7fffffff, 0x7fffffff, 0x7fffffff, 0x7fffffff};
    for (int i = 0; i < nmine; ++i) {
        // unit i landed (the 2 later units' 8 DMAs may still be in flight), for every wave
        asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
        fetch(unit_of(i + kLm3Ring - 1), (i + kLm3Ring - 1) % kLm3Ring);
        const unsigned base = lds_lane + (unsigned)((i % kLm3Ring) * kLm3Unit);
        // two k-blocks' chains at a time, interleaved step by step; their 16 fragment reads are
        // issued in (step, k-block) order and waited for two at a time (lgkmcnt counts to 15)
        q35_f32x4 c[kLmKB];
#pragma unroll
        for (int kp = 0; kp < kLmKB; kp += 2) {
            q35_u32x4 wf[8][2];
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(wf[s][h]) : "v"(base), "n"(((kp + h) * 8 + s) * 1024) : "memory");
            c[kp] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
            c[kp + 1] = (q35_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                switch (s) {      // the immediate must be a constant: reads 2s, 2s + 1 have landed
                    case 0: asm volatile("s_waitcnt lgkmcnt(14)" : "+v"(wf[0][0]), "+v"(wf[0][1])); break;
                    case 1: asm volatile("s_waitcnt lgkmcnt(12)" : "+v"(wf[1][0]), "+v"(wf[1][1])); break;
                    case 2: asm volatile("s_waitcnt lgkmcnt(10)" : "+v"(wf[2][0]), "+v"(wf[2][1])); break;
                    case 3: asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(wf[3][0]), "+v"(wf[3][1])); break;
                    case 4: asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(wf[4][0]), "+v"(wf[4][1])); break;
                    case 5: asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(wf[5][0]), "+v"(wf[5][1])); break;
                    case 6: asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(wf[6][0]), "+v"(wf[6][1])); break;
                    default: asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wf[7][0]), "+v"(wf[7][1])); break;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    c[kp + h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(af[kp + h][s]), as_bf(wf[s][h]), c[kp + h], 0, 0, 0);
            }
        }
        q35_f32x4 sum;
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] = ((c[0][r] + c[1][r]) + c[2][r]) + c[3][r];
        const int col = unit_of(i) * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 4 * (lane >> 4) + r;
            const float v = rbf(sum[r]);
            if (row < a.M && a.logits) a.logits[(unsigned)(row * a.ldl + col)] = v;
            if (v > best[r]) { best[r] = v; bidx[r] = col; }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = row0 + 4 * (lane >> 4) + r;
        argmax16(best[r], bidx[r]);
        if ((lane & 15) == 0 && row < a.M && nmine > 0) {
            a.part_val[(unsigned)(row * a.ldp + stream)] = best[r];
            a.part_idx[(unsigned)(row * a.ldp + stream)] = bidx[r];
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the clamped reloads past the end
}

// column streams of the gemm_lmhead3 launch for M <= 512 rows (128 rows per block)
static int lmhead3_streams(int M) {
    const int mb3 = (M + 127) / 128;
    return 256 / mb3 / 8 * 8;
}

// Final argmax over the per-tile partials of each row: lowest id among the maxima.
__global__ void __launch_bounds__(1024) argmax_rows(const float* pv, const int* pi, int ldp, int n,
                                                    int* out_tok, float* out_val) {
    const int row = blockIdx.x;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i0 = 0; i0 < n; i0 += 16 * 1024) {
        float v[16];
        int id[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {       // all loads first
            const int i = i0 + u * 1024 + threadIdx.x;
            v[u] = i < n ? pv[(size_t)row * ldp + i] : -INFINITY;
            id[u] = i < n ? pi[(size_t)row * ldp + i] : 0x7fffffff;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (v[u] > best || (v[u] == best && id[u] < bi)) { best = v[u]; bi = id[u]; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = __shfl_xor(best, o, 64);
        int i2 = __shfl_xor(bi, o, 64);
        if (v2 > best || (v2 == best && i2 < bi)) { best = v2; bi = i2; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
        for (int w = 1; w < 16; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) { best = sv[w]; bi = si[w]; }
        out_tok[row] = bi;
        if (out_val) out_val[row] = best;
    }
}

// kEPartial GEMMs with at least forms.partial_rows rows sum all k-block chains in the block
// (one chain left for the add+norm) instead of one block per chain
int gemm_partial_chains(int M, int K, const KernelForms& f) { return M > 16 && M >= f.partial_rows ? 1 : K / 256; }
bool wide_fullk(const KernelForms& f, int M) { return f.gemm_wide && M >= 512 && M >= f.partial_rows; }

// many rows, A in the tiled layout: K = 1024, stored or SwiGLU outputs only
static hipError_t launch_wide(const GemmArgs& a, int em, hipStream_t st) {
    if (em == kEPartial) {             // full K into chain 0 (64 x 128 blocks)
        if (a.M < a.forms.partial_rows || a.M <= 16 || a.K % 512 || !a.kpart || a.N % 16) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemm_wide64<kEPartial>, dim3(((a.N / 16 + 7) / 8) * (((a.M + 63) / 64 + 7) / 8 * 8)), dim3(512), kWideLds, st, a);
        return hipGetLastError();
    }
    if (a.K != kHidden || a.M <= 16 || (em != kEStore && em != kESiluMul) || !a.Y || (em == kESiluMul && a.N % 32) ||
        a.ldy % 8 || ((uintptr_t)a.Y & 15) || (a.y_tiled && (em != kESiluMul || a.M < 512 || a.ldy % 256)))
        return hipErrorInvalidValue;        // 16-byte row pieces in the epilogue
    const int nb = em == kESiluMul ? (a.N / 32 + 3) / 4 : (a.N / 16 + 7) / 8;
    if (a.M < 512) {                   // batched lanes: 64-row blocks
        const int mb = (a.M + 63) / 64;
        if (em == kESiluMul) hipLaunchKernelGGL(gemm_wide64<kESiluMul>, dim3((nb + 7) / 8 * 8 * mb), dim3(512), kWideLds, st, a);
        else hipLaunchKernelGGL(gemm_wide64<kEStore>, dim3((nb + 7) / 8 * 8 * mb), dim3(512), kWideLds, st, a);
        return hipGetLastError();
    }
    const int mb = (a.M + 255) / 256;
    if (em == kEStore && nb * mb > 256 && (nb * mb) % 256 <= 64 && (nb * mb) % 256 % mb == 0) {
        // a last round of at most a quarter of the CUs (the GDN in_proj's 65th column block of 2
        // tiles, the attention qkv's last 8 at 2,048 rows): whole rounds of 256 x 128 blocks, the
        // remaining columns as 64-row blocks (16 stages) in a launch of their own; the same bits
        const int nbm = (nb * mb - (nb * mb) % 256) / mb;
        GemmArgs h = a, t = a;
        h.N = nbm * 128;
        t.N = a.N - h.N;
        t.W = a.W + (size_t)(h.N / 16) * (a.K / 256) * 4096;
        t.Y = a.Y + h.N;
        hipLaunchKernelGGL(gemm_wide<kEStore>, dim3((nbm + 7) / 8 * 8 * mb), dim3(512), kWideLds, st, h);
        const int nbt = (t.N / 16 + 7) / 8;
        hipLaunchKernelGGL(gemm_wide64<kEStore>, dim3((nbt + 7) / 8 * 8 * ((a.M + 63) / 64)), dim3(512), kWideLds, st, t);
        return hipGetLastError();
    }
    if (em == kESiluMul) hipLaunchKernelGGL(gemm_wide<kESiluMul>, dim3((nb + 7) / 8 * 8 * mb), dim3(512), kWideLds, st, a);
    else hipLaunchKernelGGL(gemm_wide<kEStore>, dim3((nb + 7) / 8 * 8 * mb), dim3(512), kWideLds, st, a);
    return hipGetLastError();
}

template <int EM>
static void launch_large(const GemmArgs& a, hipStream_t st) {
    const int KB = a.K / 256;
    const int gz = EM == kEPartial ? (a.M >= a.forms.partial_rows ? 1 : KB) : 1;
    // 64-row tiles: more blocks in flight (W tiles are re-read from L2 by the M tiles)
    const int nb = EM == kESiluMul ? (a.N / 32 + 1) / 2 : (a.N / 16 + 3) / 4, mb = (a.M + 63) / 64;
    if (EM == kEArgmax && a.K == kHidden && a.N % 64 == 0 && a.forms.lmhead_persist) {
        // persistent blocks, one per CU: gemm_lmhead3 (form 3: 128 rows per block, A in
        // registers) or gemm_lmhead (form 1: 64 rows per block, A resident in LDS), row blocks x
        // column streams = 256 blocks. Above 512 rows (MTP verify: 3 rows per lane) in launches
        // of at most 256 rows: rows are independent, and one pass with more row blocks than CUs
        // would run a second partial wave of blocks.
        for (int r0 = 0; r0 < a.M; r0 += a.M > 512 ? 256 : a.M) {
            GemmArgs c = a;
            c.M = min(a.M - r0, a.M > 512 ? 256 : a.M);
            c.X = (const uint16_t*)a.X + (size_t)r0 * a.ldx;
            if (a.logits) c.logits = a.logits + (size_t)r0 * a.ldl;
            c.part_val = a.part_val + (size_t)r0 * a.ldp;
            c.part_idx = a.part_idx + (size_t)r0 * a.ldp;
            const int mbk = (c.M + 63) / 64;
            const int streams = max(8, 256 / mbk / 8 * 8);
            if (a.forms.lmhead_persist == 3) {
                const int mb3 = (c.M + 127) / 128;
                hipLaunchKernelGGL(gemm_lmhead3, dim3(lmhead3_streams(c.M) * mb3), dim3(512), kLm3Lds, st, c, mb3);
            } else
                hipLaunchKernelGGL((gemm_lmhead<8, 2>), dim3(mbk * streams), dim3(512), kLmLds, st, c, mbk);
        }
        return;
    }
    if (EM == kEArgmax) {
        // tied lm_head (N = 248,320): 16 waves x 16 columns share each staged A tile, so the
        // A rows are re-read from L2 by 4x fewer blocks (measured best of 64x64, 128x128, 64x256)
        const int nb16 = (a.N / 16 + 15) / 16;
        hipLaunchKernelGGL((gemm_large_m<EM, 4, 16>), dim3((nb16 + 7) / 8 * 8 * mb, 1, gz), dim3(1024), 0, st, a);
        return;
    }
    if ((EM == kEStore || EM == kESiluMul) && a.K == kHidden && a.forms.gemm_pre) {
        // 32-row blocks (64 KiB of A fragments: two blocks per CU); 64-row blocks (128 KiB,
        // one per CU) measured 10-35 % slower
        // 64 x 128 blocks of 8 waves (one per CU, half the L2 -> CU bytes per output of the
        // 32 x 64 tiles) when they fill the CUs in one round: gate|up at 256 lanes, 224 blocks,
        // 16.8 -> 14.8 us in the model (in_proj's 288 blocks take two rounds: 21.7 us against
        // 17.0; the attention qkv's 160 blocks leave CUs idle: 12.8 against 12.0); form 2 forces
        // them (tests)
        const int nb8 = EM == kESiluMul ? (a.N / 32 + 3) / 4 : (a.N / 16 + 7) / 8, mb4 = (a.M + 63) / 64;
        const int grid8 = (nb8 + 7) / 8 * 8 * mb4;
        if (a.forms.gemm_pre == 2 || (grid8 <= 256 && 4 * grid8 > 3 * 256)) {
            hipLaunchKernelGGL((gemm_pre<EM, 4, 8>), dim3(grid8), dim3(512), pre_lds_bytes<4>(), st, a);
            return;
        }
        const int mb2 = (a.M + 31) / 32;
        hipLaunchKernelGGL((gemm_pre<EM, 2>), dim3((nb + 7) / 8 * 8 * mb2), dim3(256), pre_lds_bytes<2>(), st, a);
        return;
    }
    if (EM == kEPartial && gz == 1)
        hipLaunchKernelGGL((gemm_large_m<EM, 4, 4, true>), dim3((nb + 7) / 8 * 8 * mb, 1, 1), dim3(256), 0, st, a);
    else if (EM == kEPartial)      // k-blocks by XCD: 8 x tiles x ceil(KB / 8) blocks
        hipLaunchKernelGGL((gemm_large_m<EM, 4, 4>), dim3(8 * nb * mb * ((gz + 7) / 8)), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_large_m<EM, 4, 4>), dim3((nb + 7) / 8 * 8 * mb, 1, 1), dim3(256), 0, st, a);
}

template <int AM, int EM>
static hipError_t launch_am_em(const GemmArgs& a, hipStream_t st) {
    const int KB = a.K / 256;
    if (a.M <= 16) {
        const int waves = EM == kEPartial ? 1 : KB;
        const size_t lds = AM == kAPlain ? 0 : (size_t)waves * (512 * 16 + 64 * 4);
        if (EM == kEPartial)
            hipLaunchKernelGGL((gemm_small_m<AM, EM>), dim3(a.N / 16, 1, KB), dim3(64), lds, st, a);
        else if ((AM == kANormX || AM == kANormXP) && EM == kEStore && a.M == 1 && a.forms.gemv_tpb == 2 &&
                 a.N % 32 == 0 && a.N >= 4096 && KB == 4) {
            if (AM == kANormXP && a.kpb <= 8)      // after out_proj / o_proj (8 chains)
                hipLaunchKernelGGL((gemm_small_m<AM, EM, 2, 8>), dim3(a.N / 32, 1, 1), dim3(64 * KB), 0, st, a);
            else if (a.N / 32 > 256 && a.N / 16 - 512 <= 256)   // GDN in_proj: 256 blocks, 2 of them 3 tiles
                hipLaunchKernelGGL((gemm_small_m<AM, EM, 2, 16, true>), dim3(256, 1, 1), dim3(64 * KB), 0, st, a);
            else
                hipLaunchKernelGGL((gemm_small_m<AM, EM, 2>), dim3(a.N / 32, 1, 1), dim3(64 * KB), 0, st, a);
        } else
            hipLaunchKernelGGL((gemm_small_m<AM, EM>), dim3(a.N / 16, 1, 1), dim3(64 * KB), lds, st, a);
        return hipGetLastError();
    }
    if (EM == kEResidual || AM == kANormX || AM == kANormXP) return hipErrorInvalidValue;   // batch-1 forms only
    if (a.x_tiled) {
        if (AM != kAPlain) return hipErrorInvalidValue;
        return launch_wide(a, EM, st);
    }
    if (AM != kAPlain) {
        // produce A once into a.prod (bf16 [M][K]), then the plain batched GEMM (the many-row
        // full-K residual projection: A produced in the tiled layout)
        if (!a.prod) return hipErrorInvalidValue;
        GemmArgs p = a;
        p.Y = a.prod;
        p.ldy = a.K;
        if (EM == kEPartial && wide_fullk(a.forms, a.M) && a.K % 512 == 0) {
            hipLaunchKernelGGL((produce_tiled_kernel<AM>), dim3((a.M + 15) / 16, a.K / 128), dim3(256), 0, st, p);
            GemmArgs g = a;
            g.X = a.prod;
            g.ldx = a.K;
            g.x_tiled = 1;
            return launch_wide(g, kEPartial, st);
        }
        hipLaunchKernelGGL((produce_kernel<AM>), dim3(a.M), dim3(256), 0, st, p);
        GemmArgs g = a;
        g.X = a.prod;
        g.ldx = a.K;
        launch_large<EM == kEResidual ? kEStore : EM>(g, st);
    } else {
        launch_large<EM == kEResidual ? kEStore : EM>(a, st);
    }
    return hipGetLastError();
}

hipError_t gemm_init() {
    const int big = 16 * (512 * 16 + 64 * 4);
#define Q35_ATTR(AMV, EMV)                                                                              \
    if (hipFuncSetAttribute((const void*)gemm_small_m<AMV, EMV>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                            big) != hipSuccess) return hipGetLastError();
    Q35_ATTR(kASiluMul, kEStore) Q35_ATTR(kASiluMul, kEPartial) Q35_ATTR(kASiluMul, kEResidual)
    Q35_ATTR(kAGatedNorm, kEStore) Q35_ATTR(kAGatedNorm, kEPartial) Q35_ATTR(kAGatedNorm, kEResidual)
    Q35_ATTR(kANormX, kEStore) Q35_ATTR(kANormX, kEArgmax) Q35_ATTR(kANormXP, kEStore)
#undef Q35_ATTR
    if (hipFuncSetAttribute((const void*)gemm_lmhead<8, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, kLmLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_lmhead3, hipFuncAttributeMaxDynamicSharedMemorySize, kLm3Lds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_pre<kEStore, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, pre_lds_bytes<2>()) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_pre<kESiluMul, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, pre_lds_bytes<2>()) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_pre<kEStore, 4, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, pre_lds_bytes<4>()) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_pre<kESiluMul, 4, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, pre_lds_bytes<4>()) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_wide<kEStore>, hipFuncAttributeMaxDynamicSharedMemorySize, kWideLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_wide<kESiluMul>, hipFuncAttributeMaxDynamicSharedMemorySize, kWideLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_wide64<kEStore>, hipFuncAttributeMaxDynamicSharedMemorySize, kWideLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_wide64<kESiluMul>, hipFuncAttributeMaxDynamicSharedMemorySize, kWideLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)gemm_wide64<kEPartial>, hipFuncAttributeMaxDynamicSharedMemorySize, kWideLds) != hipSuccess)
        return hipGetLastError();
    return hipSuccess;
}

hipError_t launch_gemm(const GemmArgs& a, int amode, int emode, hipStream_t st) {
    if (a.K % 256 || a.N % 16 || a.K > 4096 || a.M <= 0) return hipErrorInvalidValue;
    if (emode == kEPartial && (!a.kpart || a.K / 256 > 16)) return hipErrorInvalidValue;
    if (emode == kEResidual && (!a.xres || a.N != kHidden)) return hipErrorInvalidValue;
    if (amode == kANormX && a.K != kHidden) return hipErrorInvalidValue;
    if (amode == kANormXP && (a.K != kHidden || a.M != 1 || !a.kpart || !a.xres || a.kpb < 1 ||
                              a.kpb > 16 || emode != kEStore))
        return hipErrorInvalidValue;
#define Q35_AM(EMV)                                                          \
    if (amode == kAPlain) return launch_am_em<kAPlain, EMV>(a, st);          \
    if (amode == kASiluMul) return launch_am_em<kASiluMul, EMV>(a, st);      \
    if (amode == kAGatedNorm) return launch_am_em<kAGatedNorm, EMV>(a, st);  \
    return hipErrorInvalidValue;
    if (emode == kEStore) {
        if (amode == kANormX) return launch_am_em<kANormX, kEStore>(a, st);
        if (amode == kANormXP) return launch_am_em<kANormXP, kEStore>(a, st);
        Q35_AM(kEStore)
    }
    if (emode == kEPartial) { Q35_AM(kEPartial) }
    if (emode == kEResidual) { Q35_AM(kEResidual) }
    if (emode == kESiluMul) {       // batched lanes only: a plain A operand, Y = act [M][N/2]
        if (amode != kAPlain || a.M <= 16 || a.N % 32 || !a.Y) return hipErrorInvalidValue;
        if (a.x_tiled) return launch_wide(a, kESiluMul, st);
        launch_large<kESiluMul>(a, st);
        return hipGetLastError();
    }
    if (emode == kEArgmax && amode == kAPlain) return launch_am_em<kAPlain, kEArgmax>(a, st);
    if (emode == kEArgmax && amode == kANormX) return launch_am_em<kANormX, kEArgmax>(a, st);
#undef Q35_AM
    return hipErrorInvalidValue;
}

hipError_t launch_produce(const GemmArgs& a, int amode, hipStream_t st) {
    if (!a.prod || a.M <= 0 || a.K % 256) return hipErrorInvalidValue;
    GemmArgs p = a;
    p.Y = a.prod;
    p.ldy = a.K;
    if (amode == kASiluMul) hipLaunchKernelGGL((produce_kernel<kASiluMul>), dim3(a.M), dim3(256), 0, st, p);
    else if (amode == kAGatedNorm) hipLaunchKernelGGL((produce_kernel<kAGatedNorm>), dim3(a.M), dim3(256), 0, st, p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

int gemm_argmax_partials(const GemmArgs& a) {
    if (a.M > 16 && a.K == kHidden && a.N % 64 == 0 && a.forms.lmhead_persist == 3)
        return std::min(lmhead3_streams(a.M > 512 ? 256 : a.M), a.N / 16);
    return (a.N + 15) / 16;
}

hipError_t launch_argmax(const float* pv, const int* pi, int ldp, int n, int rows, int* tok,
                         float* val, hipStream_t st) {
    hipLaunchKernelGGL(argmax_rows, dim3(rows), dim3(1024), 0, st, pv, pi, ldp, n, tok, val);
    return hipGetLastError();
}

}  // namespace q35
