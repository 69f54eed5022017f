// GatedDeltaNet over a prompt wave of one lane in the chunked (UT-transform) form, chunk 64
// (speccheck/specimpl.py:187-235; the reference engine's gdn_chunk_prefill,
// engine/kernels_gdn.cpp:488). Four kernels:
//
//   gdn_chunk_conv  grid (16-row run, 256 channels): causal conv + bf16 SiLU of every (row,
//                   channel) of the wave with the recurrent kernel's arithmetic -> conv_u, and
//                   the conv window after the wave
//   gdn_chunk_prep  grid (chunk, head): L2 norms and gates with the recurrent kernel's
//                   arithmetic; then, within the chunk, the decay prefix
//                   cum_i = g_0 + .. + g_i, the pairwise-decayed products
//                   ut = (beta k~) k~^T (strictly lower) and intra = q~ k~^T (lower), the two
//                   unit-lower-triangular solves (I + ut) nv = beta v and
//                   (I + ut) kcd = beta k~ e^cum, and q' = q~ e^cum, k' = k~ e^(cum_63 - cum).
//                   Rows past the wave are zero with g = beta = 0, as the reference pads.
//   gdn_chunk_scan  grid (head, 16-column slice): the chunk recurrence, sequential over chunks
//                   with the slice S[:, n0 .. n0+16) of the f32 state in LDS:
//                     v_new = nv - kcd S;  S = e^cum_63 S + k'^T v_new
//                   on v_mfma_f32_16x16x4_f32 (f32 products, f32 accumulate). The value columns
//                   of the delta rule never mix, so 8 slices per head run independently. Each
//                   chunk's S (before its update) and v_new go to the workspace as bf16 hi / lo
//                   MFMA fragments for
//   gdn_chunk_out   grid (chunk, head): o = q' S + intra v_new of every chunk at once (off the
//                   recurrence's sequential path) on v_mfma_f32_16x16x32_bf16, each operand a
//                   bf16 hi / lo pair (x = hi + lo within 2^-18 |x|) and each product hi.hi +
//                   hi.lo + lo.hi, f32 accumulate.
//
// The state is read from slot cur and written to slot (cur + 1) % nslots (no rows pending:
// the engine applies them first), the conv window, from slot wcur to (wcur + 1) % nslots,
// likewise, exactly as the recurrent kernel does for a wave without checkpoints.
#include <type_traits>

#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

constexpr int kC = 64;                      // chunk rows
constexpr int kCWs = 4 * kC * 128 + kC * kC + 8 * 3072;   // workspace floats per (chunk, head)
// Workspace per (chunk, head), written by the prep kernel directly in the scan's MFMA operand
// order so that every scan wave reads its operands as contiguous 16-byte vectors
// (lane = 16 kq + mr, see mfma4):
//   kcd  [wave 4][lane 64][ks 32]  A[m = 16w + mr][k = 4ks + kq]      (phase 1)
//   q'   [wave 4][kb 4][part 2][lane 64] x 8 bf16  A[m = 16w + lane % 16][k = 32kb + 8(lane / 16) + e]
//   intra[wave 4][kb 2][part 2][lane 64] x 8 bf16  A[m = 16w + lane % 16][j = 32kb + 8(lane / 16) + e]
//        (gdn_chunk_out: part 0 = bf16(x), part 1 = bf16(x - part 0))
//   k'^T [wave 4][half 2][lane 64][ks 16]  A[m = 32w + 16half + mr][i = 4ks + kq] = k'[i][m]  (phase 3)
//   nv   [slice 8][wave 4][lane 64][r 4]   nv[16w + 4kq + r][16 slice + mr]   (phase 1, C layout)
//   Sb   [slice 8][kb 4][part 2][lane 64] x 8 bf16  S[32kb + 8(lane / 16) + e][16 slice + lane % 16]
//        (the chunk's state before its update; written by the scan)
//   Vb   [slice 8][kb 2][part 2][lane 64] x 8 bf16  v_new[32kb + 8(lane / 16) + e][16 slice + lane % 16]
constexpr int kWsKcd = 0, kWsQ = 8192, kWsIntra = 16384, kWsK = 20480, kWsNv = 28672, kWsSb = 36864,
              kWsVb = 53248;

// MFMA f32 16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
// D[4 (l/16) + r][l%16], r = 0..3.
__device__ __forceinline__ q35_f32x4 mfma4(float av, float bv, q35_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, c, 0, 0, 0);
}

// 8 f32 values as bf16: part 0 the rounded values (hi), part 1 the rounded remainders x - hi (lo)
__device__ __forceinline__ q35_u32x4 bf16_part8(const float (&x)[8], int part) {
    q35_u32x4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t hi = f2bf2(x[2 * w], x[2 * w + 1]);
        r[w] = part ? f2bf2(x[2 * w] - __uint_as_float(hi << 16), x[2 * w + 1] - __uint_as_float(hi & 0xffff0000u)) : hi;
    }
    return r;
}
__device__ __forceinline__ q35_f32x4 mfma_bf16(q35_u32x4 av, q35_u32x4 bv, q35_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(q35_bf16x8*)&av, *(q35_bf16x8*)&bv, c, 0, 0, 0);
}

constexpr int kConvRows = 16;

__global__ void __launch_bounds__(256) gdn_chunk_conv(GdnArgs a) {
    const int ch = blockIdx.y * 256 + threadIdx.x;       // 0..6143: q | k | v channels
    const int t0 = blockIdx.x * kConvRows;
    const int n = min(kConvRows, a.T - t0);
    const int lane = a.lane[0];
    const int cur = a.cur ? a.cur[0] : 0;
    const int wcur = a.wcur ? a.wcur[0] : cur;
    const float* Win = a.win + lane * a.W_lane + a.W_layer + wcur * a.W_slot;
    const uint2 cpk = *(const uint2*)(a.conv_w + (size_t)ch * 4);
    const float cw0 = __uint_as_float(cpk.x << 16), cw1 = __uint_as_float(cpk.x & 0xffff0000u);
    const float cw2 = __uint_as_float(cpk.y << 16), cw3 = __uint_as_float(cpk.y & 0xffff0000u);
    // raw rows t0-3 .. t0-1: earlier rows of the wave, or the lane's window before it
    auto raw = [&](int t) -> float {
        return t >= 0 ? bf2f(a.proj[(size_t)t * kGdnInRows + ch]) : Win[(t + 3) * 6144 + ch];
    };
    float w0 = raw(t0 - 3), w1 = raw(t0 - 2), w2 = raw(t0 - 1);
    uint16_t xr[kConvRows];
#pragma unroll
    for (int i = 0; i < kConvRows; ++i) xr[i] = a.proj[(size_t)min(t0 + i, a.T - 1) * kGdnInRows + ch];
    uint16_t* u = a.conv_u + (size_t)t0 * 6144 + ch;
#pragma unroll
    for (int i = 0; i < kConvRows; ++i) {
        if (i < n) {
            const float x = bf2f(xr[i]);
            float v = 0.f;
            v = v + w0 * cw0; v = v + w1 * cw1; v = v + w2 * cw2; v = v + x * cw3;
            u[(size_t)i * 6144] = f2bf(silu_f(rbf(v)));
            w0 = w1; w1 = w2; w2 = x;
        }
    }
    if (t0 + kConvRows >= a.T) {      // the run holding the wave's last row: window after the wave
        float* Wo = a.win + lane * a.W_lane + a.W_layer + ((wcur + 1) % a.nslots) * a.W_slot;
        Wo[ch] = w0; Wo[6144 + ch] = w1; Wo[12288 + ch] = w2;
    }
}

__global__ void __launch_bounds__(256) gdn_chunk_prep(GdnArgs a) {
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int t0 = c * kC;
    const int nrow = min(kC, a.T - t0);

    __shared__ float qn[kC][129], kn[kC][129], vv[kC][129];
    __shared__ float ut[kC][kC + 1], intra_s[kC][kC + 1];
    __shared__ float gl[kC], bl[kC], cum[kC], ecum[kC];

    // ---- post-conv SiLU values (gdn_chunk_conv) of the head's q, k and v channels as 16-byte
    // runs: 64 rows x 48 runs of 8 channels, 12 per thread; rows past the wave are zero
    {
        q35_u32x4 xr[12];
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int id = tid + 256 * k, row = id / 48, cc = id % 48;
            const int ch = (cc >> 4) * 2048 + h * 128 + (cc & 15) * 8;
            xr[k] = *(const q35_u32x4*)(a.conv_u + (size_t)min(t0 + row, a.T - 1) * 6144 + ch);
        }
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int id = tid + 256 * k, row = id / 48, cc = id % 48;
            float(*dst)[129] = cc < 16 ? qn : cc < 32 ? kn : vv;
            const int d0 = (cc & 15) * 8;
            const bool ok = row < nrow;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dst[row][d0 + 2 * e] = ok ? __uint_as_float(xr[k][e] << 16) : 0.f;
                dst[row][d0 + 2 * e + 1] = ok ? __uint_as_float(xr[k][e] & 0xffff0000u) : 0.f;
            }
        }
    }
    // ---- gates (rows past the wave: g = 0, beta = 0)
    if (tid < kC) {
        float g = 0.f, beta = 0.f;
        if (tid < nrow) {
            const uint16_t* pr = a.proj + (size_t)(t0 + tid) * kGdnInRows;
            const float bb = bf2f(pr[kGdnBOff + h]);
            const float aa = bf2f(pr[kGdnAOff + h]) + bf2f(a.dt_bias[h]);
            const float A = -expf(bf2f(a.A_log[h]));
            const float sp = aa > 20.f ? aa : log1pf(expf(aa));
            g = A * sp;
            beta = sigmoid_f(bb);
        }
        gl[tid] = g;
        bl[tid] = beta;
    }
    __syncthreads();
    // ---- L2 norms: wave w takes rows w, w + 4, ...; the recurrent kernel's reduction tree
    {
        const int wv = tid >> 6, ln = tid & 63;
        for (int i = wv; i < kC; i += 4) {
            const float q0 = qn[i][ln], q1 = qn[i][ln + 64], k0 = kn[i][ln], k1 = kn[i][ln + 64];
            const float rq = rsqrtf((wave_sum(q0 * q0) + wave_sum(q1 * q1)) + 1e-6f);
            const float rk = rsqrtf((wave_sum(k0 * k0) + wave_sum(k1 * k1)) + 1e-6f);
            qn[i][ln] = __fmul_rn(__fmul_rn(q0, rq), 0.08838834764831845f);
            qn[i][ln + 64] = __fmul_rn(__fmul_rn(q1, rq), 0.08838834764831845f);
            kn[i][ln] = __fmul_rn(k0, rk);
            kn[i][ln + 64] = __fmul_rn(k1, rk);
        }
        if (tid == 0) {       // cum_i = g_0 + .. + g_i, in order
            float gv[kC];
#pragma unroll
            for (int i = 0; i < kC; ++i) gv[i] = gl[i];
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < kC; ++i) { s += gv[i]; cum[i] = s; }
        }
    }
    __syncthreads();
    if (tid < kC) ecum[tid] = expf(cum[tid]);
    // ---- ut (strictly lower) and intra (lower) on MFMA: the 10 (row tile, column tile <= row
    // tile) pairs dealt round-robin to the 4 waves (3, 3, 2, 2 each: row tile w against its
    // w + 1 column tiles would give wave 3 four); A = k~ (ut) or q~ (intra) rows, B = k~^T
    float* ws = a.chunk_ws + ((size_t)c * kHv + h) * kCWs;
    {
        const int wv = tid >> 6, ln = tid & 63, mr = ln & 15, kq = ln >> 4;
        for (int pi = wv; pi < 10; pi += 4) {
            const int rt = pi < 1 ? 0 : pi < 3 ? 1 : pi < 6 ? 2 : 3;        // pair pi = (rt, nt)
            const int nt = pi - rt * (rt + 1) / 2;
            q35_f32x4 au = {0.f, 0.f, 0.f, 0.f}, ai = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
            for (int ks = 0; ks < 32; ++ks) {
                const float bk = kn[nt * 16 + mr][ks * 4 + kq];
                au = mfma4(kn[rt * 16 + mr][ks * 4 + kq], bk, au);
                ai = mfma4(qn[rt * 16 + mr][ks * 4 + kq], bk, ai);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = rt * 16 + 4 * kq + r, j = nt * 16 + mr;
                const float pair = j <= i ? expf(cum[i] - cum[j]) : 0.f;
                ut[i][j] = j < i ? (au[r] * bl[i]) * pair : 0.f;     // (beta_i k~_i) . k~_j, decayed
                intra_s[i][j] = ai[r] * pair;
            }
        }
        for (int nt = wv + 1; nt < 4; ++nt)       // upper tiles: zero
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = wv * 16 + 4 * kq + r, j = nt * 16 + mr;
                ut[i][j] = 0.f;
                intra_s[i][j] = 0.f;
            }
    }
    __syncthreads();
    // ---- q' = q~ e^cum and k' = k~ e^(cum_63 - cum) in operand order (before the solve reuses qn).
    // The workspace is written as whole 16-byte vectors, consecutive threads on consecutive
    // vectors: each thread gathers the vector's 4 elements from LDS.
    if (tid < kC) ut[tid][kC] = expf(cum[kC - 1] - cum[tid]);      // e^(cum_63 - cum_i), column kC spare
    __syncthreads();
    {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int u = tid + 256 * k;
            // q' = q~ e^cum as bf16 hi / lo: vector u = (w, kb, part, lane)
            {
                const int ln = u & 63, part = (u >> 6) & 1, kb = (u >> 7) & 3, w = u >> 9;
                const int i = 16 * w + (ln & 15), k0 = 32 * kb + 8 * (ln >> 4);
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = qn[i][k0 + e] * ecum[i];
                *(q35_u32x4*)((uint16_t*)(ws + kWsQ) + 8 * u) = bf16_part8(x, part);
            }
            // k'^T: A[m = d][kk = i] -> [d / 16][lane (i % 4, d % 16)][i / 4]; vector u = (lane slot, i/4 quad)
            {
                const int q = u & 3, ln = (u >> 2) & 63, d = (u >> 8) * 16 + (ln & 15), iq = ln >> 4;
                float4 v;
                const int i0 = 16 * q + iq;
                v.x = kn[i0][d] * ut[i0][kC];
                v.y = kn[i0 + 4][d] * ut[i0 + 4][kC];
                v.z = kn[i0 + 8][d] * ut[i0 + 8][kC];
                v.w = kn[i0 + 12][d] * ut[i0 + 12][kC];
                *(float4*)&ws[kWsK + 4 * u] = v;
            }
        }
        // intra as bf16 hi / lo: vector u = (w, kb, part, lane)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int u = tid + 256 * k;
            const int ln = u & 63, part = (u >> 6) & 1, kb = (u >> 7) & 1, w = u >> 8;
            const int i = 16 * w + (ln & 15), j0 = 32 * kb + 8 * (ln >> 4);
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = intra_s[i][j0 + e];
            *(q35_u32x4*)((uint16_t*)(ws + kWsIntra) + 8 * u) = bf16_part8(x, part);
        }
        if (tid == 0) a.chunk_cdec[c * kHv + h] = expf(cum[kC - 1]);
    }
    __syncthreads();
    // ---- (I + ut) X = R for R = beta v (X in vv) and R = beta k~ e^cum (X in qn), blocked by
    // 16 rows: R_b -= ut[b, <b] X[<b] on MFMA (wave w: 4 of the 16 column tiles of [vv | qn]),
    // then the 16-row unit-lower solve of block b, one column per thread, in registers
    {
        for (int e = tid; e < kC * 128; e += 256) {
            const int i = e >> 7, d = e & 127;
            vv[i][d] = vv[i][d] * bl[i];
            qn[i][d] = (kn[i][d] * bl[i]) * ecum[i];
        }
        const int wv = tid >> 6, ln = tid & 63, mr = ln & 15, kq = ln >> 4;
        const int col = tid & 127;
        const bool isk = tid >= 128;
        for (int bb = 0; bb < 4; ++bb) {
            __syncthreads();
            if (bb > 0) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int ntile = wv * 4 + t;                  // 0..7 -> vv, 8..15 -> qn
                    float(*Xt)[129] = ntile < 8 ? vv : qn;
                    const int n = (ntile & 7) * 16 + mr;
                    q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    for (int ks = 0; ks < bb * 4; ++ks)
                        acc = mfma4(ut[bb * 16 + mr][ks * 4 + kq], Xt[ks * 4 + kq][n], acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) Xt[bb * 16 + 4 * kq + r][n] -= acc[r];
                }
                __syncthreads();
            }
            float(*X)[129] = isk ? qn : vv;
            float x[16];
#pragma unroll
            for (int ii = 0; ii < 16; ++ii) x[ii] = X[bb * 16 + ii][col];
#pragma unroll
            for (int ii = 1; ii < 16; ++ii)
#pragma unroll
                for (int jj = 0; jj < ii; ++jj) x[ii] = fmaf(-ut[bb * 16 + ii][bb * 16 + jj], x[jj], x[ii]);
#pragma unroll
            for (int ii = 0; ii < 16; ++ii) X[bb * 16 + ii][col] = x[ii];
        }
        __syncthreads();
        // 16-byte vectors gathered from LDS, consecutive threads on consecutive vectors
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int u = tid + 256 * k;
            {   // kcd: A[m = i][k = col] -> [i / 16][lane (col % 4, i % 16)][col / 4]
                const int q = u & 7, ln = (u >> 3) & 63, i = (u >> 9) * 16 + (ln & 15), cq = ln >> 4;
                float4 v;
                v.x = qn[i][16 * q + cq];
                v.y = qn[i][16 * q + 4 + cq];
                v.z = qn[i][16 * q + 8 + cq];
                v.w = qn[i][16 * q + 12 + cq];
                *(float4*)&ws[kWsKcd + 4 * u] = v;
            }
            {   // nv: C layout of slice col / 16 -> [slice][i / 16][lane ((i % 16) / 4, col % 16)][i % 4]
                const int ln = u & 63, ib = (u >> 6) & 3, sl = u >> 8;
                const int i0 = ib * 16 + (ln >> 4) * 4, cl = sl * 16 + (ln & 15);
                float4 v;
                v.x = vv[i0][cl];
                v.y = vv[i0 + 1][cl];
                v.z = vv[i0 + 2][cl];
                v.w = vv[i0 + 3][cl];
                *(float4*)&ws[kWsNv + 4 * u] = v;
            }
        }
    }
}

__global__ void __launch_bounds__(256) gdn_chunk_scan(GdnArgs a, int nchunks) {
    const int h = blockIdx.x, n0 = blockIdx.y * 16;
    const int tid = threadIdx.x, ln = tid & 63, wv = tid >> 6;
    const int lane = a.lane[0];
    const int cur = a.cur ? a.cur[0] : 0;
    float* Sbase = a.S + lane * a.S_lane + a.S_layer + (long long)h * 16384;
    const float* Sin = Sbase + cur * a.S_slot;
    float* Sout = Sbase + ((cur + 1) % a.nslots) * a.S_slot;

    __shared__ float S[128][16];
    __shared__ float vn[kC][16];
    for (int e = tid; e < 128 * 16; e += 256) S[e >> 4][e & 15] = Sin[(e >> 4) * 128 + n0 + (e & 15)];
    __syncthreads();

    const int mr = ln & 15, kq = ln >> 4;          // A row / k-quad of this lane
    // this wave's A operands of one chunk, in registers: kcd rows 16w + mr (k = 4ks + kq), k'^T
    // rows 32w + 16 half + mr (i = 4ks + kq), and nv (16-byte vectors loaded straight into the
    // set: no copy waits for the data before its use)
    struct Ops { q35_f32x4 kcd[8], kp[2][4], nv; float cd; };
    auto load_ops = [&](int c, Ops& o) {
        const float* ws = a.chunk_ws + ((size_t)c * kHv + h) * kCWs;
        o.cd = a.chunk_cdec[c * kHv + h];
        const q35_f32x4* pk = (const q35_f32x4*)(ws + kWsKcd + (wv * 64 + ln) * 32);
        const q35_f32x4* pp0 = (const q35_f32x4*)(ws + kWsK + ((wv * 2 + 0) * 64 + ln) * 16);
        const q35_f32x4* pp1 = (const q35_f32x4*)(ws + kWsK + ((wv * 2 + 1) * 64 + ln) * 16);
        o.nv = *(const q35_f32x4*)(ws + kWsNv + ((blockIdx.y * 4 + wv) * 64 + ln) * 4);
#pragma unroll
        for (int v = 0; v < 8; ++v) o.kcd[v] = pk[v];
#pragma unroll
        for (int v = 0; v < 4; ++v) { o.kp[0][v] = pp0[v]; o.kp[1][v] = pp1[v]; }
    };
    // a ring of three operand sets: chunk c's loads are issued two chunks ahead (one chunk of
    // compute does not cover the workspace's load latency); the ring index is static (the
    // chunk loop is unrolled by 3)
    Ops ops[3];
    load_ops(0, ops[0]);
    load_ops(min(1, nchunks - 1), ops[1]);
    auto step = [&](int c, auto par) {
        constexpr int P = decltype(par)::value;
        Ops& cur_ops = ops[P];
        // operands two chunks ahead (unconditional, clamped: no branch splits the wait counts)
        load_ops(min(c + 2, nchunks - 1), ops[(P + 2) % 3]);
        // B fragments of S for phase 1 (all waves read S before the barrier)
        float sf[32];
#pragma unroll
        for (int ks = 0; ks < 32; ++ks) sf[ks] = S[ks * 4 + kq][mr];
        // this chunk's S as gdn_chunk_out's B fragments (16x16x32 layout: k = 32 kb + 8 kq + e,
        // column mr; wave w writes k-block w), bf16 hi / lo pairs
        q35_u32x4* wsc = (q35_u32x4*)(a.chunk_ws + ((size_t)c * kHv + h) * kCWs);
        {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = S[32 * wv + 8 * kq + e][mr];
            wsc[kWsSb / 4 + ((blockIdx.y * 4 + wv) * 2 + 0) * 64 + ln] = bf16_part8(x, 0);
            wsc[kWsSb / 4 + ((blockIdx.y * 4 + wv) * 2 + 1) * 64 + ln] = bf16_part8(x, 1);
        }
        // phase 1: v_new = nv - kcd S   (wave w: rows 16w .. 16w+15)
        {
            q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 32; ++ks) acc = mfma4(cur_ops.kcd[ks >> 2][ks & 3], sf[ks], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) vn[wv * 16 + 4 * kq + r][mr] = cur_ops.nv[r] - acc[r];
        }
        __syncthreads();
        float vf[16];       // B fragments of v_new for phase 3
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) vf[ks] = vn[ks * 4 + kq][mr];
        // v_new as gdn_chunk_out's B fragments (waves 0, 1: k-block w), bf16 hi / lo pairs
        if (wv < 2) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = vn[32 * wv + 8 * kq + e][mr];
            wsc[kWsVb / 4 + ((blockIdx.y * 2 + wv) * 2 + 0) * 64 + ln] = bf16_part8(x, 0);
            wsc[kWsVb / 4 + ((blockIdx.y * 2 + wv) * 2 + 1) * 64 + ln] = bf16_part8(x, 1);
        }
        // phase 3: S = e^cum_63 S + k'^T v_new   (wave w: its own state rows 32w .. 32w+31;
        // no other wave reads S after the barrier above)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int m0 = wv * 32 + half * 16;
            q35_f32x4 acc;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = S[m0 + 4 * kq + r][mr] * cur_ops.cd;
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) acc = mfma4(cur_ops.kp[half][ks >> 2][ks & 3], vf[ks], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) S[m0 + 4 * kq + r][mr] = acc[r];
        }
        __syncthreads();    // S complete and v_new consumed before the next chunk
    };
    for (int c = 0; c < nchunks; c += 3) {
        step(c, std::integral_constant<int, 0>{});
        if (c + 1 < nchunks) step(c + 1, std::integral_constant<int, 1>{});
        if (c + 2 < nchunks) step(c + 2, std::integral_constant<int, 2>{});
    }
    for (int e = tid; e < 128 * 16; e += 256) Sout[(e >> 4) * 128 + n0 + (e & 15)] = S[e >> 4][e & 15];
}

// o = q' S + intra v_new of chunk blockIdx.x, head blockIdx.y: wave w takes row tile w (rows 16w
// .. 16w + 15) over the 8 column slices; its A fragments (q' and intra hi / lo) are loaded once,
// the slices' B fragments one slice ahead. With a.y the block holds the head's whole rows, so it
// applies the gated RMSNorm itself and stores y (bf16, tiled with a.y_tiled) instead of o.
__global__ void __launch_bounds__(256) gdn_chunk_out(GdnArgs a) {
    __shared__ float ot[kC][129];                // with y: the chunk's o of this head
    __shared__ float ssl[kC][2];                 // and its rows' half-head sums of squares
    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, ln = tid & 63, wv = tid >> 6, mr = ln & 15, kq = ln >> 4;
    const q35_u32x4* ws = (const q35_u32x4*)(a.chunk_ws + ((size_t)c * kHv + h) * kCWs);
    q35_u32x4 aq[8], ai[4];
#pragma unroll
    for (int v = 0; v < 8; ++v) aq[v] = ws[kWsQ / 4 + (wv * 8 + v) * 64 + ln];      // [kb][part]
#pragma unroll
    for (int v = 0; v < 4; ++v) ai[v] = ws[kWsIntra / 4 + (wv * 4 + v) * 64 + ln];
    q35_u32x4 sb[2][8], vb[2][4];                // [slice parity][kb][part]
    auto load_b = [&](int sl, q35_u32x4 (&s8)[8], q35_u32x4 (&v4)[4]) {
#pragma unroll
        for (int v = 0; v < 8; ++v) s8[v] = ws[kWsSb / 4 + (sl * 8 + v) * 64 + ln];
#pragma unroll
        for (int v = 0; v < 4; ++v) v4[v] = ws[kWsVb / 4 + (sl * 4 + v) * 64 + ln];
    };
    load_b(0, sb[0], vb[0]);
    const int t0 = c * kC;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        const int b = sl & 1;
        if (sl + 1 < 8) load_b(sl + 1, sb[b ^ 1], vb[b ^ 1]);
        q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            acc = mfma_bf16(aq[2 * kb], sb[b][2 * kb], acc);
            acc = mfma_bf16(aq[2 * kb], sb[b][2 * kb + 1], acc);
            acc = mfma_bf16(aq[2 * kb + 1], sb[b][2 * kb], acc);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            acc = mfma_bf16(ai[2 * kb], vb[b][2 * kb], acc);
            acc = mfma_bf16(ai[2 * kb], vb[b][2 * kb + 1], acc);
            acc = mfma_bf16(ai[2 * kb + 1], vb[b][2 * kb], acc);
        }
        if (a.y) {
#pragma unroll
            for (int r = 0; r < 4; ++r) ot[wv * 16 + 4 * kq + r][sl * 16 + mr] = acc[r];
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wv * 16 + 4 * kq + r;
                if (t0 + row < a.T) a.o[(size_t)(t0 + row) * 2048 + h * 128 + sl * 16 + mr] = acc[r];
            }
        }
    }
    if (!a.y) return;
    // the gated RMSNorm of the out_proj producer (same reduction order and arithmetic): thread
    // (row, half) sums the half head's 64 squares, then 8-column pieces are gated and stored
    __syncthreads();
    if (tid < 128) {
        float v[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) v[i] = ot[tid >> 1][(tid & 1) * 64 + i];
        ssl[tid >> 1][tid & 1] = half_head_ss_regs(v);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int u = tid + 256 * k;
        const int row = (u >> 8) * 16 + (u & 15), ch = (u >> 4) & 15;    // the tile's 16 rows adjacent
        const int m = t0 + row;
        if (m >= a.T) continue;
        const float rs = head_rsqrt(ssl[row][0], ssl[row][1]);
        float ov[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ov[e] = ot[row][ch * 8 + e];
        const q35_u32x4 zz = *(const q35_u32x4*)(a.proj + (size_t)m * kGdnInRows + kGdnZOff + h * 128 + ch * 8);
        const q35_u32x4 ww = *(const q35_u32x4*)(a.gnorm + ch * 8);
        const int col = h * 128 + ch * 8;
        *(q35_u32x4*)(a.y + (a.y_tiled ? tiled_offset(m, col, 2048) : (size_t)m * 2048 + col)) = gated8(ov, zz, ww, rs);
    }
}

hipError_t launch_gdn_chunked(const GdnArgs& a, hipStream_t st) {
    if (a.nlanes != 1 || a.T < 1 || a.ckpt || !a.chunk_ws || !a.chunk_cdec) return hipErrorInvalidValue;
    const int nchunks = (a.T + kC - 1) / kC;
    if (!a.conv_u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_chunk_conv, dim3((a.T + kConvRows - 1) / kConvRows, 6144 / 256), dim3(256), 0, st, a);
    hipLaunchKernelGGL(gdn_chunk_prep, dim3(nchunks, kHv), dim3(256), 0, st, a);
    hipLaunchKernelGGL(gdn_chunk_scan, dim3(kHv, 8), dim3(256), 0, st, a, nchunks);
    hipLaunchKernelGGL(gdn_chunk_out, dim3(nchunks, kHv), dim3(256), 0, st, a);
    return hipGetLastError();
}

size_t gdn_chunk_ws_floats(int max_rows) { return (size_t)((max_rows + kC - 1) / kC) * kHv * kCWs; }

}  // namespace q35
