// GatedDeltaNet over a prompt wave of one lane in the chunked (UT-transform) form, chunk 64
// (speccheck/specimpl.py:187-235; the reference engine's gdn_chunk_prefill,
// engine/kernels_gdn.cpp:488). Two kernels:
//
//   gdn_chunk_prep  grid (chunk, head): causal conv + bf16 SiLU, L2 norms and gates with the
//                   recurrent kernel's arithmetic; then, within the chunk, the decay prefix
//                   cum_i = g_0 + .. + g_i, the pairwise-decayed products
//                   ut = (beta k~) k~^T (strictly lower) and intra = q~ k~^T (lower), the two
//                   unit-lower-triangular solves (I + ut) nv = beta v and
//                   (I + ut) kcd = beta k~ e^cum, and q' = q~ e^cum, k' = k~ e^(cum_63 - cum).
//                   Rows past the wave are zero with g = beta = 0, as the reference pads.
//   gdn_chunk_scan  grid (head, 16-column slice): the chunk recurrence, sequential over chunks
//                   with the slice S[:, n0 .. n0+16) of the f32 state in LDS:
//                     v_new = nv - kcd S;  o = q' S + intra v_new;  S = e^cum_63 S + k'^T v_new
//                   on v_mfma_f32_16x16x4_f32 (f32 products, f32 accumulate). The value columns
//                   of the delta rule never mix, so 8 slices per head run independently.
//
// The state is read from slot cur and written to slot (cur + 1) % nslots, the conv window
// likewise, exactly as the recurrent kernel does for a wave without checkpoints.
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

constexpr int kC = 64;                      // chunk rows
constexpr int kCWs = 4 * kC * 128 + kC * kC; // workspace floats per (chunk, head)
// workspace layout per (chunk, head): q' | k' | nv | kcd  ([64][128] each), intra [64][64]
constexpr int kWsQ = 0, kWsK = kC * 128, kWsNv = 2 * kC * 128, kWsKcd = 3 * kC * 128, kWsIntra = 4 * kC * 128;

__global__ void __launch_bounds__(256) gdn_chunk_prep(GdnArgs a) {
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int t0 = c * kC;
    const int nrow = min(kC, a.T - t0);
    const int lane = a.lane[0];
    const int cur = a.cur ? a.cur[lane] : 0;
    const float* Win = a.win + lane * a.W_lane + a.W_layer + cur * a.W_slot;

    __shared__ float qn[kC][129], kn[kC][129], vv[kC][129];
    __shared__ float ut[kC][kC + 1];
    __shared__ float gl[kC], bl[kC], cum[kC], ecum[kC];

    // ---- causal conv + SiLU: tid < 128 -> q channel (and v channel), else k channel
    {
        const int cqk = tid < 128 ? h * 128 + tid : 2048 + h * 128 + (tid - 128);
        const int cv = 4096 + h * 128 + tid;
        const bool hasv = tid < 128;
        const uint2 cpk = *(const uint2*)(a.conv_w + (size_t)cqk * 4);
        const float cw0 = __uint_as_float(cpk.x << 16), cw1 = __uint_as_float(cpk.x & 0xffff0000u);
        const float cw2 = __uint_as_float(cpk.y << 16), cw3 = __uint_as_float(cpk.y & 0xffff0000u);
        float vw0 = 0.f, vw1 = 0.f, vw2 = 0.f, vw3 = 0.f;
        if (hasv) {
            const uint2 d = *(const uint2*)(a.conv_w + (size_t)cv * 4);
            vw0 = __uint_as_float(d.x << 16); vw1 = __uint_as_float(d.x & 0xffff0000u);
            vw2 = __uint_as_float(d.y << 16); vw3 = __uint_as_float(d.y & 0xffff0000u);
        }
        // raw rows t0-3 .. t0-1: earlier rows of the wave, or the lane's window before it
        auto raw = [&](int t, int ch) -> float {
            return t >= 0 ? bf2f(a.proj[(size_t)t * kGdnInRows + ch]) : Win[(t + 3) * 6144 + ch];
        };
        float w0 = raw(t0 - 3, cqk), w1 = raw(t0 - 2, cqk), w2 = raw(t0 - 1, cqk);
        float v0 = 0.f, v1 = 0.f, v2 = 0.f;
        if (hasv) { v0 = raw(t0 - 3, cv); v1 = raw(t0 - 2, cv); v2 = raw(t0 - 1, cv); }
        for (int i = 0; i < kC; ++i) {
            float uq = 0.f, uvv = 0.f;
            if (i < nrow) {
                const uint16_t* pr = a.proj + (size_t)(t0 + i) * kGdnInRows;
                const float x = bf2f(pr[cqk]);
                float u = 0.f;
                u = u + w0 * cw0; u = u + w1 * cw1; u = u + w2 * cw2; u = u + x * cw3;
                uq = rbf(silu_f(rbf(u)));
                w0 = w1; w1 = w2; w2 = x;
                if (hasv) {
                    const float xv = bf2f(pr[cv]);
                    float uv = 0.f;
                    uv = uv + v0 * vw0; uv = uv + v1 * vw1; uv = uv + v2 * vw2; uv = uv + xv * vw3;
                    uvv = rbf(silu_f(rbf(uv)));
                    v0 = v1; v1 = v2; v2 = xv;
                }
            }
            if (tid < 128) qn[i][tid] = uq; else kn[i][tid - 128] = uq;
            if (hasv) vv[i][tid] = uvv;
        }
        // the chunk holding the wave's last row writes the window after the wave
        if (t0 + kC >= a.T) {
            float* Wo = a.win + lane * a.W_lane + a.W_layer + ((cur + 1) % a.nslots) * a.W_slot;
            Wo[cqk] = w0; Wo[6144 + cqk] = w1; Wo[12288 + cqk] = w2;
            if (hasv) { Wo[cv] = v0; Wo[6144 + cv] = v1; Wo[12288 + cv] = v2; }
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
        if (tid == 0) {
            float s = 0.f;
            for (int i = 0; i < kC; ++i) { s += gl[i]; cum[i] = s; }
        }
    }
    __syncthreads();
    if (tid < kC) ecum[tid] = expf(cum[tid]);
    // ---- ut (strictly lower) and intra (lower): thread -> row i = tid / 4, columns j = 16 (tid % 4) ..
    {
        const int i = tid >> 2, j0 = (tid & 3) * 16;
        float du[16], di[16];
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) { du[jj] = 0.f; di[jj] = 0.f; }
        for (int d0 = 0; d0 < 128; d0 += 16) {
            float kq[16], qq[16];
#pragma unroll
            for (int d = 0; d < 16; ++d) { kq[d] = kn[i][d0 + d]; qq[d] = qn[i][d0 + d]; }
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                float su = du[jj], si = di[jj];
#pragma unroll
                for (int d = 0; d < 16; ++d) {
                    const float kj = kn[j0 + jj][d0 + d];
                    su = fmaf(kq[d], kj, su);
                    si = fmaf(qq[d], kj, si);
                }
                du[jj] = su;
                di[jj] = si;
            }
        }
        const float bi = bl[i], ci = cum[i];
        float* intra = a.chunk_ws + ((size_t)c * kHv + h) * kCWs + kWsIntra;
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const int j = j0 + jj;
            const float pair = j <= i ? expf(ci - cum[j]) : 0.f;
            ut[i][j] = j < i ? (du[jj] * bi) * pair : 0.f;       // (beta_i k~_i) . k~_j, decayed
            intra[i * kC + j] = di[jj] * pair;
        }
    }
    __syncthreads();
    // ---- q' = q~ e^cum, k' = k~ e^(cum_63 - cum) (before the solve reuses qn)
    float* ws = a.chunk_ws + ((size_t)c * kHv + h) * kCWs;
    {
        const float clast = cum[kC - 1];
        for (int e = tid; e < kC * 128; e += 256) {
            const int i = e >> 7, d = e & 127;
            ws[kWsQ + e] = qn[i][d] * ecum[i];
            ws[kWsK + e] = kn[i][d] * expf(clast - cum[i]);
        }
        if (tid == 0) a.chunk_cdec[c * kHv + h] = expf(clast);
    }
    __syncthreads();
    // ---- forward substitution in place, one column per thread: tid < 128 -> nv (in vv),
    // else kcd (in qn, right-hand side beta k~ e^cum)
    {
        const int col = tid & 127;
        const bool isk = tid >= 128;
        float(*X)[129] = isk ? qn : vv;
        for (int i = 0; i < kC; ++i) {
            float acc = isk ? (kn[i][col] * bl[i]) * ecum[i] : vv[i][col] * bl[i];
#pragma unroll 4
            for (int j = 0; j < i; ++j) acc = fmaf(-ut[i][j], X[j][col], acc);
            X[i][col] = acc;
        }
        float* dst = ws + (isk ? kWsKcd : kWsNv);
        for (int i = 0; i < kC; ++i) dst[i * 128 + col] = X[i][col];
    }
}

// MFMA f32 16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
// D[4 (l/16) + r][l%16], r = 0..3.
__device__ __forceinline__ q35_f32x4 mfma4(float av, float bv, q35_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, c, 0, 0, 0);
}

__global__ void __launch_bounds__(256) gdn_chunk_scan(GdnArgs a, int nchunks) {
    const int h = blockIdx.x, n0 = blockIdx.y * 16;
    const int tid = threadIdx.x, ln = tid & 63, wv = tid >> 6;
    const int lane = a.lane[0];
    const int cur = a.cur ? a.cur[lane] : 0;
    float* Sbase = a.S + lane * a.S_lane + a.S_layer + (long long)h * 16384;
    const float* Sin = Sbase + cur * a.S_slot;
    float* Sout = Sbase + ((cur + 1) % a.nslots) * a.S_slot;

    __shared__ float S[128][16];
    __shared__ float vn[kC][16];
    for (int e = tid; e < 128 * 16; e += 256) S[e >> 4][e & 15] = Sin[(e >> 4) * 128 + n0 + (e & 15)];
    __syncthreads();

    const int mr = ln & 15, kq = ln >> 4;          // A row / k-quad of this lane
    for (int c = 0; c < nchunks; ++c) {
        const float* ws = a.chunk_ws + ((size_t)c * kHv + h) * kCWs;
        const int t0 = c * kC;
        // phase 1: v_new = nv - kcd S   (wave w: rows 16w .. 16w+15)
        {
            q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const float* kcd = ws + kWsKcd + (wv * 16 + mr) * 128;
#pragma unroll 8
            for (int ks = 0; ks < 32; ++ks) acc = mfma4(kcd[ks * 4 + kq], S[ks * 4 + kq][mr], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wv * 16 + 4 * kq + r;
                vn[row][mr] = ws[kWsNv + row * 128 + n0 + mr] - acc[r];
            }
        }
        __syncthreads();
        // phase 2: o = q' S + intra v_new
        {
            q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const float* qp = ws + kWsQ + (wv * 16 + mr) * 128;
#pragma unroll 8
            for (int ks = 0; ks < 32; ++ks) acc = mfma4(qp[ks * 4 + kq], S[ks * 4 + kq][mr], acc);
            const float* in = ws + kWsIntra + (wv * 16 + mr) * kC;
#pragma unroll 8
            for (int ks = 0; ks < 16; ++ks) acc = mfma4(in[ks * 4 + kq], vn[ks * 4 + kq][mr], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wv * 16 + 4 * kq + r;
                if (t0 + row < a.T) a.o[(size_t)(t0 + row) * 2048 + h * 128 + n0 + mr] = acc[r];
            }
        }
        __syncthreads();
        // phase 3: S = e^cum_63 S + k'^T v_new   (wave w: state rows 32w .. 32w+31)
        {
            const float cd = a.chunk_cdec[c * kHv + h];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int m0 = wv * 32 + half * 16;
                q35_f32x4 acc;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] = S[m0 + 4 * kq + r][mr] * cd;
                const float* kp = ws + kWsK + m0 + mr;          // k'^T [m][i] = k'[i][m]
#pragma unroll 8
                for (int ks = 0; ks < 16; ++ks) acc = mfma4(kp[(ks * 4 + kq) * 128], vn[ks * 4 + kq][mr], acc);
#pragma unroll
                for (int r = 0; r < 4; ++r) S[m0 + 4 * kq + r][mr] = acc[r];
            }
        }
        __syncthreads();
    }
    for (int e = tid; e < 128 * 16; e += 256) Sout[(e >> 4) * 128 + n0 + (e & 15)] = S[e >> 4][e & 15];
}

hipError_t launch_gdn_chunked(const GdnArgs& a, hipStream_t st) {
    if (a.nlanes != 1 || a.T < 1 || a.ckpt || !a.chunk_ws || !a.chunk_cdec) return hipErrorInvalidValue;
    const int nchunks = (a.T + kC - 1) / kC;
    hipLaunchKernelGGL(gdn_chunk_prep, dim3(nchunks, kHv), dim3(256), 0, st, a);
    hipLaunchKernelGGL(gdn_chunk_scan, dim3(kHv, 8), dim3(256), 0, st, a, nchunks);
    return hipGetLastError();
}

size_t gdn_chunk_ws_floats(int max_rows) { return (size_t)((max_rows + kC - 1) / kC) * kHv * kCWs; }

}  // namespace q35
