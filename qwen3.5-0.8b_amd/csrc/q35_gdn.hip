// GatedDeltaNet mixer for R = nlanes x T rows: causal conv (kernel 4) + SiLU, gates,
// L2 norms and the delta-rule recurrence, with the fp32 state held in VGPRs across the
// T rows of a lane. Output o (f32, pre gated-norm); the gated RMSNorm is fused into the
// out_proj GEMM's A operand (q35_gemm.hip).
//
// Math (speccheck/specimpl.py:252-294): u = bf16silu(bf16(sum_j win[j] C[:,j])) over the
// pre-conv window (f32 taps in tap order), beta = sigmoid(b),
// g = -exp(A_log) softplus(a + dt_bias), q~ = q rsqrt(|q|^2+1e-6) 128^-1/2,
// k~ = k rsqrt(|k|^2+1e-6); S = e^g S; r = S^T k~; dv = beta (v - r); S += k~ dv^T;
// o = S^T q~. Replaces engine/kernels_gdn.cpp:35-536 (conv, gates, rec) of the reference.
//
// The state is never updated in place (the conv window's q/k channels are read by every
// column-slice block of a head): the state after the last row goes to slot (cur + 1) %
// nslots and the window to slot (wcur + 1) % nslots; with `ckpt` (MTP verify candidates) the
// window after every row t goes to slot (wcur + 1 + t) % nslots and each row's state update is
// recorded as factors (gamma, k~, dv) instead of a 1 MiB state per row (GdnArgs: replaying
// them gives the same bits), so a rollback to row a is "slot cur plus pending rows 0..a".
// A decode step with `defer` records a lane's row the same way (row n of the set being read,
// when fewer than `defer` rows are pending) and leaves slot cur as it is, so the 1 MiB state
// of a lane is written once every defer + 1 steps and read every step.
// The engine advances the slots after the step.
//
// Grid: (lane group, head, column slice). A block owns VC = 128/CS value columns of one
// head and wave w owns VC/4 of them over all 128 k rows: lane (kg, column group) holds
// S[kg*KR .. kg*KR+KR) of CW adjacent columns in registers (CW = 4 when a block owns the
// whole head: 16-byte state loads and stores). The delta rule's value columns are
// independent, so the reductions over k stay inside a wave (its own columns of red_r /
// red_o, no barrier); a row needs one block barrier (after the conv phase: q~, k~, v and the
// gates are read by every wave), plus one for the fused gated norm. The conv outputs, norms
// and gates are double-buffered by row parity, so row t + 1's conv phase cannot overwrite
// what a slower wave still reads of row t.
#include "q35_common.h"
#include "q35_kernels.h"

namespace q35 {

template <int CS>
__global__ void __launch_bounds__(256) gdn_kernel(GdnArgs a) {
    constexpr int VC = 128 / CS;                 // value columns of this block
    constexpr int CW = CS == 1 ? 4 : 1;          // adjacent columns per lane (16-byte I/O)
    constexpr int WC = VC / 4;                   // value columns of a wave
    constexpr int CGW = WC / CW;                 // column groups of a wave
    constexpr int NKW = 64 / CGW;                // k-row groups of a wave
    constexpr int KR = 128 / NKW;                // k rows per lane (a multiple of 8)
    const int gi = blockIdx.x, h = blockIdx.y, cs = blockIdx.z;
    const int tid = threadIdx.x, lane64 = tid & 63, wv = tid >> 6;
    const int jc = wv * WC + (lane64 % CGW) * CW, kg = lane64 / CGW;
    const int cc = wv * WC + (lane64 % WC);      // CS = 1: the column a lane < 32 reduces
    // channels: tid < 128 -> q channel, else k channel; tid < VC also a v channel
    const int cqk = tid < 128 ? h * 128 + tid : 2048 + h * 128 + (tid - 128);
    const int cv = 4096 + h * 128 + cs * VC + tid;
    const bool hasv = tid < VC;
    const int cvc = hasv ? cv : cqk;                 // a valid channel for every thread
    // first, every load that does not depend on the row's lane and slots (one memory round
    // trip with the row metadata, instead of one more after the state): the first row's
    // projection inputs, the conv taps and the gate parameters, as raw bits
    const uint16_t* pr0 = a.proj + (size_t)(gi * a.T) * kGdnInRows;
    uint16_t xr = pr0[cqk], xvr = pr0[cvc];
    // raw b, a of row (tid mod 64) of the first 64-row chunk (the gates of a chunk's rows are made
    // at its start, one row per thread of wave 0)
    const uint16_t* pg = pr0 + (size_t)min(tid & 63, a.T - 1) * kGdnInRows;
    uint16_t gbr = pg[kGdnBOff + h], gar = pg[kGdnAOff + h];
    const uint2 cpk = *(const uint2*)(a.conv_w + (size_t)cqk * 4);
    const uint2 dpk = *(const uint2*)(a.conv_w + (size_t)cvc * 4);
    const uint16_t alogr = a.A_log[h], dtbr = a.dt_bias[h];
    const int lane = a.lane[gi * a.T];
    const int cur = a.cur ? a.cur[gi * a.T] : 0;
    const int wcur = a.wcur ? a.wcur[gi * a.T] : cur;
    const int pnd = a.pend ? a.pend[gi * a.T] : 0;
    const int npend = pnd & 15, pset = (pnd >> 4) & 1;
    const bool rec = !a.ckpt && npend < a.defer;    // this decode row becomes pending row npend

    __shared__ float qs[2][128], ks[2][128], vs[2][VC];   // by row parity
    __shared__ float wred[2][4];
    __shared__ float gate_c[2][64][2];               // (decay, beta) of a 64-row chunk's rows, by chunk parity
    constexpr int NG = 16;            // fixed reduction groups of 8 k-rows, for every CS
    constexpr int GPT = KR / 8;       // groups per lane
    __shared__ float red_r[NG][VC], red_o[NG][VC];
    __shared__ float qq[CS == 1 ? 32 : 1];           // CS = 1: the head's quads of o^2

    float* Sbase = a.S + lane * a.S_lane + a.S_layer + (long long)h * 16384;
    float* Wbase = a.win + lane * a.W_lane + a.W_layer;
    const float* Sin = Sbase + cur * a.S_slot;
    const float* Win = Wbase + wcur * a.W_slot;

    float w0 = Win[cqk], w1 = Win[6144 + cqk], w2 = Win[12288 + cqk];
    float v0 = Win[cvc], v1 = Win[6144 + cvc], v2 = Win[12288 + cvc];   // used by v channels only
    float s[KR][CW];
#pragma unroll
    for (int i = 0; i < KR; ++i) {
        const float* p = Sin + (kg * KR + i) * 128 + cs * VC + jc;
        if (CW == 4) {
            const q35_f32x4 v = __builtin_nontemporal_load((const q35_f32x4*)p);   // streamed once
            s[i][0] = v[0]; s[i][CW > 1 ? 1 : 0] = v[1]; s[i][CW > 2 ? 2 : 0] = v[2]; s[i][CW > 3 ? 3 : 0] = v[3];
        } else {
            s[i][0] = p[0];
        }
    }

    if (npend) {
        // the lane's pending rows, replayed with the recurrence's own rounded operations
        const float* F0 = a.fac + lane * a.fac_lane + pset * a.fac_set + h * kFacStride;
        for (int p = 0; p < npend; ++p) {
            const float* F = F0 + p * a.fac_row;
            const float gp = F[256];
            float kk[KR], dd[CW];
#pragma unroll
            for (int i = 0; i < KR; ++i) kk[i] = F[kg * KR + i];
#pragma unroll
            for (int c = 0; c < CW; ++c) dd[c] = F[128 + cs * VC + jc + c];
#pragma unroll
            for (int i = 0; i < KR; ++i)
#pragma unroll
                for (int c = 0; c < CW; ++c) {
                    s[i][c] = __fmul_rn(s[i][c], gp);
                    s[i][c] = delta_update(s[i][c], kk[i], dd[c]);
                }
        }
        if (a.ckpt && a.fac_write) {
            // the base of this verify's factors: slot cur + 1 (the engine moves `cur` there)
            float* So = Sbase + ((cur + 1) % a.nslots) * a.S_slot;
#pragma unroll
            for (int i = 0; i < KR; ++i) {
                float* p = So + (kg * KR + i) * 128 + cs * VC + jc;
                if (CW == 4)
                    __builtin_nontemporal_store((q35_f32x4){s[i][0], s[i][CW > 1 ? 1 : 0], s[i][CW > 2 ? 2 : 0], s[i][CW > 3 ? 3 : 0]},
                                                (q35_f32x4*)p);
                else p[0] = s[i][0];
            }
        }
    }

    float cw[4], cvw[4];
    cw[0] = __uint_as_float(cpk.x << 16); cw[1] = __uint_as_float(cpk.x & 0xffff0000u);
    cw[2] = __uint_as_float(cpk.y << 16); cw[3] = __uint_as_float(cpk.y & 0xffff0000u);
    cvw[0] = __uint_as_float(dpk.x << 16); cvw[1] = __uint_as_float(dpk.x & 0xffff0000u);
    cvw[2] = __uint_as_float(dpk.y << 16); cvw[3] = __uint_as_float(dpk.y & 0xffff0000u);
    const float A = -expf(bf2f(alogr));
    const float dtb = bf2f(dtbr);

    for (int t = 0; t < a.T; ++t) {
        const int r = gi * a.T + t;
        const int pb = t & 1;
        const uint16_t* pr = a.proj + (size_t)r * kGdnInRows;
        const uint16_t xcur = xr, xvcur = xvr;
        if (t + 1 < a.T) {      // the next row's inputs load while this row computes
            const uint16_t* pn = pr + kGdnInRows;
            xr = pn[cqk]; xvr = pn[cvc];
        }
        if ((t & 63) == 0) {
            // the gates (decay e^g, g = -e^A_log softplus(a + dt_bias); beta = sigmoid(b)) of rows
            // t .. t+63, one row per thread: off the rows' sequential path (one thread's chain of
            // transcendentals per row would sit before every row's barrier)
            if (tid < 64) {
                float bb = bf2f(gbr);
                float aa = bf2f(gar) + dtb;
                float sp = aa > 20.f ? aa : log1pf(expf(aa));
                float g = A * sp;
                gate_c[(t >> 6) & 1][tid][0] = expf(g);
                gate_c[(t >> 6) & 1][tid][1] = sigmoid_f(bb);
            }
            const uint16_t* pgn = a.proj + (size_t)(gi * a.T + min(t + 64 + (tid & 63), a.T - 1)) * kGdnInRows;
            gbr = pgn[kGdnBOff + h];           // the next chunk's
            gar = pgn[kGdnAOff + h];
        }
        // causal conv: taps over [w0, w1, w2, raw] in order, f32, one rounding, bf16 SiLU
        {
            float x = bf2f(xcur);
            float u = 0.f;
            u = u + w0 * cw[0]; u = u + w1 * cw[1]; u = u + w2 * cw[2]; u = u + x * cw[3];
            float uq = rbf(silu_f(rbf(u)));
            w0 = w1; w1 = w2; w2 = x;
            if (tid < 128) qs[pb][tid] = uq; else ks[pb][tid - 128] = uq;
            if (hasv) {
                float xv = bf2f(xvcur);
                float uv = 0.f;
                uv = uv + v0 * cvw[0]; uv = uv + v1 * cvw[1]; uv = uv + v2 * cvw[2]; uv = uv + xv * cvw[3];
                vs[pb][tid] = rbf(silu_f(rbf(uv)));
                v0 = v1; v1 = v2; v2 = xv;
            }
            // squared norms: waves 0-1 hold q, waves 2-3 hold k
            float ss = wave_sum(uq * uq);
            if ((tid & 63) == 0) wred[pb][tid >> 6] = ss;
        }
        lds_barrier();
        // q~ and k~ of this lane's rows, normalised where they are read (the same two rounded
        // products as a normalisation pass)
        const float rq = rsqrtf((wred[pb][0] + wred[pb][1]) + 1e-6f);
        const float rk = rsqrtf((wred[pb][2] + wred[pb][3]) + 1e-6f);
        const float gam = gate_c[(t >> 6) & 1][t & 63][0], beta = gate_c[(t >> 6) & 1][t & 63][1];
        float kn[KR], qn[KR];
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            kn[i] = __fmul_rn(ks[pb][kg * KR + i], rk);
            qn[i] = __fmul_rn(__fmul_rn(qs[pb][kg * KR + i], rq), 0.08838834764831845f);
        }
        // reductions over k: 8-row partial sums, then the 16 partials in order -- the same
        // arithmetic for every column-slice count, so batched lanes match batch 1 exactly
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int gq = 0; gq < GPT; ++gq) {
                float rp = 0.f;
#pragma unroll
                for (int i = gq * 8; i < gq * 8 + 8; ++i) {
                    s[i][c] = __fmul_rn(s[i][c], gam);
                    rp = fmaf(s[i][c], kn[i], rp);
                }
                red_r[kg * GPT + gq][jc + c] = rp;
            }
        wave_sync();
        float dv[CW];
        if constexpr (CW == 4) {
            // lane L < 32 sums column cc's 16 partials and leaves its dv in vs (read only
            // here); the wave's lanes then take the dv of their four columns
            if (lane64 < 32) {
                float rj = 0.f;
#pragma unroll
                for (int i = 0; i < NG; ++i) rj += red_r[i][cc];
                vs[pb][cc] = __fmul_rn(beta, vs[pb][cc] - rj);
            }
            wave_sync();
            const q35_f32x4 d4 = *(const q35_f32x4*)(vs[pb] + jc);
            dv[0] = d4[0]; dv[CW > 1 ? 1 : 0] = d4[1]; dv[CW > 2 ? 2 : 0] = d4[2]; dv[CW > 3 ? 3 : 0] = d4[3];
        } else {
            float rj = 0.f;
#pragma unroll
            for (int i = 0; i < NG; ++i) rj += red_r[i][jc];
            dv[0] = __fmul_rn(beta, vs[pb][jc] - rj);
        }
        if ((a.ckpt && a.fac_write) || rec) {
            // verify row t's factors, into the set not being read; a deferred decode row's as
            // row npend of the set being read (rows 0 .. npend-1 are the ones replayed)
            float* F = a.fac + lane * a.fac_lane + (rec ? pset : 1 - pset) * a.fac_set + (rec ? npend : t) * a.fac_row +
                       h * kFacStride;
            if (kg == 0) {
#pragma unroll
                for (int c = 0; c < CW; ++c) F[128 + cs * VC + jc + c] = dv[c];
            }
            if (cs == 0 && tid >= 128) F[tid - 128] = __fmul_rn(ks[pb][tid - 128], rk);
            if (cs == 0 && tid == 0) F[256] = gam;
        }
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int gq = 0; gq < GPT; ++gq) {
                float op = 0.f;
#pragma unroll
                for (int i = gq * 8; i < gq * 8 + 8; ++i) {
                    s[i][c] = delta_update(s[i][c], kn[i], dv[c]);
                    op = fmaf(qn[i], s[i][c], op);
                }
                red_o[kg * GPT + gq][jc + c] = op;
            }
        wave_sync();
        if constexpr (CW == 4) {
            // lane L < 32 sums column cc's o partials and stores o; with the fused gated norm
            // the head's two half sums of squares are formed as half_head_ss forms them
            // (quads in column order, each ((o0^2 + o1^2) + (o2^2 + o3^2))): a quad's four
            // lanes pair up by shuffles and its first lane leaves the quad in qq
            float oc = 0.f;
#pragma unroll
            for (int i = 0; i < NG; ++i) oc += red_o[i][cc];
            if (lane64 < 32) a.o[(size_t)r * 2048 + h * 128 + cc] = oc;
            if (a.y) {
                const float sq = __fmul_rn(oc, oc);
                const float s2 = __fadd_rn(sq, __shfl_xor(sq, 1, 64));          // lanes 4j, 4j + 2
                const float q4 = __fadd_rn(s2, __shfl_down(s2, 2, 64));         // lane 4j
                if (lane64 < 32 && (lane64 & 3) == 0) qq[cc >> 2] = q4;
                lds_barrier();
                if (lane64 < 32) {
                    float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        ss0 = __fadd_rn(ss0, qq[j]);
                        ss1 = __fadd_rn(ss1, qq[16 + j]);
                    }
                    const float rs = head_rsqrt(ss0, ss1);
                    const float z = bf2f(pr[kGdnZOff + h * 128 + cc]);
                    const float w = bf2f(a.gnorm[cc]);
                    a.y[(size_t)r * 2048 + h * 128 + cc] = f2bf(__fmul_rn(__fmul_rn(w, __fmul_rn(oc, rs)), silu_f(z)));
                }
            }
        } else {
            if (kg == 0) {
                float oj = 0.f;
#pragma unroll
                for (int i = 0; i < NG; ++i) oj += red_o[i][jc];
                a.o[(size_t)r * 2048 + h * 128 + cs * VC + jc] = oj;
            }
        }
        if ((a.ckpt && !a.fac_write) || (!a.ckpt && t == a.T - 1 && !rec)) {
            const int slot = (cur + 1 + (a.ckpt ? t : 0)) % a.nslots;
            float* So = Sbase + slot * a.S_slot;
#pragma unroll
            for (int i = 0; i < KR; ++i) {
                float* p = So + (kg * KR + i) * 128 + cs * VC + jc;
                if (CW == 4)
                    __builtin_nontemporal_store((q35_f32x4){s[i][0], s[i][CW > 1 ? 1 : 0], s[i][CW > 2 ? 2 : 0], s[i][CW > 3 ? 3 : 0]},
                                                (q35_f32x4*)p);
                else p[0] = s[i][0];
            }
        }
        if (a.ckpt || t == a.T - 1) {
            float* Wo = Wbase + ((wcur + 1 + (a.ckpt ? t : 0)) % a.nslots) * a.W_slot;
            if (cs == 0) { Wo[cqk] = w0; Wo[6144 + cqk] = w1; Wo[12288 + cqk] = w2; }
            if (hasv) { Wo[cv] = v0; Wo[6144 + cv] = v1; Wo[12288 + cv] = v2; }
        }
    }
}

// Persistent form of gdn_kernel<1> for one decode row per lane (T = 1, no checkpoints):
// each block walks (row, head) items gi*16 + h = blockIdx.x, + gridDim.x, ...; while item i
// computes, everything item i+1 reads is already in flight: its 64 KiB state and its pending
// factor rows stream into LDS with global_load_lds (no VGPRs), its conv window, conv taps,
// projection row and gates into registers. The items' row metadata (lane, slots, pending
// rows) is read once, at the start, into LDS. So an item waits on memory once, at its top,
// for loads issued a whole item earlier (and for the previous item's stores, which the same
// counter tracks). All of those loads are unconditional (clamped indices): a load under a
// branch would make the compiler wait for it where the branch joins. Same thread mapping
// and arithmetic, statement for statement, as gdn_kernel<1> with T = 1.
// Barriers are lds_barrier(): __syncthreads() would make every wave wait for the next item's
// prefetch, which would then never overlap an item's compute.

constexpr int kPersistMaxItems = 128;      // items per block: rows <= 4,096 at 512 blocks
constexpr int kPersistLds = 64 * 1024 + kMaxPend * kFacStride * 4;   // state + factor rows

template <int TR>
__global__ void __launch_bounds__(256, 2) gdn_persist(GdnArgs a, int nitems) {
    constexpr int VC = 128, CW = 4, CG = 32, KR = 16, NG = 16, GPT = 2;
    const int tid = threadIdx.x, lane64 = tid & 63, wv = tid >> 6;
    // wave w owns value columns 32w .. 32w+31 over all 128 k rows: lane (kg, quad) holds k rows
    // 16 kg .. +15 of columns jc .. jc+3. The delta rule's columns are independent, so the r and
    // o reductions over k stay inside the wave (through its own columns of red, no barrier).
    const int jc = wv * 32 + (lane64 & 7) * CW, kg = lane64 >> 3;
    const int cc = wv * 32 + (lane64 & 31);      // the column a lane < 32 reduces
    // Dynamic LDS, the only target of the LDS-DMA prefetch (so the compiler need not make an
    // access to the static arrays below wait for it): the next item's state [4 waves][16 rows]
    // [64 lanes], then its pending factor rows (row p at p * kFacStride; 5 KiB, so that two
    // blocks still fit a CU)
    extern __shared__ q35_f32x4 sbuf[];
    float* fbuf = (float*)(sbuf + 4096);
    __shared__ float qs[128], ks[128], vs[VC];
    __shared__ float red[NG][VC];            // r partials, then o partials
    __shared__ float wred[TR][4];            // per row: the waves' q / k square sums
    __shared__ float gate_s[TR > 2 ? TR : 2][2];   // (decay, beta): one row, of items with even / odd k;
                                             // verify rows: of rows 0 .. TR-1
    __shared__ float qq[32];                 // the item's 32 quads of o^2, in column order
    // item k's row metadata: lane | cur << 16 | wcur << 20 | pend code << 24
    __shared__ int meta[kPersistMaxItems];
    const int nk = (nitems - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    for (int k = tid; k < nk; k += 256) {
        const int gi = (((int)blockIdx.x + k * (int)gridDim.x) >> 4) * TR;   // the lane's first row
        const int ln = a.lane[gi];
        const int cu = a.cur ? a.cur[gi] : 0;
        const int wc = a.wcur ? a.wcur[gi] : cu;
        const int pn = a.pend ? a.pend[gi] : 0;
        meta[k] = ln | (cu << 16) | (wc << 20) | (pn << 24);
    }
    __syncthreads();

    // per-item operands in registers (loaded one item ahead; bf16 kept as raw bits until use,
    // so no conversion makes the compiler wait for a load in the fetch)
    const bool hasv = tid < VC;
    struct Ops {
        float w0, w1, w2, v0, v1, v2;
        uint16_t x[TR], xv[TR], bb[TR], aa[TR], alog, dtb;
        uint16_t z1[TR], g1;         // z and gnorm weight of column cc (y of lanes < 32)
        uint2 cpk, dpk;
    };
    const uint16_t* gnw = a.gnorm ? a.gnorm : a.dt_bias;   // any valid address when unused
    // an item's gates (decay e^g, g = -e^A_log softplus(a + dt_bias); beta = sigmoid(b)), made by
    // one thread: for item k + 1 by thread 64 while wave 0 finishes item k (waves 1-3 would
    // otherwise wait for it at the next item's first barrier), for the first item in its conv phase
    auto gates = [&](const Ops& o, int t, float* dst) {
        const float A = -expf(bf2f(o.alog));
        const float aa = bf2f(o.aa[t]) + bf2f(o.dtb);
        float sp = aa > 20.f ? aa : log1pf(expf(aa));
        float g = A * sp;
        dst[0] = expf(g);
        dst[1] = sigmoid_f(bf2f(o.bb[t]));
    };
    // the next item's state rows 4g .. 4g+3 of this thread (the four groups are issued at four
    // points of an item's compute, so the memory pipe stays busy through it instead of the
    // wave stalling on one burst of 16 DMA issues and then leaving the pipe idle)
    // (wave-uniform head base in scalar registers plus the lane's fixed 32-bit byte offset: the
    // loads take the scalar-base address form and cost no vector address arithmetic)
    const char* Snext = nullptr;
    const unsigned voff = (unsigned)(kg * KR * 128 + jc) * 4u;
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
    auto fetch_rows = [&](int g) {
#pragma unroll
        for (int i = 4 * g; i < 4 * g + 4; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(uniform_ptr(Snext + i * 512) + voff),
                                             (__attribute__((address_space(3))) void*)(sbuf + (wvu * KR + i) * 64), 16, 0, 0);
    };
    auto fetch = [&](int k, Ops& o) {
        const int item = (int)blockIdx.x + k * (int)gridDim.x;
        const int gi = item >> 4, h = item & 15;
        const int m = __builtin_amdgcn_readfirstlane(meta[k]);
        const int ln = m & 0xffff, cu = (m >> 16) & 15, wc = (m >> 20) & 15, pn = (m >> 24) & 31;
        Snext = (const char*)(a.S + ln * a.S_lane + a.S_layer + (long long)h * 16384 + cu * a.S_slot);
        fetch_rows(0);
        const float* Win = a.win + ln * a.W_lane + a.W_layer + wc * a.W_slot;
        const uint16_t* pr0 = a.proj + (size_t)gi * TR * kGdnInRows;
        const int cqk = tid < 128 ? h * 128 + tid : 2048 + h * 128 + (tid - 128);
        const int cv = 4096 + h * 128 + (tid & 127);      // threads >= 128 load a valid channel, unused
        o.w0 = Win[cqk]; o.w1 = Win[6144 + cqk]; o.w2 = Win[12288 + cqk];
        o.v0 = Win[cv]; o.v1 = Win[6144 + cv]; o.v2 = Win[12288 + cv];
        o.cpk = *(const uint2*)(a.conv_w + (size_t)cqk * 4);
        o.dpk = *(const uint2*)(a.conv_w + (size_t)cv * 4);
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            const uint16_t* pr = pr0 + (size_t)t * kGdnInRows;
            o.x[t] = pr[cqk];
            o.xv[t] = pr[cv];
            o.z1[t] = pr[kGdnZOff + h * 128 + cc];
            o.bb[t] = pr[kGdnBOff + h];
            o.aa[t] = pr[kGdnAOff + h];
        }
        o.g1 = gnw[a.gnorm ? cc : 0];
        o.alog = a.A_log[h];
        o.dtb = a.dt_bias[h];
    };
    // item k's pending factor rows 0 .. npend-1 into fbuf: 16-byte chunk c = 66 p + q of row p,
    // chunks tid, tid + 256 (issued once every wave is done with the previous rows)
    auto fetch_fac = [&](int k) {
        const int item = (int)blockIdx.x + k * (int)gridDim.x;
        const int h = item & 15;
        const int m = meta[k];
        const int ln = m & 0xffff, pn = (m >> 24) & 31;
        const int nc = (pn & 15) * (kFacStride / 4);
        const float* F0 = a.fac + ln * a.fac_lane + ((pn >> 4) & 1) * a.fac_set + h * kFacStride;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = tid + 256 * u;
            if (c < nc) {
                const int p = c / (kFacStride / 4), q = c % (kFacStride / 4);
                __builtin_amdgcn_global_load_lds((const void*)(F0 + p * a.fac_row + 4 * q),
                                                 (__attribute__((address_space(3))) void*)(fbuf + 1024 * u + wv * 256),
                                                 16, 0, 0);
            }
        }
    };
    Ops nx;
    if (nk > 0) {
        fetch(0, nx);
        fetch_fac(0);
        fetch_rows(1); fetch_rows(2); fetch_rows(3);
    }
    for (int k = 0; k < nk; ++k) {
        const int item = (int)blockIdx.x + k * (int)gridDim.x;
        const int gi = item >> 4, h = item & 15;
        const int m = meta[k];
        const int lane = m & 0xffff, cur = (m >> 16) & 15, wcur = (m >> 20) & 15, pnd = (m >> 24) & 31;
        const int npend = pnd & 15, pset = (pnd >> 4) & 1;
        const bool rec = npend < a.defer;          // this row becomes pending row npend
        float* Sbase = a.S + lane * a.S_lane + a.S_layer + (long long)h * 16384;
        float* Wbase = a.win + lane * a.W_lane + a.W_layer;
        const int cqk = tid < 128 ? h * 128 + tid : 2048 + h * 128 + (tid - 128);
        const int cv = 4096 + h * 128 + tid;
        // this item's state, factors and operands (issued one item ago)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const Ops op = nx;
        float s[KR][CW];
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            const q35_f32x4 v = sbuf[(wv * KR + i) * 64 + lane64];
            s[i][0] = v[0]; s[i][1] = v[1]; s[i][2] = v[2]; s[i][3] = v[3];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (npend) {
            lds_barrier();      // every wave's share of the factor rows has landed
            // the lane's pending rows (gdn_kernel's replay, this block's thread mapping)
            for (int p = 0; p < npend; ++p) {
                const float* F = fbuf + p * kFacStride;
                const float gp = F[256];
                float kk[KR], dd[CW];
#pragma unroll
                for (int i = 0; i < KR; ++i) kk[i] = F[kg * KR + i];
#pragma unroll
                for (int c = 0; c < CW; ++c) dd[c] = F[128 + jc + c];
#pragma unroll
                for (int i = 0; i < KR; ++i)
#pragma unroll
                    for (int c = 0; c < CW; ++c) {
                        s[i][c] = __fmul_rn(s[i][c], gp);
                        s[i][c] = delta_update(s[i][c], kk[i], dd[c]);
                    }
            }
        }
        if constexpr (TR > 1) {
            // MTP verify rows: a lane with pending rows has them applied and the result stored to
            // slot cur + 1, the base of this verify's factors (gdn_kernel's ckpt path)
            if (npend) {
                float* So = Sbase + ((cur + 1) % a.nslots) * a.S_slot;
#pragma unroll
                for (int i = 0; i < KR; ++i)
                    __builtin_nontemporal_store((q35_f32x4){s[i][0], s[i][1], s[i][2], s[i][3]},
                                                (q35_f32x4*)(So + (kg * KR + i) * 128 + jc));
            }
        }
        const bool more = k + 1 < nk;
        if (more) fetch(k + 1, nx);
        float w0 = op.w0, w1 = op.w1, w2 = op.w2, v0 = op.v0, v1 = op.v1, v2 = op.v2;
        float cw[4], cvw[4];
        cw[0] = __uint_as_float(op.cpk.x << 16); cw[1] = __uint_as_float(op.cpk.x & 0xffff0000u);
        cw[2] = __uint_as_float(op.cpk.y << 16); cw[3] = __uint_as_float(op.cpk.y & 0xffff0000u);
        cvw[0] = __uint_as_float(op.dpk.x << 16); cvw[1] = __uint_as_float(op.dpk.x & 0xffff0000u);
        cvw[2] = __uint_as_float(op.dpk.y << 16); cvw[3] = __uint_as_float(op.dpk.y & 0xffff0000u);
        // causal conv of every row first (taps over [w0, w1, w2, raw] in order, f32, one rounding,
        // bf16 SiLU), with the rows' square sums and gates: none of it reads the state, so the rows'
        // latencies overlap instead of each row waiting for its own before the state passes
        float uqr[TR], uvr[TR];
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            const float ox = bf2f(op.x[t]), oxv = bf2f(op.xv[t]);
            float u = 0.f;
            u = u + w0 * cw[0]; u = u + w1 * cw[1]; u = u + w2 * cw[2]; u = u + ox * cw[3];
            uqr[t] = rbf(silu_f(rbf(u)));
            w0 = w1; w1 = w2; w2 = ox;
            uvr[t] = 0.f;
            if (hasv) {
                float uv = 0.f;
                uv = uv + v0 * cvw[0]; uv = uv + v1 * cvw[1]; uv = uv + v2 * cvw[2]; uv = uv + oxv * cvw[3];
                uvr[t] = rbf(silu_f(rbf(uv)));
                v0 = v1; v1 = v2; v2 = oxv;
            }
            // the conv window after this row: its values are final now (verify rows: slot wcur + 1 + t)
            float* Wo = Wbase + ((wcur + 1 + t) % a.nslots) * a.W_slot;
            Wo[cqk] = w0; Wo[6144 + cqk] = w1; Wo[12288 + cqk] = w2;
            if (hasv) { Wo[cv] = v0; Wo[6144 + cv] = v1; Wo[12288 + cv] = v2; }
        }
        {
            float ss[TR];
#pragma unroll
            for (int t = 0; t < TR; ++t) ss[t] = wave_sum(uqr[t] * uqr[t]);
            if ((tid & 63) == 0) {
#pragma unroll
                for (int t = 0; t < TR; ++t) wred[t][tid >> 6] = ss[t];
            }
            if (TR == 1 && tid == 0 && k == 0) gates(op, 0, gate_s[0]);
            if (TR > 1) {       // row t's by the first thread of wave t: the rows' chains in parallel
#pragma unroll
                for (int t = 0; t < TR; ++t)
                    if (tid == 64 * t) gates(op, t, gate_s[t]);   // read after row 0's first barrier
            }
        }
#pragma unroll
        for (int t = 0; t < TR; ++t) {
        const int r = gi * TR + t;              // this row
        if (tid < 128) qs[tid] = uqr[t]; else ks[tid - 128] = uqr[t];
        if (hasv) vs[tid] = uvr[t];
        lds_barrier();
        if (more && t == 0) { fetch_fac(k + 1); fetch_rows(1); }   // fbuf's rows were read before this barrier
        if (TR > 1 && more && t == 1) fetch_rows(3);
        // q~ and k~ of this thread's 16 rows, normalised where they are read (the same two
        // rounded products as a normalisation pass, without its barrier)
        const float rq = rsqrtf((wred[t][0] + wred[t][1]) + 1e-6f);
        const float rk = rsqrtf((wred[t][2] + wred[t][3]) + 1e-6f);
        const float gam = gate_s[TR == 1 ? (k & 1) : t][0], beta = gate_s[TR == 1 ? (k & 1) : t][1];
        float kn[KR], qn[KR];
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            kn[i] = __fmul_rn(ks[kg * KR + i], rk);
            qn[i] = __fmul_rn(__fmul_rn(qs[kg * KR + i], rq), 0.08838834764831845f);
        }
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int gq = 0; gq < GPT; ++gq) {
                float rp = 0.f;
#pragma unroll
                for (int i = gq * 8; i < gq * 8 + 8; ++i) {
                    s[i][c] = __fmul_rn(s[i][c], gam);
                    rp = fmaf(s[i][c], kn[i], rp);
                }
                red[kg * GPT + gq][jc + c] = rp;
            }
        wave_sync();
        if (more && t == 0) fetch_rows(2);
        // lane L < 32 sums column cc's 16 partials in order and leaves its dv in vs[cc] (read
        // only here); the wave's lanes then take the dv of their four columns
        if (lane64 < 32) {
            float rj = 0.f;
#pragma unroll
            for (int i = 0; i < NG; ++i) rj += red[i][cc];
            vs[cc] = __fmul_rn(beta, vs[cc] - rj);
        }
        wave_sync();
        float dv[CW];
        {
            const q35_f32x4 d4 = *(const q35_f32x4*)(vs + jc);
            dv[0] = d4[0]; dv[1] = d4[1]; dv[2] = d4[2]; dv[3] = d4[3];
        }
        if (TR > 1 || rec) {
            // gdn_kernel's factor records: a deferred decode row as row npend of the set being
            // read; a verify row t into the set not being read
            float* F = a.fac + lane * a.fac_lane + (TR > 1 ? 1 - pset : pset) * a.fac_set +
                       (TR > 1 ? t : npend) * a.fac_row + h * kFacStride;
            if (kg == 0) *(q35_f32x4*)(F + 128 + jc) = (q35_f32x4){dv[0], dv[1], dv[2], dv[3]};
            if (tid >= 128) F[tid - 128] = __fmul_rn(ks[tid - 128], rk);
            if (tid == 0) F[256] = gam;
        }
        wave_sync();            // red's columns of this wave are reused for the o partials
        if (TR == 1 && more) fetch_rows(3);
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int gq = 0; gq < GPT; ++gq) {
                float op2 = 0.f;
#pragma unroll
                for (int i = gq * 8; i < gq * 8 + 8; ++i) {
                    s[i][c] = delta_update(s[i][c], kn[i], dv[c]);
                    op2 = fmaf(qn[i], s[i][c], op2);
                }
                red[kg * GPT + gq][jc + c] = op2;
            }
        if (TR == 1 && !rec) {
            const int slot = (cur + 1) % a.nslots;
            float* So = Sbase + slot * a.S_slot;
#pragma unroll
            for (int i = 0; i < KR; ++i)
                __builtin_nontemporal_store((q35_f32x4){s[i][0], s[i][1], s[i][2], s[i][3]},
                                            (q35_f32x4*)(So + (kg * KR + i) * 128 + jc));
        }
        wave_sync();
        // the head's outputs: lane L < 32 sums column cc's 16 o partials in order and stores o;
        // the gated norm needs the head's two half sums of squares, formed as half_head_ss forms
        // them (quads in column order, each ((o0^2 + o1^2) + (o2^2 + o3^2))): a quad's four
        // lanes pair up by shuffles and its first lane leaves the quad in qq. The barrier ending
        // the row also keeps the next row's conv phase (qs, ks, vs, wred) from running ahead
        // of a wave still reading them.
        float oc = 0.f;
#pragma unroll
        for (int i = 0; i < NG; ++i) oc += red[i][cc];
        {
            const float tq = __fmul_rn(oc, oc);
            const float t2 = __fadd_rn(tq, __shfl_xor(tq, 1, 64));          // lanes 4j, 4j + 2
            const float q = __fadd_rn(t2, __shfl_down(t2, 2, 64));          // lane 4j
            if (lane64 < 32) {
                a.o[(size_t)r * 2048 + h * 128 + cc] = oc;
                if ((lane64 & 3) == 0) qq[cc >> 2] = q;
            }
        }
        if (TR == 1 && more && tid == 64) gates(nx, 0, gate_s[(k + 1) & 1]);
        lds_barrier();
        if (a.y && lane64 < 32) {
            float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                ss0 = __fadd_rn(ss0, qq[j]);
                ss1 = __fadd_rn(ss1, qq[16 + j]);
            }
            const float rs = head_rsqrt(ss0, ss1);
            const float yv = __fmul_rn(__fmul_rn(bf2f(op.g1), __fmul_rn(oc, rs)), silu_f(bf2f(op.z1[t])));
            a.y[(size_t)r * 2048 + h * 128 + cc] = f2bf(yv);
        }
        }
    }
}

// Pending rows applied to a lane's state of every layer: block (row, layer, head), thread
// (k row tid / 2, value columns 64 (tid % 2) .. +64), the replay of gdn_kernel.
__global__ void __launch_bounds__(256) gdn_materialize(float* S, long long S_lane, long long S_slot, const int* lanes,
                                                       const int* curs, const int* pends, const float* fac,
                                                       long long fac_lane, long long fac_set, long long fac_layer,
                                                       long long fac_row, int nslots) {
    const int r = blockIdx.x, l = blockIdx.y, h = blockIdx.z, tid = threadIdx.x;
    const int pnd = pends[r], npend = pnd & 15, pset = (pnd >> 4) & 1;
    if (!npend) return;
    const int lane = lanes[r], cur = curs[r];
    const int i = tid >> 1, c0 = (tid & 1) * 64;
    const float* Sin = S + lane * S_lane + cur * S_slot + (long long)l * kSLayer + (long long)h * 16384 + i * 128 + c0;
    float* So = S + lane * S_lane + ((cur + 1) % nslots) * S_slot + (long long)l * kSLayer + (long long)h * 16384 + i * 128 + c0;
    float v[64];
#pragma unroll
    for (int q = 0; q < 16; ++q) *(q35_f32x4*)&v[4 * q] = *(const q35_f32x4*)(Sin + 4 * q);
    const float* F0 = fac + lane * fac_lane + pset * fac_set + l * fac_layer + h * kFacStride;
    for (int p = 0; p < npend; ++p) {
        const float* F = F0 + p * fac_row;
        const float gp = F[256], kk = F[i];
#pragma unroll
        for (int c = 0; c < 64; ++c) {
            v[c] = __fmul_rn(v[c], gp);
            v[c] = delta_update(v[c], kk, F[128 + c0 + c]);
        }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) *(q35_f32x4*)(So + 4 * q) = *(const q35_f32x4*)&v[4 * q];
}

hipError_t launch_gdn_materialize(float* S, long long S_lane, long long S_slot, const int* lane, const int* cur,
                                  const int* pend, const float* fac, long long fac_lane, long long fac_set,
                                  long long fac_layer, long long fac_row, int nslots, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gdn_materialize, dim3(n, kGdnLayers, kHv), dim3(256), 0, st, S, S_lane, S_slot, lane, cur,
                       pend, fac, fac_lane, fac_set, fac_layer, fac_row, nslots);
    return hipGetLastError();
}

hipError_t gdn_init() {
    hipError_t e = hipFuncSetAttribute((const void*)gdn_persist<1>, hipFuncAttributeMaxDynamicSharedMemorySize, kPersistLds);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)gdn_persist<2>, hipFuncAttributeMaxDynamicSharedMemorySize, kPersistLds);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void*)gdn_persist<3>, hipFuncAttributeMaxDynamicSharedMemorySize, kPersistLds);
}

hipError_t launch_gdn_persist(const GdnArgs& a, hipStream_t st) {
    // one decode row per lane, or MTP verify rows (T = 2, 3: checkpoints as factor records)
    const bool verify = a.T > 1;
    if (a.nlanes <= 0 || a.T < 1 || a.T > 3 || (verify && !(a.ckpt && a.fac_write)) || (!verify && a.ckpt))
        return hipErrorInvalidValue;
    const int nitems = a.nlanes * kHv;
    const int grid = nitems < 512 ? nitems : 512;      // two blocks per CU
    // more than 128 items per block (above 4,096 lanes): the one-block-per-(lane, head) kernel,
    // same bits
    if ((nitems + grid - 1) / grid > kPersistMaxItems) return launch_gdn(a, 1, st);
    if (a.T == 1) hipLaunchKernelGGL(gdn_persist<1>, dim3(grid), dim3(256), kPersistLds, st, a, nitems);
    else if (a.T == 2) hipLaunchKernelGGL(gdn_persist<2>, dim3(grid), dim3(256), kPersistLds, st, a, nitems);
    else hipLaunchKernelGGL(gdn_persist<3>, dim3(grid), dim3(256), kPersistLds, st, a, nitems);
    return hipGetLastError();
}

hipError_t launch_gdn(const GdnArgs& a, int col_slices, hipStream_t st) {
    if (a.nlanes <= 0 || a.T <= 0) return hipErrorInvalidValue;
    dim3 grid(a.nlanes, kHv, col_slices);
    switch (col_slices) {
        case 1: hipLaunchKernelGGL(gdn_kernel<1>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(gdn_kernel<2>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(gdn_kernel<4>, grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(gdn_kernel<8>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace q35
