// Shared device/host definitions of the Qwen3.5-0.8B MI355X (gfx950) decode engine.
//
// Model constants follow speccheck/specimpl.py:26-58 and engine/state.h:41-67 of the
// reference. Storage is IEEE bfloat16 bits in uint16_t; all accumulation is f32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q35 {

constexpr int kHidden = 1024;
constexpr int kLayers = 24;
constexpr int kGdnLayers = 18;
constexpr int kAttnLayers = 6;
constexpr int kFF = 3584;
constexpr int kVocab = 248320;
constexpr int kHv = 16;            // GDN value heads (= key heads)
constexpr int kDk = 128;
constexpr int kDv = 128;
constexpr int kConvCh = 6144;      // q 2048 | k 2048 | v 2048
constexpr int kConvK = 4;
constexpr long long kSLayer = (long long)kHv * kDk * kDv;   // one GDN layer's state, 262144 f32
constexpr long long kWLayer = 3LL * kConvCh;                // one layer's conv window, 18432 f32
constexpr int kNq = 8;
constexpr int kNkv = 2;
constexpr int kHeadDim = 256;
constexpr int kRotDim = 64;
constexpr float kEps = 1e-6f;
constexpr float kRopeTheta = 1e7f;

// Fused input projection widths (rows of the concatenated weight matrix).
constexpr int kGdnInRows = kConvCh + 2048 + 16 + 16;   // qkv | z | b | a  = 8224
constexpr int kGdnZOff = kConvCh;                      // 6144
constexpr int kGdnBOff = kConvCh + 2048;               // 8192
constexpr int kGdnAOff = kConvCh + 2048 + 16;          // 8208
constexpr int kAttnInRows = 2 * kNq * kHeadDim + 2 * kNkv * kHeadDim;   // q|gate 4096, k 512, v 512
constexpr int kAttnKOff = 2 * kNq * kHeadDim;          // 4096
constexpr int kAttnVOff = kAttnKOff + kNkv * kHeadDim; // 4608
constexpr int kGuRows = 2 * kFF;                       // gate 3584 | up 3584

constexpr bool is_attn_layer(int l) { return (l % 4) == 3; }
constexpr int gdn_slot(int l) { return l - (l + 1) / 4; }
constexpr int attn_slot(int l) { return l / 4; }

// GEMM weight tiling: 16 output rows x 256 k per tile, 8 KiB contiguous, laid out so a
// wave's 8 dwordx4 loads (step s = 0..7, lane = g*16 + n%16) are each 1 KiB contiguous.
// Element (n, k): tile (n/16, k/256); g = (k%256)/64; s = (k%64)/8; e = k%8.
constexpr int kTileN = 16;
constexpr int kTileK = 256;
// K cache of one (lane, layer, kv head): 16-slot tiles in MFMA fragment order, so a score
// step's operand (16 slots x 32 dims) is one contiguous KiB: tile slot/16, step d/32, lane
// ((d/8) % 4) * 16 + slot % 16, element d % 8. Regions are padded to whole tiles.
__host__ __device__ inline size_t kv_tiled_offset(int slot, int d) {
    return (size_t)(slot >> 4) * 4096 + (d >> 5) * 512 + ((((d >> 3) & 3) << 4) | (slot & 15)) * 8 + (d & 7);
}
__host__ __device__ inline int kv_cap_padded(int cap) { return (cap + 15) & ~15; }
// V cache of one (lane, layer, kv head): 8-slot groups, dim-major inside a group, so one
// 16-byte load holds 8 consecutive slots of one dim -- a P.V fragment on MFMA (k = slots):
// element (slot, d) at (slot/8) * 2048 + d * 8 + slot % 8.
__host__ __device__ inline size_t kv_v8_offset(int slot, int d) {
    return (size_t)(slot >> 3) * 2048 + d * 8 + (slot & 7);
}

__host__ __device__ inline size_t tiled_offset(int n, int k, int K) {
    int nt = n >> 4, kb = k >> 8, kk = k & 255;
    int g = kk >> 6, s = (kk >> 3) & 7, e = kk & 7;
    int lane = g * 16 + (n & 15);
    return ((((size_t)nt * (K >> 8) + kb) * 8 + s) * 64 + lane) * 8 + e;
}

}  // namespace q35

// ---------------------------------------------------------------- device helpers
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 q35_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float q35_f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t q35_u32x4;

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round-to-nearest-even f32 -> bf16 bits (NaN stays a quiet NaN).
// Branchless (selects, no divergent branch per element).
// f32 -> bf16, round to nearest even (NaN: the high half with the quiet bit set), by gfx950's
// v_cvt_pk_bf16_f32: one instruction for two values instead of six for one. Checked on MI355X
// against the integer form (u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN -> (u >> 16) | 0x40, for all
// 2^32 inputs: identical bits.
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}
__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)f2bf2(f, 0.f); }
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(f2bf2(0.f, f) & 0xffff0000u); }

// A block barrier for LDS traffic only: __syncthreads() also orders global memory, for which
// the compiler makes every wave wait for all of its outstanding loads first, including loads
// issued ahead for later work, which would then never overlap the current work.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// orders a wave's own LDS traffic for the compiler: one wave's LDS accesses execute in
// program order, so lanes of the wave see each other's earlier writes without a barrier
__device__ __forceinline__ void wave_sync() { asm volatile("" ::: "memory"); }

// A wave-uniform pointer as scalar registers the compiler cannot fold with a lane's offset, so
// that p + (32-bit lane offset) takes the scalar-base global address form (no vector address
// arithmetic per load).
__device__ __forceinline__ const char* uniform_ptr(const char* p) {
    const unsigned long long u = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    return (const char*)(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// __shfl_xor(v, 32) without LDS: v_permlane32_swap exchanges the two 32-lane halves
// (result [1] holds the upper half's values for lanes < 32, [0] the lower half's for lanes >= 32)
__device__ __forceinline__ float xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
// lane i <- lane i + 4 within its row of 16 (DPP row_shl:4; 0 for the last 4 lanes of a row)
__device__ __forceinline__ float row_down4(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// The delta rule's state update s + k * dv with the product rounded before the add, as the
// reference's torch path forms S + k (x) dv (speccheck/specimpl.py:287-294). HIP's __fmul_rn /
// __fadd_rn are plain operators that the compiler may fuse into one FMA; contraction is off
// here, so every kernel that updates or replays a state row gets the same two roundings.
__device__ __forceinline__ float delta_update(float s, float k, float dv) {
#pragma clang fp contract(off)
    return s + k * dv;
}

// ---------------------------------------------------------------- 1024-wide RMSNorm pieces
// The zero-centred RMSNorm's reduction tree, written once so every kernel that normalises a
// hidden row (the add+norm kernel, the GEMM A-producer) gives identical bits: element
// quad t (0..255) -> ((x0^2 + x1^2) + x2^2) + x3^2; quads t = 64w + lane summed by the
// wave xor tree; the four wave sums as (w0 + w1) + (w2 + w3).
__device__ __forceinline__ float quad_ss(float x0, float x1, float x2, float x3) {
    return __fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1)), __fmul_rn(x2, x2)),
                     __fmul_rn(x3, x3));
}
__device__ __forceinline__ float hidden_rsqrt(float ss) {
    return rsqrtf(__fadd_rn(__fmul_rn(ss, 1.0f / 1024.0f), 1e-6f));
}
// h = bf16((x * rs) * (1 + w))
__device__ __forceinline__ float norm_elem(float x, float rs, float w) {
    return rbf(__fmul_rn(__fmul_rn(x, rs), __fadd_rn(1.0f, w)));
}

// ---------------------------------------------------------------- gated-norm / SwiGLU pieces
// Shared by the GEMM A-producers and the GDN kernel's fused epilogue (identical bits).
// Sum of squares of 64 consecutive f32 (half of a 128-wide head), fixed order.
__device__ __forceinline__ float half_head_ss_regs(const float* v) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 64; i += 4)
        ss = __fadd_rn(ss, __fadd_rn(__fadd_rn(__fmul_rn(v[i], v[i]), __fmul_rn(v[i + 1], v[i + 1])),
                                     __fadd_rn(__fmul_rn(v[i + 2], v[i + 2]), __fmul_rn(v[i + 3], v[i + 3]))));
    return ss;
}
__device__ __forceinline__ float half_head_ss(const float* po) {
    float v[64];
#pragma unroll
    for (int i = 0; i < 16; ++i) *(float4*)&v[4 * i] = *(const float4*)(po + 4 * i);
    return half_head_ss_regs(v);
}
__device__ __forceinline__ float head_rsqrt(float ss_lo, float ss_hi) {
    return rsqrtf(__fadd_rn(__fmul_rn(__fadd_rn(ss_lo, ss_hi), 1.0f / 128.0f), 1e-6f));
}
// act = bf16(bf16(silu(g)) * u) for 8 packed bf16 pairs
__device__ __forceinline__ q35_u32x4 silu_mul8(q35_u32x4 g, q35_u32x4 u) {
    q35_u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float g0 = __uint_as_float(g[i] << 16), g1 = __uint_as_float(g[i] & 0xffff0000u);
        float u0 = __uint_as_float(u[i] << 16), u1 = __uint_as_float(u[i] & 0xffff0000u);
        uint32_t lo = f2bf(__fmul_rn(rbf(silu_f(g0)), u0));
        uint32_t hi = f2bf(__fmul_rn(rbf(silu_f(g1)), u1));
        r[i] = lo | (hi << 16);
    }
    return r;
}
// y = bf16(w * (o * rs) * silu(z)) for 8 elements
__device__ __forceinline__ q35_u32x4 gated8(const float* ov, q35_u32x4 zz, q35_u32x4 ww, float rs) {
    q35_u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t out2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float z = h ? __uint_as_float(zz[i] & 0xffff0000u) : __uint_as_float(zz[i] << 16);
            float w = h ? __uint_as_float(ww[i] & 0xffff0000u) : __uint_as_float(ww[i] << 16);
            float n = __fmul_rn(ov[2 * i + h], rs);
            out2[h] = f2bf(__fmul_rn(__fmul_rn(w, n), silu_f(z)));
        }
        r[i] = out2[0] | (out2[1] << 16);
    }
    return r;
}

