/* Oracle-side generator for the synthetic Qwen3.5-0.8B weights and inputs.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this. The product library carries its own generator
 * (qwen3.5-0.8b_amd/csrc/q35_init.hip); tests check that both produce the same bits.
 *
 * The reference initialises nothing itself (it loads a checkpoint, speccheck/specimpl.py:65-91);
 * the workload's init is N(0,0.02) matrices, RMSNorm weights 1.0, A_log = log U(1,16),
 * dt_bias ~ U(-1,1). This file defines a portable, transcendental-free stream so that
 * C, numpy and device code produce identical bits:
 *
 *   mix(x)         = splitmix64 finaliser of (x + 0x9E3779B97F4A7C15)
 *   key(seed, tid) = mix(mix(seed) + tid)
 *   r_j(i)         = mix(key + 3*i + j),  j = 0,1,2
 *   normal(i)      = (float)(sum of the 12 16-bit halves of r_0..r_2  - 393210) * (float)(std/65536)
 *                    (Irwin-Hall of 12 uniforms: mean 0, variance 1 up to 2^-32)
 *   uniform01(i)   = (float)(r_0 >> 40) * 2^-24
 * Values are rounded to bf16 with round-to-nearest-even.
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>

static inline uint64_t mix(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t q35o_key(uint64_t seed, uint64_t tid) { return mix(mix(seed) + tid); }

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline int32_t irwin12(uint64_t key, uint64_t i) {
    int32_t s = 0;
    for (int j = 0; j < 3; ++j) {
        uint64_t r = mix(key + 3 * i + (uint64_t)j);
        s += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) +
             (int32_t)((r >> 32) & 0xffff) + (int32_t)(r >> 48);
    }
    return s - 393210;
}

/* n normal bf16 values of stream (seed, tid), elements [start, start+n). */
void q35o_normal_bf16(uint64_t seed, uint64_t tid, float stdv, uint64_t start, uint64_t n,
                      uint16_t* out) {
    uint64_t key = q35o_key(seed, tid);
    float scale = (float)((double)stdv / 65536.0);
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < (int64_t)n; ++k) {
        volatile float v = (float)irwin12(key, start + (uint64_t)k) * scale;
        out[k] = f32_to_bf16(v);
    }
}

/* Same stream, f32 values (seeded GDN state). */
void q35o_normal_f32(uint64_t seed, uint64_t tid, float stdv, uint64_t start, uint64_t n,
                     float* out) {
    uint64_t key = q35o_key(seed, tid);
    float scale = (float)((double)stdv / 65536.0);
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < (int64_t)n; ++k) {
        volatile float v = (float)irwin12(key, start + (uint64_t)k) * scale;
        out[k] = v;
    }
}

/* uniform [0,1) f32 values of stream (seed, tid). */
void q35o_uniform_f32(uint64_t seed, uint64_t tid, uint64_t start, uint64_t n, float* out) {
    uint64_t key = q35o_key(seed, tid);
    for (uint64_t k = 0; k < n; ++k)
        out[k] = (float)(mix(key + 3 * (start + k)) >> 40) * (1.0f / 16777216.0f);
}

/* token ids uniform in [0, vocab): (r_0 >> 32) % vocab. */
void q35o_tokens(uint64_t seed, uint64_t tid, uint64_t n, uint32_t vocab, int32_t* out) {
    uint64_t key = q35o_key(seed, tid);
    for (uint64_t k = 0; k < n; ++k) out[k] = (int32_t)((mix(key + 3 * k) >> 32) % vocab);
}
