/* C ABI of the MI355X (gfx950) Qwen3.5-0.8B decode engine: libqwen35.so.
 *
 * Plain pointers and sizes only; every entry point returns 0 on success or a negative
 * q35_status, and q35_last_error() describes the last failure of the calling thread.
 * One engine owns one HIP stream, its device weights and its scratch; it is not
 * thread-safe. Host pointers are host memory unless a name says "_dev".
 *
 * Lanes are independent sequences (requests). A state holds `lanes` copies of the
 * reference's per-request tuple (engine/state.h:83-116): GDN S f32 [18][16][128][128],
 * conv window f32 [18][3][6144], K and V caches bf16 [6][2][cap][256], prefix_len, plus
 * the MTP block's own K/V [2][mtp_cap][256] and its length.
 */
#ifndef Q35_H
#define Q35_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q35_engine q35_engine;
typedef struct q35_state q35_state;

enum q35_status {
    Q35_OK = 0,
    Q35_ERR_ARG = -1,      /* bad argument: token out of range, lane out of range, NULL, ... */
    Q35_ERR_CAP = -2,      /* context capacity or row capacity exceeded */
    Q35_ERR_HIP = -3,      /* a HIP call failed */
    Q35_ERR_STATE = -4     /* call order violated (no weights, no MTP slots, ...) */
};

typedef struct q35_config {
    int device;            /* HIP device ordinal */
    int max_rows;          /* rows (lanes x tokens) one body pass may carry */
    int max_ctx;           /* largest cache capacity any state will use (sizes attention scratch) */
    int use_graph;         /* capture decode bodies in hipGraphs (1) or launch eagerly (0) */
} q35_config;

/* Engine lifetime.  Replaces WeightStore + allocate_scratch + prepare_weight_adapters
 * (engine/loader.cpp:478, engine/decode_step.h:479,595). */
int q35_create(const q35_config* cfg, q35_engine** out);
int q35_destroy(q35_engine* e);
const char* q35_last_error(void);

/* Synthetic weights of the benchmark workload: matrices N(0,0.02), RMSNorm weights 1.0,
 * A_log = log U(1,16), dt_bias ~ U(-1,1), from the portable seeded stream. */
int q35_init_random(q35_engine* e, uint64_t seed);
/* Load one tensor given in checkpoint layout and dtype bf16 (row-major, the reference's
 * names, e.g. "model.language_model.layers.0.mlp.gate_proj.weight"); engine/loader.cpp:478. */
int q35_load_tensor(q35_engine* e, const char* name, const uint16_t* host_bf16, size_t n_elems);
/* Load a checkpoint given as the bytes of its .safetensors file (replaces specimpl.Weights,
 * speccheck/specimpl.py:60-127, and the engine's loader, engine/loader.cpp:478): the
 * model.visual.* tensors are skipped, every other tensor must be one of the 335 text-tower
 * and MTP tensors with its checkpoint shape, stored as BF16, F16 or F32 (cast to bf16 with
 * round-to-nearest-even, as torch's .to(torch.bfloat16)); the file must hold 488 tensors, 153
 * of them vision (the reference's G0 gate). The tied lm_head reads the embedding. Nothing is
 * written unless the whole file passes. n_loaded / n_skipped (nullable) receive 335 / 153. */
int q35_load_safetensors(q35_engine* e, const void* file_bytes, size_t n_bytes, int32_t* n_loaded,
                         int32_t* n_skipped);
/* Parse and validate a .safetensors container without an engine (no GPU work): tensor count
 * and how many are model.visual.* (the same header checks as q35_load_safetensors). */
int q35_safetensors_scan(const void* file_bytes, size_t n_bytes, int32_t* n_tensors, int32_t* n_vision);
/* Read a tensor back in checkpoint layout (tests). */
int q35_read_tensor(q35_engine* e, const char* name, uint16_t* host_bf16, size_t n_elems);

/* Request state.  allocate_state / free_state / reset (engine/state.h:101,115-116). */
int q35_state_alloc(q35_engine* e, int lanes, int cap, int mtp_k, int mtp_cap, q35_state** out);
int q35_state_free(q35_engine* e, q35_state* s);
int q35_state_reset(q35_engine* e, q35_state* s, const int32_t* lanes, int n);
/* Seeded state of the batched benchmark: S ~ N(0,0.1) f32, K/V ~ N(0,1) bf16 (slots
 * [0, prefix_len)), window zero, prefix_len as given, for every lane. */
int q35_state_seed(q35_engine* e, q35_state* s, uint64_t seed, int prefix_len);
int q35_state_prefix_len(q35_engine* e, q35_state* s, int lane, int32_t* out);
/* Copy one lane's tensors to host: which = 0 S [18][16][128][128] f32, 1 window
 * [18][3][6144] f32, 2 keys [6][2][n][256] bf16 (first n slots), 3 values, 4 MTP keys
 * [2][n][256], 5 MTP values. */
int q35_state_read(q35_engine* e, q35_state* s, int lane, int which, int n_slots, void* host, size_t bytes);
int q35_state_write(q35_engine* e, q35_state* s, int lane, int which, int n_slots, const void* host, size_t bytes);

/* Prefix reuse and preempt / resume (specification/08-state-management.md §08.3-08.4: the
 * tuple is stored and restored verbatim, no recompute). q35_state_copy_lane forks lane
 * src_lane's tuple -- its current GDN S and conv window, K/V slots [0, prefix_len), the MTP
 * cache, the last post-final-norm row and prefix_len -- device-to-device into dst_lane (of
 * the same or another state of this engine; the destination's capacity must hold it). The
 * snapshot is one contiguous host blob of the same tuple (q35_state_snapshot with host ==
 * NULL reports its size in *bytes_needed); q35_state_restore writes it back into any lane. */
int q35_state_copy_lane(q35_engine* e, q35_state* src, int src_lane, q35_state* dst, int dst_lane);
int q35_state_snapshot(q35_engine* e, q35_state* s, int lane, void* host, size_t bytes, size_t* bytes_needed);
int q35_state_restore(q35_engine* e, q35_state* s, int lane, const void* host, size_t bytes);

/* Prompt of one lane (prefill_wave, engine/prefill.cpp:63 / specimpl.py:457-464): the
 * tokens are consumed in waves of at most max_rows rows; *y0 = greedy id after the last
 * prompt token; logits (nullable) receives that row's 248320 bf16-valued logits. */
int q35_prefill(q35_engine* e, q35_state* s, int lane, const int32_t* ids, int n, int32_t* y0,
                float* logits);

/* Prompts of n lanes at once (the batched form of prefill_wave, engine/prefill.cpp:63, which takes
 * one request): lane lanes[i] (i when NULL) consumes ids[off_i .. off_i + lens[i]) with off_i the
 * sum of the lens before it; rows of different lanes share each body pass (rounds of at most
 * max_rows rows, the same row count for every lane of a round); y0[i] = greedy id after lane i's
 * last prompt token; logits (nullable) [n][248320] that row's logits. Each lane ends as after
 * q35_prefill of its own prompt (the same kernels for prompts under 64 tokens: bit-identical;
 * a single lane takes q35_prefill's waves). */
int q35_prefill_lanes(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* ids,
                      const int32_t* lens, int32_t* y0, float* logits);

/* The same prompt with every row priced (prefill_wave with PrefillLogits::kAll,
 * engine/prefill.h:46-58,116-118, the reference's byte-identity gate mode): sampled[i] = greedy
 * id (lowest id on ties) of prompt row i, top_logit[i] (nullable) = that id's bf16-valued
 * logit, logits (nullable) = [n][248320] f32. The state advances exactly as q35_prefill's
 * (same waves, same kernels); the extra cost is one lm_head pass per row. */
int q35_prefill_all(q35_engine* e, q35_state* s, int lane, const int32_t* ids, int n, int32_t* sampled,
                    float* top_logit, float* logits);

/* One greedy decode step for n lanes (decode_step, engine/decode_step.h:582): lane
 * lanes[i] (or i when lanes is NULL) consumes tokens[i]; out_tok[i] = argmax (lowest id on
 * ties) of the bf16 logits; out_logits (nullable) is [n][248320]. */
int q35_decode_step(q35_engine* e, q35_state* s, const int32_t* lanes, int n,
                    const int32_t* tokens, int32_t* out_tok, float* out_logits);

/* MTP draft (mtpdraft::draft_round, engine/mtp_draft.h:233 / speccheck/mtp.py:57-83):
 * for each lane i, draft the token at position pos[i] from token y[i] and hidden h
 * (h_dev == NULL: the post-final-norm row the last body left for that lane). Appends one
 * entry to the lane's MTP K/V.  out_xd (nullable, host [n][1024] bf16) receives x_d. */
int q35_mtp_draft(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* y,
                  const int32_t* pos, int step, int32_t* out_tok, uint16_t* out_xd,
                  float* out_logits);

/* One speculative round (greedy_mtp body, speccheck/mtp.py:150-177 with k drafts): per
 * lane, k drafts from (cur, h), a (k+1)-row verify body over [cur, d1..dk] writing the GDN
 * state after every row to spare slots, greedy accept of the longest matching prefix a,
 * rollback (state slot after row a, prefix_len = p + a + 1, MTP K/V truncated when a < k).
 * emit[i][0..n_emit[i]) = accepted drafts + bonus token; stats (nullable, [4]) accumulates
 * drafted, accepted, bonus, target rows. */
int q35_mtp_round(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                  int k, int32_t* emit, int32_t* n_emit, int64_t* stats);

/* The same round with the session driver's stop rule (mtpaccept::session_body,
 * engine/mtp_accept.h:422-431, engine/mtp_accept.cpp:585-600): when an accepted draft equals
 * `stop` (>= 0; 248046 in the session), the accepted prefix ends before it, so that token
 * is the lane's last emit and stays pending (printed, never fed) -- the state ends where the
 * transcript does, as after a plain step that sampled it. stop < 0 is q35_mtp_round. */
int q35_mtp_round_stop(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                       int k, int32_t stop, int32_t* emit, int32_t* n_emit, int64_t* stats);

/* The verify half of a round on drafts the caller made (mtpaccept::accept_round with its
 * candidates, engine/mtp_accept.h:248): drafts [n][k] (draft step j of lane i at i * k + j, as
 * q35_mtp_draft steps 0 .. k-1 made them, whose MTP K/V entries are then kept on a full accept);
 * the (k+1)-row verify body over [cur, drafts], accept, rollback, emit, n_emit, stop and stats as
 * in q35_mtp_round_stop. Drafts from elsewhere verify the same way (greedy verification is
 * lossless whatever the drafts); only the drafter's own cache assumes they came from it. */
int q35_mtp_verify(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur, int k,
                   const int32_t* drafts, int32_t stop, int32_t* emit, int32_t* n_emit, int64_t* stats);

/* Adaptive speculation depth (mtpadapt::Tracker, engine/mtp_adaptive.h:1-254): one policy per
 * request decides the depth of its next round -- 2, 1, or 0 (plain steps for the rest of the
 * request) -- from the tokens its own rounds emitted: the window estimate is emitted tokens per
 * step-equivalent over the last 32 rounds (a round at depth k billed cost_k plain steps; <= 0
 * selects the reference's 1.58 / 1.90); after 16 rounds at k = 2 an estimate below 0.95 demotes
 * to 1, after 24 rounds at k = 1 one below 0.90 abandons; the window clears on a change and
 * there is no re-promotion. Host-only; no GPU work. */
typedef struct q35_mtp_policy q35_mtp_policy;
int q35_mtp_policy_create(int start_k, double cost_k1, double cost_k2, q35_mtp_policy** out);
int q35_mtp_policy_free(q35_mtp_policy* p);
int q35_mtp_policy_k(const q35_mtp_policy* p, int32_t* k);
/* Feed one round (its depth and emitted token count). change (nullable, [3]) = {from, to, rounds
 * seen} when the depth changed, else {-1, -1, -1}; est (nullable) = the window estimate. */
int q35_mtp_policy_note(q35_mtp_policy* p, int k_round, int emitted, int32_t* change, double* est);
/* One turn of n lanes at their policies' depths: lanes at depth 2 run one k = 2 round together,
 * depth 1 one k = 1 round, depth 0 one plain decode step; every round's emitted count is fed to
 * its lane's policy. emit [n][3] (unused entries -1), n_emit [n], depth (nullable) [n] = the depth
 * each lane ran at; stop as in q35_mtp_round_stop; stats as in q35_mtp_round (rounds only). */
int q35_mtp_adaptive_step(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                          q35_mtp_policy* const* pol, int32_t stop, int32_t* emit, int32_t* n_emit,
                          int32_t* depth, int64_t* stats);

/* Per-op entry points on caller device buffers (benchmark and parity harness). */
/* Y[M][N] = X[M][K] . W^T with W in checkpoint row-major layout, tiled into scratch first
 * by q35_op_tile_weight. */
int q35_op_tile_weight(q35_engine* e, const uint16_t* w_rowmajor_dev, int N, int K, uint16_t* w_tiled_dev);
int q35_op_gemm(q35_engine* e, const uint16_t* w_tiled_dev, int N, int K, const uint16_t* x_dev,
                int M, uint16_t* y_dev);
/* One GatedDeltaNet decode step for B independent lanes (benchmark config 2; the layer's
 * conv + gates + L2 norms + delta rule, engine/kernels_gdn.cpp:35-536): proj [B][8224] bf16
 * (qkv 6144 | z 2048 | b 16 | a 16), conv_w [6144][4] bf16, A_log / dt_bias [16] bf16;
 * S2 [B][2][16][128][128] f32 and W2 [B][2][3][6144] f32 hold the input state in slot 0 and
 * receive the new state in slot 1; o [B][2048] f32 (before the gated norm). */
int q35_op_gdn_step(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                    const uint16_t* dt_bias, float* S2, float* W2, float* o, int B);
/* q35_op_gdn_step without any allocation, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops); it has no counterpart in the reference. Same arguments and
 * results; its scratch (the lane list, B ints) is a fixed per-GPU device array of 4,096 entries
 * held until the process ends, so B <= 4096 (larger B: Q35_ERR_CAP). Enqueued on the engine
 * stream without waiting (q35_sync waits). Calls of one engine are ordered on its stream; a call
 * by another engine on the same GPU while the last call there is unfinished would race on the
 * array and is refused (Q35_ERR_STATE): synchronise that engine first. */
int q35_op_gdn_step_noalloc(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                            const uint16_t* dt_bias, float* S2, float* W2, float* o, int B);
/* The same step with the layer's gated RMSNorm (engine/kernels_gdn.cpp:525, specimpl.py:142-147,
 * 304-305): y [B][2048] bf16 = bf16(w * (o * rsqrt(mean_head(o^2) + 1e-6)) * silu(z)) per
 * 128-wide head, with gnorm [128] bf16, made where the engine makes it for B lanes: in the
 * recurrence's epilogue for B > 64 (form 0: the persistent kernel; form 1: the non-persistent
 * whole-head kernel of the MTP verify path), by the out_proj GEMM's batched A producer for
 * B <= 64 (form 1: the whole-head kernel's epilogue instead). B <= max_rows. */
int q35_op_gdn_step_norm(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                         const uint16_t* dt_bias, const uint16_t* gnorm, float* S2, float* W2, float* o,
                         uint16_t* y, int B, int form);
/* Y[M][N] = A . W^T with A made by one of the GEMM's A producers from X (and X2): amode 0 A = X
 * (bf16 [M][K]); 1 SwiGLU A = bf16(bf16(silu(X)) * X2) (X, X2 bf16 [M][K]); 2 gated RMSNorm
 * A = bf16(aux_w * (X * rsqrt(mean_head(X^2) + 1e-6)) * silu(X2)) (X f32 [M][K], X2 bf16 z,
 * aux_w [128]); 3 A = X through the many-row kernel (K = 1024, 17 <= M <= max_rows: X is tiled into
 * the engine's staging, then the GEMM prompt waves of >= 512 rows use); 5 A = X with the batched
 * SwiGLU epilogue, Y [M][N/2] = bf16(bf16(silu(bf16(X.Wg^T))) * bf16(X.Wu^T)) for W = [gate; up];
 * 6 the same through the many-row kernel. M <= 16 uses the one-row GEMM's in-register producer,
 * M > 16 the batched one. */
int q35_op_gemm_a(q35_engine* e, const uint16_t* w_tiled_dev, int N, int K, int amode, const void* x_dev, int ldx,
                  const void* x2_dev, int ldx2, const uint16_t* aux_dev, int M, uint16_t* y_dev);
/* One gated GQA attention layer of the decode path on a state's K/V cache (attn_decode_layer,
 * engine/kernels_attn.cpp:415; speccheck/specimpl.py:320-397): for lane i = lanes[i] (i when
 * NULL), T rows at positions p_i .. p_i + T - 1 (p_i = pos[i], or the lane's prefix_len when pos
 * is NULL; the lane's prefix_len is not changed). proj_dev [n*T][5120] bf16 holds the attention
 * input projection rows in the engine's order ((q | gate) per q head x 8, k x 2, v x 2, 256
 * each); q_norm_dev / k_norm_dev [256] bf16. Each row's q and k get the zero-centred RMSNorm and
 * partial rope (64 dims, theta 1e7, position p_i + t); bf16(k) and v are written into attention
 * layer `layer`'s cache slots p_i + t; each row attends causally over slots 0 .. p_i + t with
 * scale 1/16, and out_dev [n*T][2048] bf16 = bf16(bf16(softmax . V) * sigmoid(gate)), the input
 * of o_proj. form: 0 the engine's choice for the shape, 1 split (one-wave score, P.V and combine
 * kernels), 2 split in 4-wave score / dim-quarter P.V blocks, 3 fused, 4 fused with two items per
 * block (T = 1), 5 one block per (lane, kv head) for all T = 2 or 3 rows, 6 flash prompt form
 * (one lane, T >= 64); a form the shape cannot take is Q35_ERR_ARG. Synchronous. */
int q35_op_attn_decode(q35_engine* e, q35_state* s, int layer, const int32_t* lanes, const int32_t* pos, int n,
                       int T, const uint16_t* proj_dev, const uint16_t* q_norm_dev, const uint16_t* k_norm_dev,
                       uint16_t* out_dev, int form);
int q35_op_lm_head_argmax(q35_engine* e, const uint16_t* x_dev, int M, int32_t* tok_dev, float* logits_dev);
int q35_sync(q35_engine* e);
/* Live per-kernel timing: with option "kprof" = family (1 projection/MLP GEMMs, 2 lm_head
 * GEMM, 3 GDN recurrence, 4 attention core, 0 off), each launch of that family is bracketed
 * by HIP events on the engine stream; this returns the summed duration and launch count
 * since the option was set or last read, and resets them. */
int q35_kprof_read(q35_engine* e, float* total_ms, int* launches);
/* Options: "layers" (diagnostic: bodies run only the first n of the 24 layers, the final
 * norm then applies to that layer's output), "graph" (0/1: capture decode steps), "kprof"
 * (above), "gdn_chunked" (0/1: chunked GDN form for prompt waves of >= 64 rows). Kernel-form
 * switches of this engine only (each engine holds its own; setting one drops the engine's
 * captured steps), each bit-identical to its alternative and kept for A/B measurement:
 * "b1_partials" (one-row bodies leave k-block chains for the next norm GEMV), "gemv_tpb" (1/2
 * column tiles per block of the one-row norm GEMVs), "gemm_pre" (batched K = 1024 GEMMs; 0: k-block
 * pipelined, 1: all loads issued up front, in 64 x 128 blocks when those fit the CUs in one
 * round, else 32 x 64; 2: always 64 x 128), "lmhead_persist" (lm_head at batched lanes: 0 tiled, 1 persistent with A in LDS, 3 -- the
 * default -- persistent with A in registers and a running argmax per column stream), "partial_rows"
 * (>= 17: batched out/o/down GEMMs with at least this many rows sum their k-block chains in
 * the block, one chain for the add+norm; default 1,024), "attn_split4" (split attention path
 * in 4-wave score blocks and dim-quarter P.V blocks), "attn_pair" (default 1: the fused
 * attention of one row per lane at batched lanes runs two (row, kv head) items per block when
 * their LDS fits the CU, so the two items on a CU finish together), "attn_rows" (default 1: MTP
 * verify bodies of 2-3 rows per lane at >= 128 lanes run one attention block per (lane, kv
 * head) for all of the lane's rows, streaming its K/V once), "gdn_rows" (default 1: those verify
 * bodies' GDN layers in the persistent kernel, the next (lane, head) item prefetched),
 * "gdn_defer" (0 .. 4, default 3: a decode
 * step keeps each lane's GDN state update as pending factors for up to this many steps and
 * writes the state with the next one; 0 writes it every step). Not bit-identical, a different
 * rounding point within the stated tolerance: "attn_prompt" (1: prompt waves of one lane with
 * >= 64 rows use the flash-form MFMA attention kernel, 0: the one-row kernels); "prompt_exact" (1:
 * prompt waves run the decode step's arithmetic -- the one-row attention kernels and the recurrent
 * GDN kernel -- so a prompt is byte-identical to feeding its tokens one decode step at a time,
 * the reference's own equivalence for its prefill wave, engine/prefill.h:5-9; 0: the flash
 * attention and chunked GDN forms, the default, equal to it within the stated tolerance). */
int q35_set_option(q35_engine* e, const char* name, int value);
/* Copy the current content of a named scratch buffer ("x", "h", "nrm", "delta", "proj",
 * "o", "gu", "aout", "q") to host, after the stream drains (diagnostics and tests). */
int q35_read_scratch(q35_engine* e, const char* name, void* host, size_t bytes);
/* Timing of the engine stream with HIP events: begin/end bracket; elapsed in ms. */
int q35_timer_begin(q35_engine* e);
int q35_timer_end(q35_engine* e, float* ms);

#ifdef __cplusplus
}
#endif
#endif
