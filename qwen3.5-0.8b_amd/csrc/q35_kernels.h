// Internal launcher interface between the engine (q35_engine.cpp) and the device code.
// Raw device pointers, no synchronisation; every launcher returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q35 {

enum { kAPlain = 0, kASiluMul = 1, kAGatedNorm = 2, kANormX = 3, kANormXP = 4 };
enum { kEStore = 0, kEArgmax = 1, kEPartial = 2, kEResidual = 3, kESiluMul = 4 };
// kESiluMul (batched lanes): N = 2F columns [gate | up]; each block pairs gate tiles with the
// matching up tiles and stores act = bf16(bf16(silu(bf16 g)) * bf16 u) into Y [M][F].

// Kernel-form choices of one engine (q35_set_option), each bit-identical to its alternative
// except attn_prompt (a different rounding point within the stated tolerance). They travel
// with the launch arguments, so engines of one process never see each other's settings.
struct KernelForms {
    int gemv_tpb = 2;          // one-row norm GEMVs (N >= 4096): column tiles per block, 1 or 2
    int gemm_pre = 1;          // batched K = 1024 GEMMs: all loads up front (1) or k-block pipelined (0)
    int lmhead_persist = 3;    // tied lm_head at batched lanes: 64 x 256 tiles (0), persistent with A in LDS
                               // (1), persistent with A in registers, the weights through an LDS ring
                               // and one argmax partial per (row, column stream) (3)
    int partial_rows = 1024;   // batched kEPartial GEMMs with M >= this leave one (summed) chain
    int attn_split4 = 1;       // split attention path: 4-wave score blocks, P.V split over dim quarters
    int attn_pair = 1;         // fused attention, one row per lane: two (row, kv head) items per block
    int attn_rows = 2;         // MTP verify (2-3 rows per lane) at >= 128 lanes: one block per (lane, kv head)
                               // (1: 4 waves, two blocks per CU; 2: 8 waves, one per CU, a larger LDS tail)
    int attn_prompt = 1;       // prompt waves of >= 64 rows: flash-form MFMA kernel (1) or one-row kernels (0)
    int mid_partials = 1;      // bodies of 2 .. 16 rows: k-block chains + add+norm (0: residual-epilogue GEMMs)
    int gdn_rows = 1;          // MTP verify (2-3 rows per lane, whole-head blocks): the persistent GDN kernel
    int gemm_wide = 1;         // K = 1024 GEMMs of >= 512 rows: 256 x 128 tiles through an LDS ring, A tiled
    int gdn_defer = 3;         // decode steps: a lane's GDN state update is kept as pending factors for up
                               // to this many steps, the state written on the next (0: every step)
};

struct GemmArgs {
    const uint16_t* W;     // tiled [N/16][K/256] x 8 KiB
    int N, K, M;
    const void* X;         // A source (bf16; f32 o for kAGatedNorm; residual x for kANormX)
    int ldx;
    const void* X2;        // second source: u (kASiluMul) or z (kAGatedNorm)
    int ldx2;
    const uint16_t* aux_w; // gated-norm weight [128] / RMSNorm weight [1024] (kANormX)
    uint16_t* Y;           // kEStore output
    int ldy;
    float* logits;         // kEArgmax: optional f32 copy of the bf16 logits
    int ldl;
    float* part_val;       // kEArgmax: per-(row, tile) max
    int* part_idx;
    int ldp;
    float* kpart;          // kEPartial: k-block chains [K/256][M][N] f32
    uint16_t* prod;        // M > 16 with a producer: bf16 [M][K] staging of the produced A
    uint16_t* xres;        // kEResidual: residual rows [M][1024], x <- bf16(x + bf16(sum))
    uint16_t* hout;        // kANormX (optional): the normalised rows [M][1024] are written here
    int kpb;               // kANormXP: k-block chains of the producing GEMM pending in kpart
    int x_tiled;           // X in the weights' tiled fragment layout (tiled_offset, rows as n): the
                           // many-row K = 1024 GEMM (gemm_wide); M rows padded to whole 16-row tiles
    int y_tiled;           // gemm_wide's SwiGLU epilogue: Y in that tiled layout (K = ldy) for a
                           // consumer that reads it as x_tiled (the many-row full-K down projection)
    KernelForms forms;
};
// One-time kernel attribute setup (dynamic LDS above 64 KiB for the batch-1 producers).
hipError_t gemm_init();
// k-block chains a batched kEPartial GEMM leaves in kpart
int gemm_partial_chains(int M, int K, const KernelForms& f);
hipError_t launch_gemm(const GemmArgs& a, int amode, int emode, hipStream_t st);
// the many-row full-K residual projection (gemm_wide64<kEPartial>, A tiled) takes an M-row GEMM
bool wide_fullk(const KernelForms& f, int M);
// kEArgmax: how many (max, index) partials per row the launch for `a` writes (launch_argmax's n)
int gemm_argmax_partials(const GemmArgs& a);
// The batched A producer alone: a.prod [M][K] bf16 = the producer's A operand (kASiluMul or
// kAGatedNorm), as launch_gemm stages it for M > 16.
hipError_t launch_produce(const GemmArgs& a, int amode, hipStream_t st);
hipError_t launch_argmax(const float* pv, const int* pi, int ldp, int n, int rows, int* tok,
                         float* val, hipStream_t st);

// Row metadata of one engine call: rows are grouped by lane, T consecutive rows per lane.
struct RowMeta {
    const int* lane;       // [R] state lane of the row
    const int* pos;        // [R] rope position
    const int* slot;       // [R] cache slot written by this row; the row attends to slots [0, slot]
};

// Residual add + zero-centred RMSNorm (specimpl.py:135-139, pairing :426-451).
//   mode 0: x = E[tok[r]];  mode 1: x = bf16(x + delta);  mode 2: x unchanged;
//   mode 3: x = bf16(x + bf16(sum_kb kpart[kb][r]));  mode 4: x = bf16(sum_kb kpart[kb][r])
//   (k-block chains summed in k-block order, the GEMM's canonical reduction)
//   then h = rmsnorm_zc(x, w) (skipped when h == nullptr)
hipError_t launch_addnorm(int mode, const int* tok, const uint16_t* E, uint16_t* x,
                          const uint16_t* delta, const float* kpart, int kblocks,
                          const uint16_t* w, uint16_t* h, int rows, hipStream_t st,
                          int h_tiled = 0);
// MTP fc input: cat[rmsnorm_zc(E[tok], we) | rmsnorm_zc(hin, wh)] -> out [rows][2048]
hipError_t launch_mtp_concat(const int* tok, const uint16_t* E, const uint16_t* hin, int ldh,
                             const uint16_t* we, const uint16_t* wh, uint16_t* out, int rows,
                             hipStream_t st);

struct GdnArgs {
    const uint16_t* proj;      // [R][8224]: qkv | z | b | a
    float* o;                  // [R][2048] f32 output (pre gated-norm)
    const uint16_t* conv_w;    // [6144][4]
    const uint16_t* A_log;     // [16]
    const uint16_t* dt_bias;   // [16]
    // State S f32 [16][128][128] and conv window f32 [3][6144] of (lane, slot, layer) at
    // base + lane*X_lane + slot*X_slot + X_layer (element offsets).
    float* S;
    long long S_lane, S_slot, S_layer;
    float* win;
    long long W_lane, W_slot, W_layer;
    const int* cur;            // [R] state slot of each row's lane (null: slot 0)
    const int* wcur;           // [R] conv window slot of each row's lane (null: = cur)
    int nslots;
    int ckpt;                  // 0: state after the last row -> slot (cur + 1) % nslots, window
                               //    -> slot (wcur + 1) % nslots;
                               // 1: window after row t -> slot (wcur + 1 + t) % nslots, and the
                               //    state after every row as factors (below) if fac_write, else
                               //    the state after row t -> slot (cur + 1 + t) % nslots
    // Pending rank-1 updates (MTP verify rows): the state of a lane is the one in slot `cur`
    // followed by its pending rows p = 0 .. n-1, each S = e^g S; S += k~ dv^T with the
    // recorded f32 (gamma, k~, dv) -- the same two rounded operations as the recurrence, so
    // replaying them gives the verify kernel's bits. pend[r] = n | (set << 4); fac points at
    // this layer's factors of lane 0, set 0, row 0: [lane][set][layer][row][head][kFacStride].
    const int* pend;           // [R] (null: none pending)
    float* fac;
    long long fac_lane, fac_set, fac_row;
    int fac_write;             // ckpt: write row t's factors into set 1 - (pending set), keep no
                               // per-row state; a lane with pending rows first has them
                               // applied and the result stored to slot (cur + 1) % nslots
    int defer;                 // decode rows (T = 1, ckpt = 0): a lane with n < defer pending rows
                               // records this row as pending row n of its own set (factors) and
                               // keeps slot cur; otherwise its state goes to slot (cur + 1) % nslots
    const int* lane;           // [R] state lane of each row
    int T;                     // rows per lane (rows of one lane are consecutive)
    int nlanes;
    // Optional fused gated RMSNorm (whole-head blocks and the chunked form's output kernel):
    // y[r][h*128 + j] = bf16(w[j] * (o * rsqrt(mean_head(o^2) + eps)) * silu(z)), bf16 [R][2048]
    uint16_t* y;
    const uint16_t* gnorm;     // [128]
    int y_tiled;               // chunked form: y in the GEMMs' tiled fragment layout (K = 2048)
    // Chunked prompt form (one lane, no checkpoints): per-(chunk, head) workspace and decays,
    // and the wave's post-conv SiLU values [T][6144] bf16
    float* chunk_ws;
    float* chunk_cdec;
    uint16_t* conv_u;
};
hipError_t launch_gdn(const GdnArgs& a, int col_slices, hipStream_t st);
// Chunked (UT-transform, chunk 64) form over the T rows of one lane: same state/window slot
// semantics as launch_gdn without checkpoints; o only (the gated norm is the consumer's).
hipError_t launch_gdn_chunked(const GdnArgs& a, hipStream_t st);
size_t gdn_chunk_ws_floats(int max_rows);
// Persistent whole-head form for one decode row per lane (T = 1, ckpt = 0): the same bits
// as launch_gdn(a, 1, st), with the next item's state prefetched into LDS.
hipError_t launch_gdn_persist(const GdnArgs& a, hipStream_t st);
hipError_t gdn_init();     // one-time kernel attribute setup
constexpr int kFacStride = 264;   // per (row, head): k~ [128] | dv [128] | gamma | pad
constexpr int kMaxDefer = 4;      // factor rows per set available to deferred decode rows
constexpr int kMaxPend = 5;       // pending rows a lane can hold (MTP verify: k + 1 <= 5 rows)
// Applies the pending rows of n lanes to their states: for each row r < n (lanes lane[r],
// slots cur[r], pend[r] as in GdnArgs), every GDN layer's state in slot cur -> slot (cur + 1)
// % nslots. fac points at lane 0, set 0, layer 0, row 0; fac_layer is the layer stride.
hipError_t launch_gdn_materialize(float* S, long long S_lane, long long S_slot, const int* lane, const int* cur,
                                  const int* pend, const float* fac, long long fac_lane, long long fac_set,
                                  long long fac_layer, long long fac_row, int nslots, int n, hipStream_t st);

struct AttnArgs {
    const uint16_t* proj;  // [R][5120]: (q|gate) x 8 heads interleaved, k, v
    const uint16_t* q_norm;    // [256]
    const uint16_t* k_norm;    // [256]
    uint16_t* kc;          // key cache base: lane stride kv_lane, layer at + kv_layer_off, [2][cap][256]
    uint16_t* vc;
    long long kv_lane, kv_layer_off;
    int cap;
    RowMeta rm;
    float* q;              // scratch [R][8][256] f32 post-rope q
    float* sc;             // scratch scores [R][8][sc_ld]
    int sc_ld;
    float* stats;          // scratch [R][8][4 * max_chunks][2] (64-slot slices)
    float* part;           // scratch [R][2 * max_chunks][8][256] (128-slot parts)
    int max_chunks;
    uint16_t* out;         // [R][2048] gated attention output (input of o_proj)
    int out_tiled;         // attn_prompt only: out in the GEMMs' tiled fragment layout (K = 2048)
    int R;
    int T;                 // rows per lane (a lane's rows are consecutive; MTP verify: k + 1)
    const float* inv_freq; // [32] f32 rope inverse frequencies
    int prompt_flash;      // KernelForms::attn_prompt of the calling engine
    int split4;            // KernelForms::attn_split4: split path in 4-wave score / dim-split P.V blocks
    int fused_pair;        // KernelForms::attn_pair
    int rows_form;         // KernelForms::attn_rows
    int force;             // 0: the form chosen from the shape; else one form (AttnForce), for
                           // the op-level parity harness; a form the shape cannot take is an error
};
enum AttnForce { kAttnAuto = 0, kAttnSplit = 1, kAttnSplit4 = 2, kAttnFused = 3, kAttnFusedPair = 4,
                 kAttnRows = 5, kAttnPrompt = 6 };
hipError_t launch_attn_prep(const AttnArgs& a, hipStream_t st);   // q/k norm + rope, cache append
hipError_t launch_attn_core(const AttnArgs& a, hipStream_t st);   // scores, softmax, P.V, gate
bool attn_form_ok(const AttnArgs& a);     // the forced form (AttnArgs::force) can run this shape
bool attn_prompt_form(const AttnArgs& a); // launch_attn_core runs attn_prompt (honours out_tiled)
hipError_t attn_init();   // one-time kernel attribute setup

// Synthetic init (portable stream, see q35_init.hip).
hipError_t launch_gen_normal_tiled(uint64_t key, float scale, int N, int K, int row_off_dst,
                                   uint16_t* dst, int Kdst, hipStream_t st);
hipError_t launch_gen_normal_kv_tiled(uint64_t key, float scale, int n_slots, uint16_t* dst, hipStream_t st);
hipError_t launch_gen_normal_kv_v8(uint64_t key, float scale, int n_slots, uint16_t* dst, hipStream_t st);
hipError_t launch_gen_normal_plain(uint64_t key, float scale, long long n, uint16_t* dst,
                                   hipStream_t st);
hipError_t launch_gen_normal_f32(uint64_t key, float scale, long long n, float* dst,
                                 hipStream_t st);

hipError_t launch_tile(const uint16_t* src, int N, int K, uint16_t* dst, int row_off, int inverse,
                       hipStream_t st);
hipError_t launch_copy_rows(const uint16_t* src, const int* src_rows, uint16_t* dst, const int* dst_rows,
                            int n, int width, hipStream_t st);
// The decode step's last kernel: copy rows src -> dst and advance each row's position, cache
// slot, state and window slots (cur, wcur) for the next step of the same lanes. With the
// step's `defer` (GdnArgs::defer) a row with n < defer pending rows keeps cur and has n + 1
// pending rows after the step; any other row moves cur to the next slot with none pending
// (the pending set bit is kept).
hipError_t launch_copy_rows_advance(const uint16_t* src, const int* src_rows, uint16_t* dst, const int* dst_rows,
                                    int n, int width, int* pos, int* slot, int* cur, int* wcur, int* pend, int nslots,
                                    int defer, hipStream_t st);

}  // namespace q35
