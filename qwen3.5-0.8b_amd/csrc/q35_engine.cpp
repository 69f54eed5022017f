// Engine host side and C ABI (include/q35.h).
//
// Follows the reference's decode order (engine/decode_step.cpp:448-1354, specification
// 07-decode-step.md:6-20): embed -> input norm -> 24 blocks (GDN or gated attention, then
// the MLP, with the residual add fused into the next norm) -> final norm -> tied lm_head ->
// greedy argmax. Every pass is a "body" over R rows = nlanes x T tokens; decode is T = 1,
// a prompt wave is one lane with T tokens, an MTP verify is T = k + 1.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/q35.h"
#include "q35_common.h"
#include "q35_kernels.h"
#include "q35_safetensors.h"

using namespace q35;

namespace {

thread_local std::string g_err;

struct Q35Error : std::runtime_error {
    int code;
    Q35Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HCK(x)                                                                              \
    do {                                                                                    \
        hipError_t _e = (x);                                                                \
        if (_e != hipSuccess)                                                               \
            throw Q35Error(Q35_ERR_HIP, std::string(#x) + ": " + hipGetErrorString(_e));   \
    } while (0)
#define REQ(cond, code, msg)                                  \
    do {                                                      \
        if (!(cond)) throw Q35Error((code), (msg));           \
    } while (0)

uint64_t hmix(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (unsigned char c : s) { h ^= c; h *= 0x100000001B3ull; }
    return h;
}
uint64_t stream_key(uint64_t seed, const std::string& name) { return hmix(hmix(seed) + fnv1a64(name)); }
uint16_t h_f2bf(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

enum Kind { kNormal, kOne, kAlog, kDtBias };

// Where a checkpoint tensor lives on the device.
struct Placement {
    uint16_t* base = nullptr;  // plain: the tensor; tiled: the combined matrix
    int rows = 0, cols = 0;    // logical shape (cols = K for matrices; 1-D: rows = n, cols = 1)
    bool tiled = false;
    int row_off = 0;           // tiled: first row inside the combined matrix
    Kind kind = kNormal;
};

struct LayerW {
    uint16_t *norm_in, *norm_post, *W_in, *W_out, *W_gu, *W_down;
    uint16_t *conv_w, *A_log, *dt_bias, *gnorm;   // GDN
    uint16_t *q_norm, *k_norm;                     // attention
};

}  // namespace

struct q35_state {
    int lanes = 0, cap = 0, mtp_cap = 0, nslots = 2, mtp_k = 0;
    int capT = 0, mtp_capT = 0;   // K/V region strides: capacities padded to whole 16-slot K tiles
    float* S = nullptr;      // [lanes][nslots][18][16][128][128]
    float* win = nullptr;    // [lanes][nslots][18][3][6144]
    uint16_t *kc = nullptr, *vc = nullptr;    // [lanes][6][2][cap][256]
    uint16_t *mkc = nullptr, *mvc = nullptr;  // [lanes][2][mtp_cap][256]
    uint16_t* hlast = nullptr;                // [lanes][1024] post-final-norm row of the last body
    // GDN state updates kept as factors (GdnArgs), MTP verify rows and deferred decode rows:
    // [lanes][2 sets][18][max(mtp_k + 1, kMaxDefer) rows][16 heads][kFacStride]
    float* fac = nullptr;
    // per lane: GDN state slot `cur`, conv window slot `wcur`, pending rows applied on top of
    // slot cur (`pend`, from factor set `pset`)
    std::vector<int> prefix, mtp_len, cur, wcur, pend, pset;
    long long fac_row() const { return (long long)kHv * kFacStride; }
    long long fac_layer() const { return (long long)std::max(mtp_k + 1, kMaxDefer) * fac_row(); }
    long long fac_set() const { return (long long)kGdnLayers * fac_layer(); }
    long long fac_lane() const { return 2 * fac_set(); }
    // the per-row encoding of a lane's pending rows (GdnArgs::pend)
    int pend_code(int l) const { return pend[l] | (pset[l] << 4); }
    long long S_lane() const { return (long long)nslots * kGdnLayers * kSLayer; }
    long long W_lane() const { return (long long)nslots * kGdnLayers * 18432; }
    long long kv_lane() const { return (long long)kAttnLayers * 2 * capT * 256; }
    long long mkv_lane() const { return (long long)2 * mtp_capT * 256; }
};

struct q35_engine {
    int device = 0, R = 0, max_ctx = 0, use_graph = 0;
    int n_layers = kLayers;          // diagnostic: run only the first n layers of a body
    int kprof = 0;                   // kernel family timed with HIP events (0 = off)
    int gdn_chunked = 1;             // prompt waves of one lane use the chunked GDN form
    int b1_partials = 1;             // one-row bodies: 1024-wide GEMVs leave k-block chains
    KernelForms forms;               // this engine's kernel-form choices (q35_set_option)
    float *gchunk = nullptr, *gcdec = nullptr;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> kev;
    size_t kev_used = 0;
    hipStream_t st = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipEvent_t noalloc_ev = nullptr;   // recorded after each allocation-free call of this engine
    uint16_t* blob = nullptr;
    size_t blob_bytes = 0;
    bool weights_ready = false;
    std::map<std::string, Placement> reg;
    std::vector<std::string> order;
    LayerW L[kLayers];
    LayerW M;                        // MTP block (attention layer shape)
    uint16_t *E = nullptr, *final_norm = nullptr, *mtp_pre_e = nullptr, *mtp_pre_h = nullptr,
             *mtp_fc = nullptr, *mtp_norm = nullptr;
    // scratch
    uint16_t *x, *h, *delta, *nrm, *proj, *gu, *aout, *cat;
    float *o, *q, *sc, *stats, *part, *pval, *inv_freq;
    float* kpart;
    uint16_t* prod;
    int *pidx, *tok_dev, *rlane, *rpos, *rslot, *rcur, *rwcur, *rpend, *ridx_src, *ridx_dst, *din = nullptr;
    int sc_ld = 0, max_chunks = 0;
    float* logits_dev = nullptr;
    int logits_rows = 0;
    float* topv_dev = nullptr;       // [R] the argmax's logit value per row (all-rows prefill)
    std::map<std::string, hipGraphExec_t> graphs;   // captured decode steps
    // pinned staging
    int *h_tok, *h_lane, *h_pos, *h_slot, *h_rcur, *h_rwcur, *h_rpend, *h_out, *h_src, *h_dst, *hin = nullptr;
    // Row metadata on the device (token, lane, position, slot, the state slot of the row's lane, row indices)
    // changes only by the uploads below, which bump meta_epoch, and by a decode step, which
    // advances positions, slots and `cur` on the device and leaves its sampled tokens in the
    // token row. The next decode step of the same state and lanes, fed exactly those tokens
    // with the host's prefix and `cur` still at the values the step left, needs no upload.
    // Every other call that changes a state's host prefix / cur or the device rows (reset,
    // seed, lane copy, restore, MTP rounds, allocation and release) bumps meta_epoch too.
    uint64_t meta_epoch = 0, fast_epoch = ~0ull;
    const void* fast_s = nullptr;
    std::vector<int> fast_lanes, fast_prefix, fast_cur, fast_wcur, fast_pend, fast_tok;
};

namespace {

// Kernel families for the live per-kernel timing (q35_set_option "kprof").
enum KFam { kFamNone = 0, kFamGemm = 1, kFamLmHead = 2, kFamGdn = 3, kFamAttn = 4, kFamGlue = 5 };

struct KTimer {
    q35_engine* e;
    bool on;
    KTimer(q35_engine* e_, int fam) : e(e_), on(e_->kprof == fam) {
        if (!on) return;
        if (e->kev_used == e->kev.size()) {
            hipEvent_t a, b;
            HCK(hipEventCreate(&a));
            HCK(hipEventCreate(&b));
            e->kev.push_back({a, b});
        }
        HCK(hipEventRecord(e->kev[e->kev_used].first, e->st));
    }
    ~KTimer() {
        if (on) {
            hipEventRecord(e->kev[e->kev_used].second, e->st);
            ++e->kev_used;
        }
    }
};

template <typename T>
T* dalloc(size_t n) {
    void* p = nullptr;
    HCK(hipMalloc(&p, n * sizeof(T) > 0 ? n * sizeof(T) : 16));
    return (T*)p;
}
template <typename T>
T* halloc(size_t n) {
    void* p = nullptr;
    HCK(hipHostMalloc(&p, n * sizeof(T) > 0 ? n * sizeof(T) : 16, hipHostMallocDefault));
    return (T*)p;
}

// Blocking copy ordered on the engine stream (the stream is non-blocking, so null-stream
// copies would not be ordered with its kernels).
void copy_sync(q35_engine* e, void* dst, const void* src, size_t n, hipMemcpyKind kind) {
    HCK(hipMemcpyAsync(dst, src, n, kind, e->st));
    HCK(hipStreamSynchronize(e->st));
}

// ------------------------------------------------------------------ allocation-free GDN step
// q35_op_gdn_step_noalloc's only scratch (the row -> lane index list of its rows) lives in this
// file-scope device array: one copy per GPU, held until the process ends, shared by every
// call on that GPU. In host code `scratch` names a host-side stand-in, so its device address
// is looked up once per device (at q35_create, with the device current) and only that
// address is ever passed to kernels.
constexpr int kNoAllocMaxLanes = 4096;
static __device__ __align__(256) int scratch[kNoAllocMaxLanes];
std::mutex g_scratch_mu;
std::map<int, int*> g_scratch_ptr;   // device ordinal -> device address of `scratch`

std::map<int, std::string> g_scratch_err;   // device ordinal -> why the lookup failed
// device ordinal -> the engine whose allocation-free call used the array last, and the event
// that engine records after each such call: another engine (another stream) is refused while
// that event is pending, instead of racing on the array
std::map<int, std::pair<const void*, hipEvent_t>> g_scratch_owner;

// Never fails the caller (q35_create): a failed lookup is recorded and reported by the
// allocation-free entry point, the only user of the array.
void init_noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr.count(device) || g_scratch_err.count(device)) return;
    int* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        g_scratch_err[device] = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(rc);
        return;
    }
    g_scratch_ptr[device] = p;
}

// The array of `device` for a call by `owner`, whose work will be followed on its stream by
// `ev`: refused while another owner's last call may still be running. The caller holds
// g_scratch_mu until it has enqueued its work and recorded `ev`.
int* noalloc_scratch(int device, const void* owner, hipEvent_t ev) {
    auto it = g_scratch_ptr.find(device);
    if (it == g_scratch_ptr.end()) {
        auto er = g_scratch_err.find(device);
        throw Q35Error(Q35_ERR_HIP, er != g_scratch_err.end() ? er->second : "scratch of this device was not set up");
    }
    auto ow = g_scratch_owner.find(device);
    if (ow != g_scratch_owner.end() && ow->second.first != owner) {
        const hipError_t q = hipEventQuery(ow->second.second);
        if (q == hipErrorNotReady)
            throw Q35Error(Q35_ERR_STATE, "the allocation-free scratch of this GPU is in use by another engine's "
                                          "unfinished call (calls on one GPU share it): wait for that engine first");
        (void)hipGetLastError();
    }
    g_scratch_owner[device] = {owner, ev};
    return it->second;
}

// An engine going away gives up its claim on the array.
void noalloc_release(int device, const void* owner) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto ow = g_scratch_owner.find(device);
    if (ow != g_scratch_owner.end() && ow->second.first == owner) g_scratch_owner.erase(ow);
}

__global__ void iota_kernel(int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = i;
}

// ------------------------------------------------------------------ weight registry
struct Planner {
    size_t off = 0;
    std::vector<std::pair<uint16_t**, size_t>> pending;
    void take(uint16_t** p, size_t elems) {
        pending.push_back({p, off});
        off += (elems * 2 + 255) / 256 * 256;
    }
};

void plan_weights(q35_engine* e) {
    Planner pl;
    auto& reg = e->reg;
    auto add_plain = [&](const std::string& n, uint16_t** slot, int rows, Kind k) {
        pl.take(slot, rows);
        Placement p;
        p.rows = rows; p.cols = 1; p.kind = k;
        reg[n] = p;
        e->order.push_back(n);
    };
    // tiled tensors are registered after allocation; remember (name, combined ptr, rows, K, off)
    struct TDef { std::string n; uint16_t** base; int rows, K, off; };
    std::vector<TDef> tdefs;
    auto add_tiled = [&](const std::string& n, uint16_t** base, int rows, int K, int off) {
        tdefs.push_back({n, base, rows, K, off});
        e->order.push_back(n);
    };
    auto attn_layer = [&](LayerW& w, const std::string& p, const std::string& sa) {
        pl.take(&w.W_in, (size_t)kAttnInRows * kHidden);
        add_tiled(sa + "q_proj.weight", &w.W_in, 4096, kHidden, 0);
        add_tiled(sa + "k_proj.weight", &w.W_in, 512, kHidden, kAttnKOff);
        add_tiled(sa + "v_proj.weight", &w.W_in, 512, kHidden, kAttnVOff);
        add_plain(sa + "q_norm.weight", &w.q_norm, 256, kOne);
        add_plain(sa + "k_norm.weight", &w.k_norm, 256, kOne);
        pl.take(&w.W_out, (size_t)kHidden * 2048);
        add_tiled(sa + "o_proj.weight", &w.W_out, kHidden, 2048, 0);
        (void)p;
    };
    auto mlp = [&](LayerW& w, const std::string& p) {
        pl.take(&w.W_gu, (size_t)kGuRows * kHidden);
        add_tiled(p + "gate_proj.weight", &w.W_gu, kFF, kHidden, 0);
        add_tiled(p + "up_proj.weight", &w.W_gu, kFF, kHidden, kFF);
        pl.take(&w.W_down, (size_t)kHidden * kFF);
        add_tiled(p + "down_proj.weight", &w.W_down, kHidden, kFF, 0);
    };
    for (int l = 0; l < kLayers; ++l) {
        LayerW& w = e->L[l];
        std::memset(&w, 0, sizeof(w));
        std::string pre = "model.language_model.layers." + std::to_string(l) + ".";
        add_plain(pre + "input_layernorm.weight", &w.norm_in, kHidden, kOne);
        add_plain(pre + "post_attention_layernorm.weight", &w.norm_post, kHidden, kOne);
        if (!is_attn_layer(l)) {
            std::string la = pre + "linear_attn.";
            pl.take(&w.W_in, (size_t)kGdnInRows * kHidden);
            add_tiled(la + "in_proj_qkv.weight", &w.W_in, kConvCh, kHidden, 0);
            add_tiled(la + "in_proj_z.weight", &w.W_in, 2048, kHidden, kGdnZOff);
            add_tiled(la + "in_proj_b.weight", &w.W_in, 16, kHidden, kGdnBOff);
            add_tiled(la + "in_proj_a.weight", &w.W_in, 16, kHidden, kGdnAOff);
            add_plain(la + "conv1d.weight", &w.conv_w, kConvCh * 4, kNormal);
            add_plain(la + "A_log", &w.A_log, 16, kAlog);
            add_plain(la + "dt_bias", &w.dt_bias, 16, kDtBias);
            add_plain(la + "norm.weight", &w.gnorm, 128, kOne);
            pl.take(&w.W_out, (size_t)kHidden * 2048);
            add_tiled(la + "out_proj.weight", &w.W_out, kHidden, 2048, 0);
        } else {
            attn_layer(w, pre, pre + "self_attn.");
        }
        mlp(w, pre + "mlp.");
    }
    pl.take(&e->E, (size_t)kVocab * kHidden);
    add_tiled("model.language_model.embed_tokens.weight", &e->E, kVocab, kHidden, 0);
    add_plain("model.language_model.norm.weight", &e->final_norm, kHidden, kOne);
    add_plain("mtp.pre_fc_norm_embedding.weight", &e->mtp_pre_e, kHidden, kOne);
    add_plain("mtp.pre_fc_norm_hidden.weight", &e->mtp_pre_h, kHidden, kOne);
    pl.take(&e->mtp_fc, (size_t)kHidden * 2048);
    add_tiled("mtp.fc.weight", &e->mtp_fc, kHidden, 2048, 0);
    std::memset(&e->M, 0, sizeof(e->M));
    add_plain("mtp.layers.0.input_layernorm.weight", &e->M.norm_in, kHidden, kOne);
    attn_layer(e->M, "mtp.layers.0.", "mtp.layers.0.self_attn.");
    add_plain("mtp.layers.0.post_attention_layernorm.weight", &e->M.norm_post, kHidden, kOne);
    mlp(e->M, "mtp.layers.0.mlp.");
    add_plain("mtp.norm.weight", &e->mtp_norm, kHidden, kOne);

    e->blob_bytes = pl.off;
    HCK(hipMalloc(&e->blob, e->blob_bytes));
    for (auto& pp : pl.pending) *pp.first = (uint16_t*)((char*)e->blob + pp.second);
    // plain placements: re-walk pointers in registration order (pending order == add order)
    // simpler: resolve by name below
    for (auto& t : tdefs) {
        Placement p;
        p.base = *t.base; p.rows = t.rows; p.cols = t.K; p.tiled = true; p.row_off = t.off; p.kind = kNormal;
        reg[t.n] = p;
    }
}

// plain placements need their pointers: build a name->pointer table after planning
void resolve_plain(q35_engine* e) {
    auto set = [&](const std::string& n, uint16_t* p) { e->reg.at(n).base = p; };
    for (int l = 0; l < kLayers; ++l) {
        LayerW& w = e->L[l];
        std::string pre = "model.language_model.layers." + std::to_string(l) + ".";
        set(pre + "input_layernorm.weight", w.norm_in);
        set(pre + "post_attention_layernorm.weight", w.norm_post);
        if (!is_attn_layer(l)) {
            std::string la = pre + "linear_attn.";
            set(la + "conv1d.weight", w.conv_w);
            set(la + "A_log", w.A_log);
            set(la + "dt_bias", w.dt_bias);
            set(la + "norm.weight", w.gnorm);
        } else {
            set(pre + "self_attn.q_norm.weight", w.q_norm);
            set(pre + "self_attn.k_norm.weight", w.k_norm);
        }
    }
    set("model.language_model.norm.weight", e->final_norm);
    set("mtp.pre_fc_norm_embedding.weight", e->mtp_pre_e);
    set("mtp.pre_fc_norm_hidden.weight", e->mtp_pre_h);
    set("mtp.layers.0.input_layernorm.weight", e->M.norm_in);
    set("mtp.layers.0.self_attn.q_norm.weight", e->M.q_norm);
    set("mtp.layers.0.self_attn.k_norm.weight", e->M.k_norm);
    set("mtp.layers.0.post_attention_layernorm.weight", e->M.norm_post);
    set("mtp.norm.weight", e->mtp_norm);
}

void alloc_scratch(q35_engine* e) {
    const size_t R = e->R;
    e->x = dalloc<uint16_t>(R * kHidden);
    e->h = dalloc<uint16_t>((R + 15) / 16 * 16 * kHidden);   // whole 16-row tiles (tiled layout)
    e->delta = dalloc<uint16_t>(R * kHidden);
    e->nrm = dalloc<uint16_t>(R * kHidden);
    e->proj = dalloc<uint16_t>(R * kGdnInRows);
    e->gu = dalloc<uint16_t>(R * kGuRows);
    e->aout = dalloc<uint16_t>(R * 2048);
    e->cat = dalloc<uint16_t>(R * 2048);
    e->o = dalloc<float>(R * 2048);
    e->q = dalloc<float>(R * kNq * 256);
    e->sc_ld = (e->max_ctx + 255) / 256 * 256;
    e->max_chunks = e->sc_ld / 256;
    e->sc = dalloc<float>(R * kNq * (size_t)e->sc_ld);
    e->stats = dalloc<float>(R * kNq * (size_t)e->max_chunks * 8);
    e->part = dalloc<float>(R * (size_t)e->max_chunks * 4 * kNq * 256);
    e->pval = dalloc<float>(R * (size_t)(kVocab / 16));
    e->pidx = dalloc<int>(R * (size_t)(kVocab / 16));
    e->kpart = dalloc<float>(R * 16 * kHidden);
    e->topv_dev = dalloc<float>(R);
    e->gchunk = dalloc<float>(gdn_chunk_ws_floats(R));
    e->gcdec = dalloc<float>((size_t)((R + 63) / 64) * kHv);
    e->prod = dalloc<uint16_t>(R * kFF);
    // row metadata: one device block and one pinned host block,
    // [tok|lane|pos|slot|cur|wcur|pend|src|dst] with stride R, so a step's inputs go up in a
    // single copy; cur / wcur / pend are the GDN state slot, window slot and pending verify
    // rows of the row's lane (read together with the lane, so the GDN kernels' addresses wait
    // for one load, not two dependent ones)
    e->din = dalloc<int>(9 * (size_t)R);
    e->hin = halloc<int>(9 * (size_t)R);
    int* d[9];
    int* hh[9];
    for (int i = 0; i < 9; ++i) { d[i] = e->din + (size_t)i * R; hh[i] = e->hin + (size_t)i * R; }
    e->tok_dev = d[0]; e->rlane = d[1]; e->rpos = d[2]; e->rslot = d[3]; e->rcur = d[4]; e->rwcur = d[5];
    e->rpend = d[6]; e->ridx_src = d[7]; e->ridx_dst = d[8];
    e->h_tok = hh[0]; e->h_lane = hh[1]; e->h_pos = hh[2]; e->h_slot = hh[3]; e->h_rcur = hh[4]; e->h_rwcur = hh[5];
    e->h_rpend = hh[6]; e->h_src = hh[7]; e->h_dst = hh[8];
    e->h_out = halloc<int>(R);
    // rope inverse frequencies, f32 as the oracle forms them (specimpl.py:151-156):
    // inv_i = 1 / f32(theta ** f32(2i/64))
    float invf[32];
    for (int i = 0; i < 32; ++i) {
        float ex = (float)(2 * i) / 64.0f;
        float pw = (float)std::pow(1e7, (double)ex);
        invf[i] = 1.0f / pw;
    }
    e->inv_freq = dalloc<float>(32);
    copy_sync(e, e->inv_freq, invf, sizeof(invf), hipMemcpyHostToDevice);
}

void ensure_logits(q35_engine* e, int rows) {
    if (e->logits_rows >= rows) return;
    if (e->logits_dev) {
        // captured graphs hold the old pointer
        HCK(hipStreamSynchronize(e->st));
        for (auto& kv : e->graphs) hipGraphExecDestroy(kv.second);
        e->graphs.clear();
        HCK(hipFree(e->logits_dev));
    }
    e->logits_dev = dalloc<float>((size_t)rows * kVocab);
    e->logits_rows = rows;
}

// ------------------------------------------------------------------ body pass
// Row metadata must already be staged in e->h_lane/h_pos/h_slot/h_tok for R rows.
// One copy of the metadata block from tok through region `upto` (rows [0, n) of it).
void upload_meta(q35_engine* e, int upto, int n) {
    ++e->meta_epoch;
    HCK(hipMemcpyAsync(e->din, e->hin, ((size_t)upto * e->R + n) * sizeof(int), hipMemcpyHostToDevice, e->st));
}
void upload_rows(q35_engine* e, int R) { upload_meta(e, 6, R); }   // tok, lane, pos, slot, cur, wcur, pend
// src / dst row indices only (tok_dev may hold device-written tokens): one copy
void upload_idx(q35_engine* e, int n) {
    ++e->meta_epoch;
    HCK(hipMemcpyAsync(e->ridx_src, e->h_src, ((size_t)e->R + n) * sizeof(int), hipMemcpyHostToDevice, e->st));
}

// Per-row state slots and pending rows from the lanes' host values (rows staged in h_lane).
void stage_rcur(q35_engine* e, q35_state* s, int R) {
    for (int r = 0; r < R; ++r) {
        const int l = e->h_lane[r];
        e->h_rcur[r] = s->cur[l];
        e->h_rwcur[r] = s->wcur[l];
        e->h_rpend[r] = s->pend_code(l);
    }
}

// After a body without checkpoints over these lanes: both slots advance, nothing pending.
void advance_lane(q35_state* s, int l) {
    s->cur[l] = (s->cur[l] + 1) % s->nslots;
    s->wcur[l] = (s->wcur[l] + 1) % s->nslots;
    s->pend[l] = 0;
}
// After a decode step run with `defer` (the host side of copy_rows_advance_kernel): a lane
// with fewer than `defer` pending rows gained one (its state slot stays), else its state moved.
void advance_decode(q35_state* s, int l, int defer) {
    if (s->pend[l] < defer) {
        s->pend[l] += 1;
        s->wcur[l] = (s->wcur[l] + 1) % s->nslots;
    } else {
        advance_lane(s, l);
    }
}
// The deferral depth of a decode step (GdnArgs::defer), bounded by the factor rows per set.
int step_defer(const q35_engine* e) { return std::min(std::max(e->forms.gdn_defer, 0), kMaxDefer); }

// Applies pending verify rows to the states of these lanes (before host reads, copies and the
// chunked prompt form, which take a state slot as it stands).
void materialize(q35_engine* e, q35_state* s, const std::vector<int>& lanes) {
    std::vector<int> ls;
    for (int l : lanes)
        if (s->pend[l] > 0) ls.push_back(l);
    if (ls.empty()) return;
    const int n = (int)ls.size();
    REQ(n <= e->R, Q35_ERR_CAP, "too many lanes to materialize at once");
    HCK(hipStreamSynchronize(e->st));
    for (int i = 0; i < n; ++i) { e->h_lane[i] = ls[i]; }
    stage_rcur(e, s, n);
    upload_meta(e, 6, n);
    HCK(launch_gdn_materialize(s->S, s->S_lane(), (long long)kGdnLayers * kSLayer, e->rlane, e->rcur, e->rpend, s->fac,
                               s->fac_lane(), s->fac_set(), s->fac_layer(), s->fac_row(), s->nslots, n, e->st));
    HCK(hipStreamSynchronize(e->st));
    for (int l : ls) { s->cur[l] = (s->cur[l] + 1) % s->nslots; s->pend[l] = 0; }
}

// Y != nullptr: bf16 store; Y == nullptr: k-block chains to e->kpart (summed by the next
// add+norm); emode kEResidual: x <- bf16(x + bf16(sum)) (batch-1 path).
void gemm(q35_engine* e, const uint16_t* W, int N, int K, int M, const void* X, int ldx,
          uint16_t* Y, int ldy, int amode = kAPlain, const void* X2 = nullptr, int ldx2 = 0,
          const uint16_t* aux = nullptr, int emode = -1, uint16_t* xres = nullptr, bool x_tiled = false,
          bool y_tiled = false) {
    GemmArgs a{};
    a.W = W; a.N = N; a.K = K; a.M = M; a.X = X; a.ldx = ldx; a.X2 = X2; a.ldx2 = ldx2; a.x_tiled = x_tiled ? 1 : 0;
    a.y_tiled = y_tiled ? 1 : 0;
    a.aux_w = aux; a.Y = Y; a.ldy = ldy;
    a.kpart = e->kpart; a.prod = e->prod; a.xres = xres; a.forms = e->forms;
    KTimer kt(e, kFamGemm);
    HCK(launch_gemm(a, amode, emode >= 0 ? emode : (Y ? kEStore : kEPartial), e->st));
}

// Batch-1 path (<= 16 rows): the residual add lives in the producing GEMM's epilogue and the
// RMSNorm in the consuming GEMM's A operand, so no add+norm launches remain.
inline bool small_rows(int R) { return R <= 16; }
// Whether the K = 1024 GEMM of width N over R normed rows takes them in the weights' tiled
// fragment layout (the producing add+norm writes e->h so) and runs gemm_wide: bodies of >= 512
// rows (prompt waves, MTP verify at many lanes, 256-row tiles) and batched lanes of 17 .. 511
// rows (64-row tiles) except the GDN in_proj, whose 65 column blocks x 4 row blocks at 256 rows
// would not fit the 256 CUs in one round (gemm_pre instead: 13.9 against 13.7 us in two rounds).
inline bool wide_for(const q35_engine* e, int R, int N) {
    return e->forms.gemm_wide && R > 16 && (R >= 512 || N != kGdnInRows);
}
inline int in_rows(int l) { return is_attn_layer(l) ? kAttnInRows : kGdnInRows; }

// One-row bodies (a batch-1 decode step, a one-token prompt): the 1024-wide GEMVs (out_proj,
// o_proj, down) run one wave per (column tile, k-block) and leave their k-block chains in
// e->kpart (8x or 14x the blocks of the residual-epilogue form, whose 64 blocks use a quarter
// of the CUs); the next norm GEMM folds them into the residual row (kANormXP) and writes the
// new row to the other buffer of a pair; the final add+norm folds the last layer's chains.
inline bool b1_partials(const q35_engine* e, int R, int T, bool ckpt) {
    return e->b1_partials && R == 1 && T == 1 && !ckpt;
}
// Bodies of 2 .. 16 rows (MTP verify at batch 1, short prompt waves, a few lanes): the same
// one-wave-per-(column tile, k-block) chains, folded by the add+norm kernel of the batched path
// (one launch for all rows: a GEMM producer per row would repeat the fold in every block), the
// norm GEMMs then taking the normed rows as plain A. 10.2 -> ~4.5 + 3 us for down at 3 rows.
inline bool mid_partials(const q35_engine* e, int R) { return e->forms.mid_partials && R > 1 && small_rows(R); }
// Whether the body leaves the final-normed rows in e->nrm (else the lm_head applies the norm).
inline bool body_final_normed(const q35_engine* e, int R, int T, bool ckpt) {
    return !small_rows(R) || b1_partials(e, R, T, ckpt) || mid_partials(e, R);
}
struct B1Res {
    uint16_t* cur;     // residual row as of the last fold
    uint16_t* alt;     // receives the next fold
    int pend = 0;      // k-block chains pending in e->kpart
    bool mid = false;  // 2 .. 16 rows: chains folded by the add+norm kernel into e->x (in place)
};

// RMSNorm GEMM of the residual row: folds pending chains first (one-row bodies).
void norm_gemm(q35_engine* e, B1Res* rr, const uint16_t* W, int N, int R, uint16_t* Y, int ldy,
               const uint16_t* normw) {
    if (!rr || (rr->mid && !rr->pend)) {
        gemm(e, W, N, kHidden, R, e->x, kHidden, Y, ldy, kANormX, nullptr, 0, normw);
        return;
    }
    if (rr->mid) {
        HCK(launch_addnorm(3, nullptr, nullptr, e->x, nullptr, e->kpart, rr->pend, normw, e->h, R, e->st));
        rr->pend = 0;
        gemm(e, W, N, kHidden, R, e->h, kHidden, Y, ldy);
        return;
    }
    GemmArgs a{};
    a.W = W; a.N = N; a.K = kHidden; a.M = 1; a.X = rr->cur; a.ldx = kHidden;
    a.aux_w = normw; a.Y = Y; a.ldy = ldy; a.forms = e->forms;
    int amode = kANormX;
    if (rr->pend) {
        amode = kANormXP;
        a.kpart = e->kpart; a.kpb = rr->pend; a.xres = rr->alt;
        std::swap(rr->cur, rr->alt);
        rr->pend = 0;
    }
    KTimer kt(e, kFamGemm);
    HCK(launch_gemm(a, amode, kEStore, e->st));
}

// A 1024-wide output projection feeding the residual: epilogue add (<= 16 rows), k-block
// chains for the next fold (one-row bodies) or chains for the add+norm kernel (batched).
void resid_gemm(q35_engine* e, B1Res* rr, const uint16_t* W, int K, int R, const void* X, int ldx,
                int amode = kAPlain, const void* X2 = nullptr, int ldx2 = 0, const uint16_t* aux = nullptr,
                bool x_tiled = false) {
    if (rr) {
        REQ(rr->pend == 0, Q35_ERR_STATE, "unfolded k-block chains");
        gemm(e, W, kHidden, K, R, X, ldx, nullptr, 0, amode, X2, ldx2, aux, kEPartial);
        rr->pend = K / 256;
    } else {
        gemm(e, W, kHidden, K, R, X, ldx, nullptr, 0, amode, X2, ldx2, aux, small_rows(R) ? kEResidual : -1, e->x,
             x_tiled);
    }
}

void attention_layer(q35_engine* e, const LayerW& w, int R, uint16_t* kc, uint16_t* vc,
                     long long kv_lane, long long layer_off, int cap, int T = 1, B1Res* rr = nullptr) {
    if (small_rows(R))
        norm_gemm(e, rr, w.W_in, kAttnInRows, R, e->proj, kAttnInRows, w.norm_in);
    else
        gemm(e, w.W_in, kAttnInRows, kHidden, R, e->h, kHidden, e->proj, kAttnInRows, kAPlain, nullptr, 0, nullptr, -1,
             nullptr, wide_for(e, R, kAttnInRows));
    AttnArgs a{};
    a.proj = e->proj; a.q_norm = w.q_norm; a.k_norm = w.k_norm;
    a.kc = kc; a.vc = vc; a.kv_lane = kv_lane; a.kv_layer_off = layer_off; a.cap = cap;
    a.rm.lane = e->rlane; a.rm.pos = e->rpos; a.rm.slot = e->rslot;
    a.q = e->q; a.sc = e->sc; a.sc_ld = e->sc_ld; a.stats = e->stats; a.part = e->part;
    a.max_chunks = (cap + 255) / 256;
    REQ(a.max_chunks <= e->max_chunks, Q35_ERR_CAP, "cache capacity exceeds engine max_ctx");
    a.out = e->aout; a.R = R; a.T = T; a.inv_freq = e->inv_freq; a.prompt_flash = e->forms.attn_prompt;
    a.split4 = e->forms.attn_split4;
    a.fused_pair = e->forms.attn_pair;
    a.rows_form = e->forms.attn_rows;
    // a prompt wave's o_proj in the many-row full-K form: attn_prompt writes its output tiled
    const bool tiled = !rr && wide_fullk(e->forms, R) && attn_prompt_form(a);
    a.out_tiled = tiled ? 1 : 0;
    HCK(launch_attn_prep(a, e->st));
    {
        KTimer kt(e, kFamAttn);      // the attention core alone (scores, softmax, P.V, gate)
        HCK(launch_attn_core(a, e->st));
    }
    resid_gemm(e, rr, w.W_out, 2048, R, e->aout, 2048, kAPlain, nullptr, 0, nullptr, tiled);
}

// MLP sub-block; on the batched path it leaves chains that `finish_norm` folds in.
void mlp_layer(q35_engine* e, const LayerW& w, int R, B1Res* rr = nullptr) {
    if (small_rows(R)) {
        norm_gemm(e, rr, w.W_gu, kGuRows, R, e->gu, kGuRows, w.norm_post);
        resid_gemm(e, rr, w.W_down, kFF, R, e->gu, kGuRows, kASiluMul, e->gu + kFF, kGuRows);
        return;
    }
    HCK(launch_addnorm(3, nullptr, nullptr, e->x, nullptr, e->kpart, gemm_partial_chains(R, 2048, e->forms), w.norm_post, e->h, R, e->st,
                       wide_for(e, R, kGuRows)));
    // gate|up GEMM with the SwiGLU product in its epilogue: act [R][3584] -> plain down GEMM;
    // prompt waves of >= partial_rows rows: act in the tiled layout for the many-row full-K down
    const bool tiled = wide_fullk(e->forms, R);
    gemm(e, w.W_gu, kGuRows, kHidden, R, e->h, kHidden, e->gu, kFF, kAPlain, nullptr, 0, nullptr, kESiluMul, nullptr,
         wide_for(e, R, kGuRows), tiled);
    gemm(e, w.W_down, kHidden, kFF, R, e->gu, kFF, nullptr, 0, kAPlain, nullptr, 0, nullptr, -1, nullptr, tiled);
}

// Batched path: fold the down-projection chains into x and normalise for the next consumer (a
// K = 1024 GEMM of width next_n when out is e->h).
void finish_norm(q35_engine* e, int R, const uint16_t* nw, uint16_t* out, int next_n = 0) {
    if (small_rows(R)) return;
    HCK(launch_addnorm(3, nullptr, nullptr, e->x, nullptr, e->kpart, gemm_partial_chains(R, kFF, e->forms), nw, out, R, e->st,
                       out == e->h && wide_for(e, R, next_n)));
}

// Runs the 24-layer body over R = nl * T rows (rows of one lane consecutive) and leaves the
// final-normed rows in e->nrm. ckpt: write the GDN state after every row (MTP verify).
void body_kernels(q35_engine* e, q35_state* s, int R, int T, bool ckpt, int defer = 0);

void body(q35_engine* e, q35_state* s, int R, int T, bool ckpt) {
    REQ(e->weights_ready, Q35_ERR_STATE, "weights not initialised");
    REQ(R > 0 && R <= e->R, Q35_ERR_CAP, "rows exceed engine max_rows");
    if (R / T == 1 && e->gdn_chunked && !small_rows(R) && T >= 64 && !ckpt && s->pend[e->h_lane[0]] > 0) {
        // the chunked prompt form reads a state slot as it stands: apply the pending rows first
        std::vector<int> keep(e->h_lane, e->h_lane + R), pos(e->h_pos, e->h_pos + R), sl(e->h_slot, e->h_slot + R),
            tk(e->h_tok, e->h_tok + R);
        materialize(e, s, {keep[0]});
        std::copy(keep.begin(), keep.end(), e->h_lane);
        std::copy(pos.begin(), pos.end(), e->h_pos);
        std::copy(sl.begin(), sl.end(), e->h_slot);
        std::copy(tk.begin(), tk.end(), e->h_tok);
    }
    stage_rcur(e, s, R);
    upload_rows(e, R);
    body_kernels(e, s, R, T, ckpt);
}

// The launches of one body pass (no host transfers: capturable in a hipGraph). defer: a
// decode step's GDN deferral depth (T = 1, no checkpoints; GdnArgs::defer).
void body_kernels(q35_engine* e, q35_state* s, int R, int T, bool ckpt, int defer) {
    const int nl = R / T;
    const int cs = nl <= 8 ? 8 : nl <= 32 ? 4 : nl <= 64 ? 2 : 1;
    const bool small = small_rows(R);
    B1Res res{e->x, e->h};          // one-row bodies: e->h is the second residual buffer
    res.mid = mid_partials(e, R);   // 2 .. 16 rows: e->x folded in place, e->h the normed rows
    B1Res* rr = b1_partials(e, R, T, ckpt) || res.mid ? &res : nullptr;
    HCK(launch_addnorm(0, e->tok_dev, e->E, e->x, nullptr, nullptr, 0, e->L[0].norm_in, small ? nullptr : e->h,
                       R, e->st, !small && wide_for(e, R, in_rows(0))));
    for (int l = 0; l < e->n_layers; ++l) {
        const LayerW& w = e->L[l];
        if (!is_attn_layer(l)) {
            if (small)
                norm_gemm(e, rr, w.W_in, kGdnInRows, R, e->proj, kGdnInRows, w.norm_in);
            else
                gemm(e, w.W_in, kGdnInRows, kHidden, R, e->h, kHidden, e->proj, kGdnInRows, kAPlain, nullptr, 0, nullptr,
                     -1, nullptr, wide_for(e, R, kGdnInRows));
            GdnArgs g{};
            g.proj = e->proj; g.o = e->o; g.conv_w = w.conv_w; g.A_log = w.A_log; g.dt_bias = w.dt_bias;
            g.S = s->S; g.S_lane = s->S_lane(); g.S_slot = (long long)kGdnLayers * kSLayer;
            g.S_layer = (long long)gdn_slot(l) * kSLayer;
            g.win = s->win; g.W_lane = s->W_lane(); g.W_slot = (long long)kGdnLayers * 18432;
            g.W_layer = (long long)gdn_slot(l) * 18432;
            g.cur = e->rcur; g.wcur = e->rwcur; g.pend = e->rpend; g.nslots = s->nslots; g.ckpt = ckpt ? 1 : 0;
            g.fac = s->fac + (long long)gdn_slot(l) * s->fac_layer();
            g.fac_lane = s->fac_lane(); g.fac_set = s->fac_set(); g.fac_row = s->fac_row();
            g.fac_write = ckpt ? 1 : 0;
            g.defer = T == 1 && !ckpt ? defer : 0;
            g.lane = e->rlane; g.T = T; g.nlanes = nl;
            // a prompt wave of one lane: chunked (UT-transform) form
            const bool chunked = e->gdn_chunked && !small && nl == 1 && T >= 64 && !ckpt;
            const bool fused_norm = !small && cs == 1 && !chunked;   // whole-head blocks: norm in the GDN kernel
            if (fused_norm) { g.y = e->prod; g.gnorm = w.gnorm; }
            // the chunked form's output kernel applies the gated norm too (tiled for the many-row
            // full-K out_proj)
            const bool tiled = chunked && wide_fullk(e->forms, R);
            if (chunked) { g.y = e->prod; g.gnorm = w.gnorm; g.y_tiled = tiled ? 1 : 0; }
            g.chunk_ws = e->gchunk; g.chunk_cdec = e->gcdec; g.conv_u = e->gu;   // gu is free until the MLP
            {
                KTimer kt(e, kFamGdn);
                if (chunked) HCK(launch_gdn_chunked(g, e->st));
                else if (cs == 1 && T == 1 && !ckpt) HCK(launch_gdn_persist(g, e->st));
                else if (cs == 1 && ckpt && (T == 2 || T == 3) && e->forms.gdn_rows)
                    HCK(launch_gdn_persist(g, e->st));         // MTP verify rows, persistent
                else HCK(launch_gdn(g, cs, e->st));
            }
            if (fused_norm)
                gemm(e, w.W_out, kHidden, 2048, R, e->prod, 2048, nullptr, 0);
            else if (chunked)
                resid_gemm(e, rr, w.W_out, 2048, R, e->prod, 2048, kAPlain, nullptr, 0, nullptr, tiled);
            else
                resid_gemm(e, rr, w.W_out, 2048, R, e->o, 2048, kAGatedNorm, e->proj + kGdnZOff, kGdnInRows, w.gnorm);
        } else {
            attention_layer(e, w, R, s->kc, s->vc, s->kv_lane(),
                            (long long)attn_slot(l) * 2 * s->capT * 256, s->capT, T, rr);
        }
        mlp_layer(e, w, R, rr);
        const bool lastl = l + 1 == e->n_layers;
        const uint16_t* nw = lastl ? e->final_norm : e->L[l + 1].norm_in;
        finish_norm(e, R, nw, lastl ? e->nrm : e->h, lastl ? 0 : in_rows(l + 1));
    }
    // one-row body: the last layer's chains and the final norm in one add+norm launch; the
    // normed row is in e->nrm, so the caller's lm_head takes no norm weight
    if (rr) HCK(launch_addnorm(3, nullptr, nullptr, rr->cur, nullptr, e->kpart, rr->pend, e->final_norm, e->nrm,
                               rr->mid ? R : 1, e->st));
}

// lm_head + argmax over rows [row0, row0 + M); tokens into e->tok_dev[0..M). After a
// batched body the normed rows are in e->nrm; after a batch-1 body (`normw` given) the
// final RMSNorm of the residual rows is applied first.
void lm_head(q35_engine* e, int row0, int M, bool want_logits, const uint16_t* normw = nullptr,
             float* top_val = nullptr, const uint16_t* rows = nullptr) {
    GemmArgs a{};
    a.W = e->E; a.N = kVocab; a.K = kHidden; a.M = M; a.ldx = kHidden;
    a.X = (rows ? rows : e->nrm) + (size_t)row0 * kHidden;   // rows: final-normed rows given by the caller
    a.forms = e->forms;
    const int amode = kAPlain;
    if (normw)   // one small norm launch: cheaper than normalising in each of the 15,520 blocks
        HCK(launch_addnorm(2, nullptr, nullptr, e->x + (size_t)row0 * kHidden, nullptr, nullptr, 0, normw,
                           e->nrm + (size_t)row0 * kHidden, M, e->st));
    if (want_logits) { ensure_logits(e, M); a.logits = e->logits_dev; a.ldl = kVocab; }
    a.part_val = e->pval; a.part_idx = e->pidx; a.ldp = kVocab / 16;
    {
        KTimer kt(e, kFamLmHead);
        HCK(launch_gemm(a, amode, kEArgmax, e->st));
    }
    HCK(launch_argmax(e->pval, e->pidx, kVocab / 16, gemm_argmax_partials(a), M, e->tok_dev, top_val, e->st));
}

void save_hlast(q35_engine* e, q35_state* s, const std::vector<int>& src_rows, const std::vector<int>& lanes) {
    const int n = (int)src_rows.size();
    HCK(hipStreamSynchronize(e->st));
    for (int i = 0; i < n; ++i) { e->h_src[i] = src_rows[i]; e->h_dst[i] = lanes[i]; }
    upload_idx(e, n);
    HCK(launch_copy_rows(e->nrm, e->ridx_src, s->hlast, e->ridx_dst, n, kHidden, e->st));
}

void check_lane(q35_state* s, int lane) { REQ(lane >= 0 && lane < s->lanes, Q35_ERR_ARG, "lane out of range"); }
void check_tok(int t) { REQ(t >= 0 && t < kVocab, Q35_ERR_ARG, "token out of range"); }

// One MTP draft pass over n lanes (speccheck/mtp.py:57-83).  hsrc: [n][1024] device rows of
// h; tokens, pos staged by the caller in h_tok / h_pos; slots = mtp_len + step.
void mtp_draft_pass(q35_engine* e, q35_state* s, int n, const uint16_t* hsrc) {
    REQ(s->mtp_cap > 0, Q35_ERR_STATE, "state has no MTP cache");
    upload_rows(e, n);
    HCK(launch_mtp_concat(e->tok_dev, e->E, hsrc, kHidden, e->mtp_pre_e, e->mtp_pre_h, e->cat, n, e->st));
    if (small_rows(n)) {
        gemm(e, e->mtp_fc, kHidden, 2048, n, e->cat, 2048, e->x, kHidden);
    } else {
        gemm(e, e->mtp_fc, kHidden, 2048, n, e->cat, 2048, nullptr, 0);
        HCK(launch_addnorm(4, nullptr, nullptr, e->x, nullptr, e->kpart, gemm_partial_chains(n, 2048, e->forms), e->M.norm_in, e->h, n, e->st,
                           wide_for(e, n, kAttnInRows)));
    }
    attention_layer(e, e->M, n, s->mkc, s->mvc, s->mkv_lane(), 0, s->mtp_capT);
    mlp_layer(e, e->M, n);
    finish_norm(e, n, e->mtp_norm, e->nrm);
}

// One tensor in checkpoint layout (bf16 bits) into its placement: plain tensors are copied,
// matrices tiled into their combined GEMM operand.
void load_one(q35_engine* e, const std::string& name, const uint16_t* host, size_t n) {
    auto it = e->reg.find(name);
    REQ(it != e->reg.end(), Q35_ERR_ARG, "unknown tensor " + name);
    const Placement& p = it->second;
    REQ(n == (size_t)p.rows * p.cols, Q35_ERR_ARG, "element count mismatch: " + name);
    if (p.tiled) {
        uint16_t* tmp = dalloc<uint16_t>(n);
        copy_sync(e, tmp, host, n * 2, hipMemcpyHostToDevice);
        HCK(launch_tile(tmp, p.rows, p.cols, p.base, p.row_off, 0, e->st));
        HCK(hipStreamSynchronize(e->st));
        HCK(hipFree(tmp));
    } else {
        copy_sync(e, p.base, host, n * 2, hipMemcpyHostToDevice);
    }
}

// The checkpoint's shape of a registered tensor: [rows, K] for matrices, [n] for vectors,
// [6144, 1, 4] for the depthwise conv weights (specimpl.py:92-127, the G1 shape table).
bool shape_ok(const Placement& p, const std::string& name, const std::vector<int64_t>& sh) {
    if (p.tiled) return sh.size() == 2 && sh[0] == p.rows && sh[1] == p.cols;
    if (name.size() > 13 && name.compare(name.size() - 13, 13, "conv1d.weight") == 0)
        return sh.size() == 3 && sh[0] == kConvCh && sh[1] == 1 && sh[2] == 4;
    return sh.size() == 1 && sh[0] == p.rows;
}

int guard(const std::function<void()>& f) {
    try {
        f();
        return Q35_OK;
    } catch (const Q35Error& ex) {
        g_err = ex.what();
        return ex.code;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return Q35_ERR_STATE;
    }
}
}  // namespace

// The calling thread's error text, for the other translation units of the library (the MTP
// policy entry points) that return a status without going through guard().
void q35_set_error(const char* msg) { g_err = msg; }

// ====================================================================== C ABI
extern "C" {

const char* q35_last_error(void) { return g_err.c_str(); }

int q35_create(const q35_config* cfg, q35_engine** out) {
    return guard([&] {
        REQ(cfg && out, Q35_ERR_ARG, "null argument");
        REQ(cfg->max_rows > 0 && cfg->max_rows <= 65536, Q35_ERR_ARG, "max_rows out of range");
        REQ(cfg->max_ctx > 0 && cfg->max_ctx <= 262144, Q35_ERR_ARG, "max_ctx out of range");
        auto* e = new q35_engine();
        e->device = cfg->device; e->R = cfg->max_rows; e->max_ctx = cfg->max_ctx; e->use_graph = cfg->use_graph;
        HCK(hipSetDevice(e->device));
        init_noalloc_scratch(e->device);
        HCK(gemm_init());
        HCK(attn_init());
        HCK(gdn_init());
        HCK(hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking));
        HCK(hipEventCreate(&e->ev0));
        HCK(hipEventCreate(&e->ev1));
        HCK(hipEventCreateWithFlags(&e->noalloc_ev, hipEventDisableTiming));
        plan_weights(e);
        resolve_plain(e);
        alloc_scratch(e);
        *out = e;
    });
}

int q35_destroy(q35_engine* e) {
    return guard([&] {
        if (!e) return;
        hipStreamSynchronize(e->st);
        for (auto& kv : e->graphs) hipGraphExecDestroy(kv.second);
        e->graphs.clear();
        void* ds[] = {e->blob, e->x, e->h, e->delta, e->nrm, e->proj, e->gu, e->aout, e->cat, e->o, e->q,
                      e->sc, e->stats, e->part, e->pval, e->pidx, e->prod, e->din, e->inv_freq,
                      e->logits_dev, e->kpart, e->gchunk, e->gcdec, e->topv_dev};
        for (void* p : ds) if (p) hipFree(p);
        void* hs[] = {e->hin, e->h_out};
        for (void* p : hs) if (p) hipHostFree(p);
        noalloc_release(e->device, e);
        hipEventDestroy(e->ev0);
        hipEventDestroy(e->ev1);
        if (e->noalloc_ev) hipEventDestroy(e->noalloc_ev);
        hipStreamDestroy(e->st);
        delete e;
    });
}

int q35_init_random(q35_engine* e, uint64_t seed) {
    return guard([&] {
        REQ(e, Q35_ERR_ARG, "null engine");
        const float scale = (float)(0.02 / 65536.0);
        for (const auto& n : e->order) {
            const Placement& p = e->reg.at(n);
            const uint64_t key = stream_key(seed, n);
            if (p.kind == kNormal) {
                if (p.tiled) HCK(launch_gen_normal_tiled(key, scale, p.rows, p.cols, p.row_off, p.base, p.cols, e->st));
                else HCK(launch_gen_normal_plain(key, scale, p.rows, p.base, e->st));
            } else if (p.kind == kOne) {
                HCK(hipMemsetD16Async((hipDeviceptr_t)p.base, 0x3F80, p.rows, e->st));
            } else {
                std::vector<uint16_t> v(p.rows);
                for (int i = 0; i < p.rows; ++i) {
                    float u = (float)(hmix(key + 3ull * i) >> 40) * (1.0f / 16777216.0f);
                    double d = p.kind == kAlog ? std::log(1.0 + 15.0 * (double)u) : -1.0 + 2.0 * (double)u;
                    v[i] = h_f2bf((float)d);
                }
                HCK(hipMemcpyAsync(p.base, v.data(), v.size() * 2, hipMemcpyHostToDevice, e->st));
                HCK(hipStreamSynchronize(e->st));
            }
        }
        HCK(hipStreamSynchronize(e->st));
        e->weights_ready = true;
    });
}

int q35_load_tensor(q35_engine* e, const char* name, const uint16_t* host, size_t n) {
    return guard([&] {
        REQ(e && name && host, Q35_ERR_ARG, "null argument");
        load_one(e, name, host, n);
        e->weights_ready = true;
    });
}

int q35_safetensors_scan(const void* file, size_t n, int32_t* n_tensors, int32_t* n_vision) {
    return guard([&] {
        REQ(file && n_tensors && n_vision, Q35_ERR_ARG, "null argument");
        std::vector<StTensor> ts;
        std::string err;
        REQ(parse_safetensors(file, n, ts, err), Q35_ERR_ARG, "safetensors: " + err);
        int vis = 0;
        for (const auto& t : ts) vis += t.name.rfind("model.visual.", 0) == 0;
        *n_tensors = (int32_t)ts.size();
        *n_vision = vis;
    });
}

int q35_load_safetensors(q35_engine* e, const void* file, size_t n, int32_t* n_loaded, int32_t* n_skipped) {
    return guard([&] {
        REQ(e && file, Q35_ERR_ARG, "null argument");
        std::vector<StTensor> ts;
        std::string err;
        REQ(parse_safetensors(file, n, ts, err), Q35_ERR_ARG, "safetensors: " + err);
        // the reference loader's gate (specimpl.py:60-62, 88-91): 488 tensors, the 153
        // model.visual.* ones skipped, 335 loaded. Everything is checked before the first
        // tensor is written, so a refused file leaves the engine's weights as they were.
        std::vector<const StTensor*> keep;
        int skipped = 0;
        for (const auto& t : ts) {
            if (t.name.rfind("model.visual.", 0) == 0) { ++skipped; continue; }
            auto it = e->reg.find(t.name);
            REQ(it != e->reg.end(), Q35_ERR_ARG, "unknown tensor " + t.name);
            REQ(shape_ok(it->second, t.name, t.shape), Q35_ERR_ARG, "shape mismatch: " + t.name);
            REQ(t.dtype == "BF16" || t.dtype == "F32" || t.dtype == "F16", Q35_ERR_ARG,
                "tensor " + t.name + " has dtype " + t.dtype + " (BF16, F16 or F32 expected)");
            keep.push_back(&t);
        }
        REQ(ts.size() == 488 && skipped == 153 && keep.size() == e->reg.size(), Q35_ERR_ARG,
            "expected 488 tensors (153 vision, 335 text tower + MTP), found " + std::to_string(ts.size()) +
                " (" + std::to_string(skipped) + " vision)");
        std::vector<uint16_t> bits;
        for (const StTensor* t : keep) {      // casts as Tensor.to(torch.bfloat16) (specimpl.py:84)
            REQ(to_bf16(*t, bits, err), Q35_ERR_ARG, err);
            load_one(e, t->name, bits.data(), bits.size());
        }
        e->weights_ready = true;
        if (n_loaded) *n_loaded = (int32_t)keep.size();
        if (n_skipped) *n_skipped = skipped;
    });
}

int q35_read_tensor(q35_engine* e, const char* name, uint16_t* host, size_t n) {
    return guard([&] {
        REQ(e && name && host, Q35_ERR_ARG, "null argument");
        auto it = e->reg.find(name);
        REQ(it != e->reg.end(), Q35_ERR_ARG, std::string("unknown tensor ") + name);
        const Placement& p = it->second;
        REQ(n == (size_t)p.rows * p.cols, Q35_ERR_ARG, "element count mismatch");
        if (p.tiled) {
            uint16_t* tmp = dalloc<uint16_t>(n);
            HCK(launch_tile(p.base, p.rows, p.cols, tmp, p.row_off, 1, e->st));
            HCK(hipStreamSynchronize(e->st));
            copy_sync(e, host, tmp, n * 2, hipMemcpyDeviceToHost);
            HCK(hipFree(tmp));
        } else {
            HCK(hipStreamSynchronize(e->st));
            copy_sync(e, host, p.base, n * 2, hipMemcpyDeviceToHost);
        }
    });
}

int q35_state_alloc(q35_engine* e, int lanes, int cap, int mtp_k, int mtp_cap, q35_state** out) {
    return guard([&] {
        if (e) ++e->meta_epoch;           // a state buffer may reuse a freed address
        REQ(e && out, Q35_ERR_ARG, "null argument");
        REQ(lanes > 0 && lanes <= 65535 && cap > 0 && mtp_k >= 0 && mtp_k <= 4 && mtp_cap >= 0, Q35_ERR_ARG,
            "bad state shape");
        REQ(cap <= e->max_ctx && mtp_cap <= e->max_ctx, Q35_ERR_CAP, "cap exceeds engine max_ctx");
        auto* s = new q35_state();
        s->lanes = lanes; s->cap = cap; s->mtp_cap = mtp_cap; s->mtp_k = mtp_k;
        s->capT = kv_cap_padded(cap); s->mtp_capT = kv_cap_padded(mtp_cap);
        s->nslots = mtp_k > 0 ? mtp_k + 2 : 2;
        s->S = dalloc<float>((size_t)lanes * s->S_lane());
        s->win = dalloc<float>((size_t)lanes * s->W_lane());
        s->kc = dalloc<uint16_t>((size_t)lanes * s->kv_lane());
        s->vc = dalloc<uint16_t>((size_t)lanes * s->kv_lane());
        if (mtp_cap > 0) {
            s->mkc = dalloc<uint16_t>((size_t)lanes * s->mkv_lane());
            s->mvc = dalloc<uint16_t>((size_t)lanes * s->mkv_lane());
        }
        s->hlast = dalloc<uint16_t>((size_t)lanes * kHidden);
        s->fac = dalloc<float>((size_t)lanes * s->fac_lane());
        s->prefix.assign(lanes, 0);
        s->mtp_len.assign(lanes, 0);
        s->cur.assign(lanes, 0);
        s->wcur.assign(lanes, 0);
        s->pend.assign(lanes, 0);
        s->pset.assign(lanes, 0);
        // zeroed on the engine stream (non-blocking: a null-stream memset could still be
        // running when the first body's kernels start)
        HCK(hipMemsetAsync(s->S, 0, (size_t)lanes * s->S_lane() * 4, e->st));
        HCK(hipMemsetAsync(s->win, 0, (size_t)lanes * s->W_lane() * 4, e->st));
        HCK(hipMemsetAsync(s->hlast, 0, (size_t)lanes * kHidden * 2, e->st));
        HCK(hipStreamSynchronize(e->st));
        *out = s;
    });
}

int q35_state_free(q35_engine* e, q35_state* s) {
    return guard([&] {
        if (e) ++e->meta_epoch;           // a state buffer may reuse a freed address
        if (!s) return;
        if (e) {
            hipStreamSynchronize(e->st);
            char pre[64];
            std::snprintf(pre, sizeof pre, "dec:%p:", (void*)s);
            for (auto it = e->graphs.begin(); it != e->graphs.end();) {
                if (it->first.rfind(pre, 0) == 0) { hipGraphExecDestroy(it->second); it = e->graphs.erase(it); }
                else ++it;
            }
        }
        void* ds[] = {s->S, s->win, s->kc, s->vc, s->mkc, s->mvc, s->hlast, s->fac};
        for (void* p : ds) if (p) hipFree(p);
        delete s;
    });
}

int q35_state_reset(q35_engine* e, q35_state* s, const int32_t* lanes, int n) {
    return guard([&] {
        REQ(e && s, Q35_ERR_ARG, "null argument");
        HCK(hipStreamSynchronize(e->st));
        ++e->meta_epoch;                 // host prefix / cur change: the next step uploads
        for (int i = 0; i < (lanes ? n : s->lanes); ++i) {
            int l = lanes ? lanes[i] : i;
            check_lane(s, l);
            HCK(hipMemsetAsync(s->S + l * s->S_lane(), 0, s->S_lane() * 4, e->st));
            HCK(hipMemsetAsync(s->win + l * s->W_lane(), 0, s->W_lane() * 4, e->st));
            s->prefix[l] = 0; s->mtp_len[l] = 0; s->cur[l] = 0; s->wcur[l] = 0; s->pend[l] = 0; s->pset[l] = 0;
        }
        HCK(hipStreamSynchronize(e->st));
    });
}

int q35_state_seed(q35_engine* e, q35_state* s, uint64_t seed, int prefix_len) {
    return guard([&] {
        REQ(e && s, Q35_ERR_ARG, "null argument");
        REQ(prefix_len >= 0 && prefix_len < s->cap, Q35_ERR_CAP, "prefix_len must leave room in the cache");
        ++e->meta_epoch;
        const float s01 = (float)(0.1 / 65536.0), s1 = (float)(1.0 / 65536.0);
        for (int l = 0; l < s->lanes; ++l) {
            float* S0 = s->S + l * s->S_lane();   // slot 0
            HCK(launch_gen_normal_f32(stream_key(seed, "state.gdn." + std::to_string(l)), s01,
                                      (long long)kGdnLayers * kSLayer, S0, e->st));
            HCK(hipMemsetAsync(s->win + l * s->W_lane(), 0, s->W_lane() * 4, e->st));
            for (int a = 0; a < kAttnLayers; ++a)
                for (int j = 0; j < kNkv; ++j) {
                    size_t off = l * s->kv_lane() + ((size_t)(a * 2 + j) * s->capT) * 256;
                    std::string tag = std::to_string(l) + "." + std::to_string(a) + "." + std::to_string(j);
                    HCK(launch_gen_normal_kv_tiled(stream_key(seed, "state.k." + tag), s1, prefix_len, s->kc + off, e->st));
                    HCK(launch_gen_normal_kv_v8(stream_key(seed, "state.v." + tag), s1, prefix_len, s->vc + off, e->st));
                }
            s->prefix[l] = prefix_len; s->mtp_len[l] = 0; s->cur[l] = 0; s->wcur[l] = 0; s->pend[l] = 0; s->pset[l] = 0;
        }
        HCK(hipStreamSynchronize(e->st));
    });
}

int q35_state_prefix_len(q35_engine* e, q35_state* s, int lane, int32_t* out) {
    return guard([&] {
        REQ(e && s && out, Q35_ERR_ARG, "null argument");
        check_lane(s, lane);
        *out = s->prefix[lane];
    });
}

static void state_io(q35_engine* e, q35_state* s, int lane, int which, int n_slots, void* host,
                     size_t bytes, bool write) {
    REQ(e && s && host, Q35_ERR_ARG, "null argument");
    check_lane(s, lane);
    HCK(hipStreamSynchronize(e->st));
    auto cp = [&](void* dev, size_t off_bytes, size_t nb) {
        REQ(off_bytes + nb <= bytes, Q35_ERR_ARG, "host buffer too small");
        if (write) copy_sync(e, dev, (char*)host + off_bytes, nb, hipMemcpyHostToDevice);
        else copy_sync(e, (char*)host + off_bytes, dev, nb, hipMemcpyDeviceToHost);
    };
    if (which == 0) {
        if (!write) materialize(e, s, {lane});   // the state with its pending verify rows applied
        cp(s->S + lane * s->S_lane() + (long long)s->cur[lane] * kGdnLayers * kSLayer, 0, (size_t)kGdnLayers * kSLayer * 4);
        if (write) s->pend[lane] = 0;            // the written state replaces them
    } else if (which == 1) {
        cp(s->win + lane * s->W_lane() + (long long)s->wcur[lane] * kGdnLayers * 18432, 0, (size_t)kGdnLayers * 18432 * 4);
    } else if (which >= 2 && which <= 5) {
        // K / V caches: [heads][n_slots][256] bf16 row-major on the host; on the device K is
        // stored in 16-slot tiles (kv_tiled_offset) and V in 8-slot groups (kv_v8_offset),
        // converted here.
        const bool mtp = which >= 4, isk = which == 2 || which == 4;
        const int cap = mtp ? s->mtp_cap : s->cap, capT = mtp ? s->mtp_capT : s->capT;
        const int heads = mtp ? 2 : kAttnLayers * 2;
        REQ(!mtp || s->mtp_cap > 0, Q35_ERR_ARG, "state has no MTP cache");
        REQ(n_slots >= 0 && n_slots <= cap, Q35_ERR_ARG, "n_slots out of range");
        REQ((size_t)heads * n_slots * 512 <= bytes, Q35_ERR_ARG, "host buffer too small");
        uint16_t* base = (mtp ? (isk ? s->mkc : s->mvc) : (isk ? s->kc : s->vc)) +
                         lane * (mtp ? s->mkv_lane() : s->kv_lane());
        if (n_slots > 0) {
            const int nt = (n_slots + 15) / 16;      // whole 16-slot tiles (K) / pairs of 8-slot groups (V)
            std::vector<uint16_t> tiles((size_t)nt * 4096);
            uint16_t* h = (uint16_t*)host;
            auto off = [&](int t, int d) { return isk ? kv_tiled_offset(t, d) : kv_v8_offset(t, d); };
            for (int a = 0; a < heads; ++a) {
                uint16_t* dev = base + (size_t)a * capT * 256;
                if (write) {   // keep the padding slots of the last tile as they are on the device
                    copy_sync(e, tiles.data(), dev, tiles.size() * 2, hipMemcpyDeviceToHost);
                    for (int t = 0; t < n_slots; ++t)
                        for (int d = 0; d < 256; ++d) tiles[off(t, d)] = h[((size_t)a * n_slots + t) * 256 + d];
                    copy_sync(e, dev, tiles.data(), tiles.size() * 2, hipMemcpyHostToDevice);
                } else {
                    copy_sync(e, tiles.data(), dev, tiles.size() * 2, hipMemcpyDeviceToHost);
                    for (int t = 0; t < n_slots; ++t)
                        for (int d = 0; d < 256; ++d) h[((size_t)a * n_slots + t) * 256 + d] = tiles[off(t, d)];
                }
            }
        }
    } else {
        throw Q35Error(Q35_ERR_ARG, "unknown state tensor");
    }
}

// ---- whole-tuple copies: prefix reuse and preempt / resume (specification/08-state-management.md
// §08.3-08.4: the tuple S, conv window, KV[0..P), prefix_len is stored and restored verbatim)
// One lane's tuple, in the lane's current GDN slot: device-to-device into another lane.
static void copy_lane(q35_engine* e, q35_state* src, int sl, q35_state* dst, int dl) {
    check_lane(src, sl);
    check_lane(dst, dl);
    const int P = src->prefix[sl], M = src->mtp_len[sl];
    REQ(P <= dst->cap, Q35_ERR_CAP, "prefix exceeds the destination lane's cache capacity");
    REQ(dst->mtp_cap == 0 || M <= dst->mtp_cap, Q35_ERR_CAP, "MTP cache exceeds the destination's");
    if (src == dst && sl == dl) return;
    materialize(e, src, {sl});
    auto d2d = [&](void* d, const void* s_, size_t nb) {
        if (nb) HCK(hipMemcpyAsync(d, s_, nb, hipMemcpyDeviceToDevice, e->st));
    };
    const long long sS = (long long)kGdnLayers * kSLayer, sW = (long long)kGdnLayers * 18432;
    d2d(dst->S + dl * dst->S_lane() + dst->cur[dl] * sS, src->S + sl * src->S_lane() + src->cur[sl] * sS, sS * 4);
    d2d(dst->win + dl * dst->W_lane() + dst->wcur[dl] * sW, src->win + sl * src->W_lane() + src->wcur[sl] * sW, sW * 4);
    // K: whole 16-slot tiles, V: whole 8-slot groups (the slots past P of the last tile or
    // group are never read before written)
    const size_t ktile = (size_t)(P + 15) / 16 * 4096 * 2, vrows = (size_t)(P + 7) / 8 * 4096;
    for (int a = 0; a < kAttnLayers * 2; ++a) {
        d2d(dst->kc + dl * dst->kv_lane() + (size_t)a * dst->capT * 256,
            src->kc + sl * src->kv_lane() + (size_t)a * src->capT * 256, ktile);
        d2d(dst->vc + dl * dst->kv_lane() + (size_t)a * dst->capT * 256,
            src->vc + sl * src->kv_lane() + (size_t)a * src->capT * 256, vrows);
    }
    const int Mc = dst->mtp_cap > 0 && src->mtp_cap > 0 ? M : 0;
    for (int a = 0; a < 2 && Mc > 0; ++a) {
        d2d(dst->mkc + dl * dst->mkv_lane() + (size_t)a * dst->mtp_capT * 256,
            src->mkc + sl * src->mkv_lane() + (size_t)a * src->mtp_capT * 256, (size_t)(Mc + 15) / 16 * 4096 * 2);
        d2d(dst->mvc + dl * dst->mkv_lane() + (size_t)a * dst->mtp_capT * 256,
            src->mvc + sl * src->mkv_lane() + (size_t)a * src->mtp_capT * 256, (size_t)(Mc + 7) / 8 * 4096);
    }
    d2d(dst->hlast + (size_t)dl * kHidden, src->hlast + (size_t)sl * kHidden, kHidden * 2);
    HCK(hipStreamSynchronize(e->st));
    dst->prefix[dl] = P;
    dst->mtp_len[dl] = Mc;
    dst->pend[dl] = 0;
}

// Snapshot blob: a header, then S f32 [18][16][128][128], window f32 [18][3][6144], K and V
// bf16 [12][P][256] (row layout), MTP K and V bf16 [2][M][256], last hidden row bf16 [1024].
struct SnapHeader {
    char magic[8];               // "Q35SNAP1"
    int32_t prefix_len, mtp_len, gdn_layers, attn_layers;
    int64_t bytes;               // whole blob
    int32_t reserved[8];
};

static size_t snap_bytes(int P, int M) {
    return sizeof(SnapHeader) + (size_t)kGdnLayers * kSLayer * 4 + (size_t)kGdnLayers * 18432 * 4 +
           2 * (size_t)kAttnLayers * 2 * P * 512 + 2 * (size_t)2 * M * 512 + kHidden * 2;
}

static void snapshot_lane(q35_engine* e, q35_state* s, int lane, void* host, size_t bytes, size_t* need) {
    check_lane(s, lane);
    const int P = s->prefix[lane], M = s->mtp_cap > 0 ? s->mtp_len[lane] : 0;
    const size_t n = snap_bytes(P, M);
    if (need) *need = n;
    if (!host) return;
    REQ(bytes >= n, Q35_ERR_ARG, "host buffer too small for the snapshot");
    SnapHeader h{};
    std::memcpy(h.magic, "Q35SNAP1", 8);
    h.prefix_len = P; h.mtp_len = M; h.gdn_layers = kGdnLayers; h.attn_layers = kAttnLayers; h.bytes = (int64_t)n;
    char* p = (char*)host;
    std::memcpy(p, &h, sizeof h);
    size_t off = sizeof h;
    const size_t nS = (size_t)kGdnLayers * kSLayer * 4, nW = (size_t)kGdnLayers * 18432 * 4;
    const size_t nKV = (size_t)kAttnLayers * 2 * P * 512, nM = (size_t)2 * M * 512;
    state_io(e, s, lane, 0, 0, p + off, nS, false); off += nS;
    state_io(e, s, lane, 1, 0, p + off, nW, false); off += nW;
    state_io(e, s, lane, 2, P, p + off, nKV, false); off += nKV;
    state_io(e, s, lane, 3, P, p + off, nKV, false); off += nKV;
    if (M > 0) {
        state_io(e, s, lane, 4, M, p + off, nM, false); off += nM;
        state_io(e, s, lane, 5, M, p + off, nM, false); off += nM;
    }
    copy_sync(e, p + off, s->hlast + (size_t)lane * kHidden, kHidden * 2, hipMemcpyDeviceToHost);
}

static void restore_lane(q35_engine* e, q35_state* s, int lane, const void* host, size_t bytes) {
    check_lane(s, lane);
    REQ(bytes >= sizeof(SnapHeader), Q35_ERR_ARG, "snapshot too short");
    SnapHeader h;
    std::memcpy(&h, host, sizeof h);
    REQ(std::memcmp(h.magic, "Q35SNAP1", 8) == 0 && h.gdn_layers == kGdnLayers && h.attn_layers == kAttnLayers,
        Q35_ERR_ARG, "not a snapshot of this engine's state layout");
    const int P = h.prefix_len, M = h.mtp_len;
    REQ(P >= 0 && M >= 0 && h.bytes == (int64_t)snap_bytes(P, M) && bytes >= (size_t)h.bytes, Q35_ERR_ARG,
        "snapshot size does not match its header");
    REQ(P <= s->cap, Q35_ERR_CAP, "snapshot prefix exceeds the lane's cache capacity");
    REQ(M == 0 || M <= s->mtp_cap, Q35_ERR_CAP, "snapshot MTP cache exceeds the state's");
    char* p = (char*)host;
    size_t off = sizeof h;
    const size_t nS = (size_t)kGdnLayers * kSLayer * 4, nW = (size_t)kGdnLayers * 18432 * 4;
    const size_t nKV = (size_t)kAttnLayers * 2 * P * 512, nM = (size_t)2 * M * 512;
    state_io(e, s, lane, 0, 0, p + off, nS, true); off += nS;
    state_io(e, s, lane, 1, 0, p + off, nW, true); off += nW;
    state_io(e, s, lane, 2, P, p + off, nKV, true); off += nKV;
    state_io(e, s, lane, 3, P, p + off, nKV, true); off += nKV;
    if (M > 0) {
        state_io(e, s, lane, 4, M, p + off, nM, true); off += nM;
        state_io(e, s, lane, 5, M, p + off, nM, true); off += nM;
    }
    copy_sync(e, s->hlast + (size_t)lane * kHidden, p + off, kHidden * 2, hipMemcpyHostToDevice);
    s->prefix[lane] = P;
    s->mtp_len[lane] = s->mtp_cap > 0 ? M : 0;
}

int q35_state_copy_lane(q35_engine* e, q35_state* src, int src_lane, q35_state* dst, int dst_lane) {
    return guard([&] {
        REQ(e && src && dst, Q35_ERR_ARG, "null argument");
        HCK(hipStreamSynchronize(e->st));
        ++e->meta_epoch;
        copy_lane(e, src, src_lane, dst, dst_lane);
    });
}
int q35_state_snapshot(q35_engine* e, q35_state* s, int lane, void* host, size_t bytes, size_t* bytes_needed) {
    return guard([&] {
        REQ(e && s && (host || bytes_needed), Q35_ERR_ARG, "null argument");
        snapshot_lane(e, s, lane, host, bytes, bytes_needed);
    });
}
int q35_state_restore(q35_engine* e, q35_state* s, int lane, const void* host, size_t bytes) {
    return guard([&] {
        REQ(e && s && host, Q35_ERR_ARG, "null argument");
        ++e->meta_epoch;
        restore_lane(e, s, lane, host, bytes);
    });
}

int q35_state_read(q35_engine* e, q35_state* s, int lane, int which, int n_slots, void* host, size_t bytes) {
    return guard([&] { state_io(e, s, lane, which, n_slots, host, bytes, false); });
}
int q35_state_write(q35_engine* e, q35_state* s, int lane, int which, int n_slots, const void* host, size_t bytes) {
    return guard([&] { state_io(e, s, lane, which, n_slots, const_cast<void*>(host), bytes, true); });
}

// The wave loop of a prompt (prefill_wave, engine/prefill.cpp:63). all_rows: every row of every
// wave is priced (PrefillLogits::kAll, engine/prefill.h:46-58): its argmax into sampled[], its
// top logit into top[] and its logits into logits[] (nullable), in lm_head launches of at most
// kAllChunk rows; otherwise only the prompt's last row (*sampled, logits nullable).
constexpr int kAllChunk = 256;
void prefill_waves(q35_engine* e, q35_state* s, int lane, const int32_t* ids, int n, bool all_rows,
                   int32_t* sampled, float* top, float* logits) {
    REQ(e && s && ids && sampled, Q35_ERR_ARG, "null argument");
    REQ(n > 0, Q35_ERR_ARG, "empty prompt");
    check_lane(s, lane);
    REQ(s->prefix[lane] + n <= s->cap, Q35_ERR_CAP, "prompt exceeds the lane's cache capacity");
    for (int i = 0; i < n; ++i) check_tok(ids[i]);
    int done = 0;
    while (done < n) {
        const int T = std::min(e->R, n - done);
        HCK(hipStreamSynchronize(e->st));
        for (int t = 0; t < T; ++t) {
            e->h_tok[t] = ids[done + t];
            e->h_lane[t] = lane;
            e->h_pos[t] = s->prefix[lane] + t;
            e->h_slot[t] = s->prefix[lane] + t;
        }
        body(e, s, T, T, false);
        s->prefix[lane] += T;
        advance_lane(s, lane);
        const uint16_t* normw = !body_final_normed(e, T, T, false) ? e->final_norm : nullptr;
        if (all_rows) {
            // the body's tokens are consumed: lm_head leaves row r0 + i's id in tok_dev[i]
            for (int r0 = 0; r0 < T; r0 += kAllChunk) {
                const int M = std::min(kAllChunk, T - r0);
                lm_head(e, r0, M, logits != nullptr, normw, e->topv_dev);
                HCK(hipMemcpyAsync(sampled + done + r0, e->tok_dev, M * sizeof(int), hipMemcpyDeviceToHost, e->st));
                if (top) HCK(hipMemcpyAsync(top + done + r0, e->topv_dev, M * sizeof(float), hipMemcpyDeviceToHost, e->st));
                if (logits)
                    HCK(hipMemcpyAsync(logits + (size_t)(done + r0) * kVocab, e->logits_dev, (size_t)M * kVocab * 4,
                                       hipMemcpyDeviceToHost, e->st));
                HCK(hipStreamSynchronize(e->st));
            }
        }
        done += T;
        if (done == n) {
            if (!all_rows) lm_head(e, T - 1, 1, logits != nullptr, normw);
            save_hlast(e, s, {T - 1}, {lane});
        }
    }
    if (!all_rows) {
        HCK(hipMemcpyAsync(e->h_out, e->tok_dev, sizeof(int), hipMemcpyDeviceToHost, e->st));
        if (logits) HCK(hipMemcpyAsync(logits, e->logits_dev, (size_t)kVocab * 4, hipMemcpyDeviceToHost, e->st));
        HCK(hipStreamSynchronize(e->st));
        *sampled = e->h_out[0];
    }
    HCK(hipStreamSynchronize(e->st));
}

// Prompts of several lanes in shared body passes (the batched form of prefill_wave,
// engine/prefill.cpp:63, one wave per request there): every round takes the lanes with prompt
// tokens left, at most max_rows rows, T rows per lane (the fewest any of them has left), so rows
// of different lanes share each GEMM; a lane whose prompt ends in the round gets its greedy id
// from its last row. A single lane takes the one-lane waves of q35_prefill (chunked GDN, flash
// attention for >= 64 rows).
static void prefill_lanes(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* ids,
                          const int32_t* lens, int32_t* y0, float* logits) {
    REQ(e && s && ids && lens && y0 && n > 0, Q35_ERR_ARG, "null argument");
    std::vector<int> ls(n), off(n), left(n);
    long long tot = 0;
    for (int i = 0; i < n; ++i) {
        ls[i] = lanes ? lanes[i] : i;
        check_lane(s, ls[i]);
        for (int j = 0; j < i; ++j) REQ(ls[j] != ls[i], Q35_ERR_ARG, "duplicate lane in one prefill");
        REQ(lens[i] > 0, Q35_ERR_ARG, "empty prompt");
        REQ(s->prefix[ls[i]] + lens[i] <= s->cap, Q35_ERR_CAP, "prompt exceeds the lane's cache capacity");
        off[i] = (int)tot;
        left[i] = lens[i];
        tot += lens[i];
    }
    for (long long t = 0; t < tot; ++t) check_tok(ids[t]);
    REQ(e->weights_ready, Q35_ERR_STATE, "weights not initialised");
    if (n == 1) {
        prefill_waves(e, s, ls[0], ids, lens[0], false, y0, nullptr, logits);
        return;
    }
    for (;;) {
        std::vector<int> act;
        for (int i = 0; i < n; ++i) if (left[i] > 0) act.push_back(i);
        if (act.empty()) break;
        for (size_t g0 = 0; g0 < act.size(); g0 += (size_t)e->R) {
            const std::vector<int> grp(act.begin() + g0, act.begin() + std::min(act.size(), g0 + (size_t)e->R));
            const int nl = (int)grp.size();
            int T = e->R / nl;
            for (int i : grp) T = std::min(T, left[i]);
            HCK(hipStreamSynchronize(e->st));
            for (int k = 0; k < nl; ++k) {
                const int i = grp[k], l = ls[i], done = lens[i] - left[i];
                for (int t = 0; t < T; ++t) {
                    const int r = k * T + t;
                    e->h_tok[r] = ids[off[i] + done + t];
                    e->h_lane[r] = l; e->h_pos[r] = s->prefix[l] + t; e->h_slot[r] = s->prefix[l] + t;
                }
            }
            const int R = nl * T;
            body(e, s, R, T, false);
            if (!body_final_normed(e, R, T, false))
                HCK(launch_addnorm(2, nullptr, nullptr, e->x, nullptr, nullptr, 0, e->final_norm, e->nrm, R, e->st));
            std::vector<int> fin, src, fl;
            for (int k = 0; k < nl; ++k) {
                const int i = grp[k], l = ls[i];
                s->prefix[l] += T;
                advance_lane(s, l);
                left[i] -= T;
                if (left[i] == 0) { fin.push_back(i); src.push_back(k * T + T - 1); fl.push_back(l); }
            }
            if (fin.empty()) continue;
            const int m = (int)fin.size();
            save_hlast(e, s, src, fl);
            // the finishing lanes' last rows, gathered contiguously for one lm_head pass
            HCK(hipStreamSynchronize(e->st));
            for (int k = 0; k < m; ++k) { e->h_src[k] = src[k]; e->h_dst[k] = k; }
            upload_idx(e, m);
            HCK(launch_copy_rows(e->nrm, e->ridx_src, e->h, e->ridx_dst, m, kHidden, e->st));
            lm_head(e, 0, m, logits != nullptr, nullptr, nullptr, e->h);
            HCK(hipMemcpyAsync(e->h_out, e->tok_dev, m * sizeof(int), hipMemcpyDeviceToHost, e->st));
            if (logits)
                for (int k = 0; k < m; ++k)
                    HCK(hipMemcpyAsync(logits + (size_t)fin[k] * kVocab, e->logits_dev + (size_t)k * kVocab,
                                       (size_t)kVocab * 4, hipMemcpyDeviceToHost, e->st));
            HCK(hipStreamSynchronize(e->st));
            for (int k = 0; k < m; ++k) y0[fin[k]] = e->h_out[k];
        }
    }
    ++e->meta_epoch;
}

int q35_prefill_lanes(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* ids,
                      const int32_t* lens, int32_t* y0, float* logits) {
    return guard([&] { prefill_lanes(e, s, lanes, n, ids, lens, y0, logits); });
}

int q35_prefill(q35_engine* e, q35_state* s, int lane, const int32_t* ids, int n, int32_t* y0, float* logits) {
    return guard([&] { prefill_waves(e, s, lane, ids, n, false, y0, nullptr, logits); });
}

int q35_prefill_all(q35_engine* e, q35_state* s, int lane, const int32_t* ids, int n, int32_t* sampled,
                    float* top_logit, float* logits) {
    return guard([&] { prefill_waves(e, s, lane, ids, n, true, sampled, top_logit, logits); });
}

int q35_decode_step(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* tokens,
                    int32_t* out_tok, float* out_logits) {
    return guard([&] {
        REQ(e && s && tokens && out_tok, Q35_ERR_ARG, "null argument");
        REQ(n > 0 && n <= e->R, Q35_ERR_CAP, "lane count exceeds max_rows");
        HCK(hipStreamSynchronize(e->st));
        std::vector<int> ls(n);
        for (int i = 0; i < n; ++i) {
            const int l = lanes ? lanes[i] : i;
            check_lane(s, l);
            check_tok(tokens[i]);
            REQ(s->prefix[l] < s->cap, Q35_ERR_CAP, "lane cache is full");
            for (int j = 0; j < i; ++j) REQ(ls[j] != l, Q35_ERR_ARG, "duplicate lane in one step");
            ls[i] = l;
            e->h_tok[i] = tokens[i]; e->h_lane[i] = l; e->h_pos[i] = s->prefix[l]; e->h_slot[i] = s->prefix[l];
        }
        REQ(e->weights_ready, Q35_ERR_STATE, "weights not initialised");
        for (int i = 0; i < n; ++i) { e->h_src[i] = i; e->h_dst[i] = ls[i]; }
        bool fast = e->fast_s == (const void*)s && e->fast_epoch == e->meta_epoch && (int)e->fast_lanes.size() == n;
        for (int i = 0; fast && i < n; ++i)
            fast = e->fast_lanes[i] == ls[i] && e->fast_tok[i] == tokens[i] &&
                   e->fast_prefix[i] == s->prefix[ls[i]] && e->fast_cur[i] == s->cur[ls[i]] &&
                   e->fast_wcur[i] == s->wcur[ls[i]] && e->fast_pend[i] == s->pend_code(ls[i]);
        e->fast_s = nullptr;                 // re-armed only when this step completes
        if (!fast) {
            stage_rcur(e, s, n);
            upload_meta(e, 8, n);        // tok, lane, pos, slot, cur, wcur, pend, src, dst in one copy
        }
        const int defer = step_defer(e);
        auto step = [&] {
            body_kernels(e, s, n, 1, false, defer);
            lm_head(e, 0, n, out_logits != nullptr, !body_final_normed(e, n, 1, false) ? e->final_norm : nullptr);
            HCK(launch_copy_rows_advance(e->nrm, e->ridx_src, s->hlast, e->ridx_dst, n, kHidden, e->rpos, e->rslot,
                                         e->rcur, e->rwcur, e->rpend, s->nslots, defer, e->st));
        };
        if (e->use_graph && e->kprof == 0) {
            if (out_logits) ensure_logits(e, n);
            char key[128];
            std::snprintf(key, sizeof key, "dec:%p:%d:%d:%d:%d", (void*)s, n, out_logits ? 1 : 0, e->n_layers, defer);
            auto it = e->graphs.find(key);
            if (it == e->graphs.end()) {
                hipGraph_t g;
                HCK(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
                try {
                    step();
                } catch (...) {
                    hipStreamEndCapture(e->st, &g);
                    throw;
                }
                HCK(hipStreamEndCapture(e->st, &g));
                hipGraphExec_t ex;
                HCK(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
                HCK(hipGraphDestroy(g));
                it = e->graphs.emplace(key, ex).first;
            }
            HCK(hipGraphLaunch(it->second, e->st));
        } else {
            step();
        }
        for (int i = 0; i < n; ++i) {
            s->prefix[ls[i]] += 1;
            advance_decode(s, ls[i], defer);
        }
        HCK(hipMemcpyAsync(e->h_out, e->tok_dev, n * sizeof(int), hipMemcpyDeviceToHost, e->st));
        if (out_logits) HCK(hipMemcpyAsync(out_logits, e->logits_dev, (size_t)n * kVocab * 4, hipMemcpyDeviceToHost, e->st));
        HCK(hipStreamSynchronize(e->st));
        for (int i = 0; i < n; ++i) out_tok[i] = e->h_out[i];
        e->fast_lanes.assign(ls.begin(), ls.begin() + n);
        e->fast_tok.assign(out_tok, out_tok + n);
        e->fast_prefix.resize(n);
        e->fast_cur.resize(n);
        e->fast_wcur.resize(n);
        e->fast_pend.resize(n);
        for (int i = 0; i < n; ++i) {
            e->fast_prefix[i] = s->prefix[ls[i]]; e->fast_cur[i] = s->cur[ls[i]]; e->fast_wcur[i] = s->wcur[ls[i]];
            e->fast_pend[i] = s->pend_code(ls[i]);
        }
        e->fast_epoch = e->meta_epoch;
        e->fast_s = s;
    });
}

int q35_mtp_draft(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* y,
                  const int32_t* pos, int step, int32_t* out_tok, uint16_t* out_xd, float* out_logits) {
    return guard([&] {
        REQ(e && s && y && pos && out_tok, Q35_ERR_ARG, "null argument");
        REQ(n > 0 && n <= e->R, Q35_ERR_CAP, "lane count exceeds max_rows");
        HCK(hipStreamSynchronize(e->st));
        std::vector<int> ls(n);
        for (int i = 0; i < n; ++i) {
            const int l = lanes ? lanes[i] : i;
            check_lane(s, l);
            check_tok(y[i]);
            REQ(s->mtp_len[l] + step < s->mtp_cap, Q35_ERR_CAP, "MTP cache is full");
            ls[i] = l;
            e->h_tok[i] = y[i]; e->h_lane[i] = l; e->h_pos[i] = pos[i]; e->h_slot[i] = s->mtp_len[l] + step;
            e->h_src[i] = l; e->h_dst[i] = i;
        }
        // h rows: lane's hlast (post-final-norm row of the last body) -> e->h as scratch source
        upload_idx(e, n);
        HCK(launch_copy_rows(s->hlast, e->ridx_src, e->delta, e->ridx_dst, n, kHidden, e->st));
        mtp_draft_pass(e, s, n, e->delta);
        lm_head(e, 0, n, out_logits != nullptr, small_rows(n) ? e->mtp_norm : nullptr);
        // x_d becomes the lane's h for the next draft (speccheck/mtp.py:153-157)
        std::vector<int> rows(n);
        for (int i = 0; i < n; ++i) rows[i] = i;
        HCK(hipMemcpyAsync(e->h_out, e->tok_dev, n * sizeof(int), hipMemcpyDeviceToHost, e->st));
        if (out_xd) HCK(hipMemcpyAsync(out_xd, e->nrm, (size_t)n * kHidden * 2, hipMemcpyDeviceToHost, e->st));
        save_hlast(e, s, rows, ls);
        if (out_logits) HCK(hipMemcpyAsync(out_logits, e->logits_dev, (size_t)n * kVocab * 4, hipMemcpyDeviceToHost, e->st));
        HCK(hipStreamSynchronize(e->st));
        for (int i = 0; i < n; ++i) out_tok[i] = e->h_out[i];
    });
}

int q35_mtp_round(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                  int k, int32_t* emit, int32_t* n_emit, int64_t* stats) {
    return q35_mtp_round_stop(e, s, lanes, n, cur, k, -1, emit, n_emit, stats);
}

// stop >= 0: an accepted draft equal to `stop` ends the accepted prefix (the target row before
// it chose the same token, so it is emitted as the bonus and left pending, never fed): the
// session driver's stop cut, engine/mtp_accept.cpp:585-600
// The verify body of a speculative round and its greedy accept / rollback (speccheck/mtp.py:
// 150-177; mtpaccept::accept_round, engine/mtp_accept.h:248): per lane, the (k+1)-row body
// over [cur, d1..dk] with per-row GDN factors, accept of the longest prefix the target rows
// confirm (the stop cut applied), then the state, window and MTP cache kept for rows 0..a.
static void mtp_verify_accept(q35_engine* e, q35_state* s, const std::vector<int>& ls, const std::vector<int>& P,
                   const int32_t* cur, int k, const std::vector<std::vector<int>>& drafts, int32_t stop,
                   int32_t* emit, int32_t* n_emit, int64_t* stats) {
    const int n = (int)ls.size();
    // verify body over [cur, d1..dk] per lane with per-row GDN checkpoints
    HCK(hipStreamSynchronize(e->st));
    const int T = k + 1, R = n * T;
    for (int i = 0; i < n; ++i)
        for (int t = 0; t < T; ++t) {
            int r = i * T + t;
            e->h_tok[r] = t == 0 ? cur[i] : drafts[i][t - 1];
            e->h_lane[r] = ls[i]; e->h_pos[r] = P[i] + t; e->h_slot[r] = P[i] + t;
        }
    body(e, s, R, T, true);
    lm_head(e, 0, R, false, !body_final_normed(e, R, T, true) ? e->final_norm : nullptr);
    HCK(hipMemcpyAsync(e->h_out, e->tok_dev, R * sizeof(int), hipMemcpyDeviceToHost, e->st));
    HCK(hipStreamSynchronize(e->st));
    std::vector<int> rows(n);
    for (int i = 0; i < n; ++i) {
        const int* tgt = e->h_out + i * T;
        int a = 0;
        while (a < k && drafts[i][a] == tgt[a] && drafts[i][a] != stop) ++a;
        int m = 0;
        for (int j = 0; j < a; ++j) emit[i * (k + 1) + m++] = drafts[i][j];
        emit[i * (k + 1) + m++] = tgt[a];
        n_emit[i] = m;
        const int l = ls[i];
        s->prefix[l] = P[i] + a + 1;
        // the verify body recorded every row as factors on top of slot cur (after moving
        // the lane's earlier pending rows into slot cur + 1): rows 0..a are now pending
        if (s->pend[l] > 0) s->cur[l] = (s->cur[l] + 1) % s->nslots;
        s->pend[l] = a + 1;
        s->pset[l] ^= 1;
        s->wcur[l] = (s->wcur[l] + 1 + a) % s->nslots;
        if (a == k) s->mtp_len[l] += k;
        rows[i] = i * T + a;
        if (stats) { stats[0] += k; stats[1] += a; stats[2] += 1; stats[3] += T; }
    }
    save_hlast(e, s, rows, ls);
    HCK(hipStreamSynchronize(e->st));
}

int q35_mtp_round_stop(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                       int k, int32_t stop, int32_t* emit, int32_t* n_emit, int64_t* stats) {
    return guard([&] {
        REQ(e && s && cur && emit && n_emit, Q35_ERR_ARG, "null argument");
        REQ(k >= 1 && k <= s->mtp_k, Q35_ERR_STATE, "k exceeds the state's MTP slots");
        REQ(n > 0 && n * (k + 1) <= e->R, Q35_ERR_CAP, "rows exceed max_rows");
        ++e->meta_epoch;                 // drafts and the verify body rewrite the row metadata
        std::vector<int> ls(n), P(n);
        for (int i = 0; i < n; ++i) {
            ls[i] = lanes ? lanes[i] : i;
            check_lane(s, ls[i]);
            P[i] = s->prefix[ls[i]];
            REQ(P[i] + k + 1 <= s->cap, Q35_ERR_CAP, "lane cache is full");
        }
        // each draft leaves x_d in hlast (the next draft's h); the verify row a replaces it
        std::vector<std::vector<int>> drafts(n, std::vector<int>(k));
        std::vector<int32_t> y(cur, cur + n), pos(n), dt(n);
        for (int j = 0; j < k; ++j) {
            for (int i = 0; i < n; ++i) pos[i] = P[i] + 1 + j;
            int rc = q35_mtp_draft(e, s, ls.data(), n, y.data(), pos.data(), j, dt.data(), nullptr, nullptr);
            if (rc) throw Q35Error(rc, g_err);
            for (int i = 0; i < n; ++i) { drafts[i][j] = dt[i]; y[i] = dt[i]; }
        }
        mtp_verify_accept(e, s, ls, P, cur, k, drafts, stop, emit, n_emit, stats);
    });
}

// The verify half of a round on drafts the caller made (mtpaccept::accept_round's candidates,
// engine/mtp_accept.h:248): draft step j of lane i in drafts[i * k + j].
int q35_mtp_verify(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur, int k,
                   const int32_t* drafts, int32_t stop, int32_t* emit, int32_t* n_emit, int64_t* stats) {
    return guard([&] {
        REQ(e && s && cur && drafts && emit && n_emit, Q35_ERR_ARG, "null argument");
        REQ(k >= 1 && k <= s->mtp_k, Q35_ERR_STATE, "k exceeds the state's MTP slots");
        REQ(n > 0 && n * (k + 1) <= e->R, Q35_ERR_CAP, "rows exceed max_rows");
        ++e->meta_epoch;
        std::vector<int> ls(n), P(n);
        std::vector<std::vector<int>> dr(n, std::vector<int>(k));
        for (int i = 0; i < n; ++i) {
            ls[i] = lanes ? lanes[i] : i;
            check_lane(s, ls[i]);
            check_tok(cur[i]);
            for (int j = 0; j < i; ++j) REQ(ls[j] != ls[i], Q35_ERR_ARG, "duplicate lane in one round");
            P[i] = s->prefix[ls[i]];
            REQ(P[i] + k + 1 <= s->cap, Q35_ERR_CAP, "lane cache is full");
            REQ(s->mtp_len[ls[i]] + k <= s->mtp_cap, Q35_ERR_CAP, "MTP cache is full");
            for (int j = 0; j < k; ++j) {
                check_tok(drafts[i * k + j]);
                dr[i][j] = drafts[i * k + j];
            }
        }
        mtp_verify_accept(e, s, ls, P, cur, k, dr, stop, emit, n_emit, stats);
    });
}

// One decoding turn of n lanes, each at its own adaptive depth (engine/mtp_adaptive.h; the
// reference drives one request per process, decode_run.cpp:4857-5010 / mtp_accept.cpp:525-640):
// the lanes at depth 2 run one k = 2 round together, those at depth 1 one k = 1 round, the
// abandoned ones one plain step; each round's emitted count is fed to its lane's policy.
int q35_mtp_adaptive_step(q35_engine* e, q35_state* s, const int32_t* lanes, int n, const int32_t* cur,
                          q35_mtp_policy* const* pol, int32_t stop, int32_t* emit, int32_t* n_emit,
                          int32_t* depth, int64_t* stats) {
    return guard([&] {
        REQ(e && s && cur && pol && emit && n_emit, Q35_ERR_ARG, "null argument");
        REQ(n > 0, Q35_ERR_ARG, "no lanes");
        std::vector<int> grp[3];
        for (int i = 0; i < n; ++i) {
            REQ(pol[i], Q35_ERR_ARG, "null policy");
            int32_t k = 0;
            q35_mtp_policy_k(pol[i], &k);
            REQ(k <= s->mtp_k, Q35_ERR_STATE, "policy depth exceeds the state's MTP slots");
            grp[k].push_back(i);
            if (depth) depth[i] = k;
        }
        // every group's preconditions before any group runs: a later group's refusal must not
        // leave earlier groups advanced with their emits unreported
        for (int i = 0; i < n; ++i) {
            const int l = lanes ? lanes[i] : i;
            check_lane(s, l);
            check_tok(cur[i]);
            for (int j = 0; j < i; ++j) REQ((lanes ? lanes[j] : j) != l, Q35_ERR_ARG, "duplicate lane in one step");
        }
        for (int k = 2; k >= 0; --k) {
            const int m = (int)grp[k].size();
            REQ(m * (k + 1) <= e->R, Q35_ERR_CAP, "rows exceed max_rows");
            for (int i : grp[k]) {
                const int l = lanes ? lanes[i] : i;
                REQ(s->prefix[l] + k + 1 <= s->cap, Q35_ERR_CAP, "lane cache is full");
                REQ(k == 0 || s->mtp_len[l] + k <= s->mtp_cap, Q35_ERR_CAP, "MTP cache is full");
            }
        }
        for (int k = 2; k >= 0; --k) {
            const int m = (int)grp[k].size();
            if (!m) continue;
            std::vector<int32_t> ls(m), cs(m), em((size_t)m * (k + 1)), ne(m);
            for (int j = 0; j < m; ++j) { ls[j] = lanes ? lanes[grp[k][j]] : grp[k][j]; cs[j] = cur[grp[k][j]]; }
            int rc;
            if (k > 0) {
                rc = q35_mtp_round_stop(e, s, ls.data(), m, cs.data(), k, stop, em.data(), ne.data(), stats);
            } else {
                rc = q35_decode_step(e, s, ls.data(), m, cs.data(), em.data(), nullptr);
                for (int j = 0; j < m; ++j) ne[j] = 1;
            }
            if (rc) throw Q35Error(rc, g_err);
            for (int j = 0; j < m; ++j) {
                const int i = grp[k][j];
                n_emit[i] = ne[j];
                for (int t = 0; t < 3; ++t) emit[i * 3 + t] = t < ne[j] ? em[(size_t)j * (k + 1) + t] : -1;
                if (k > 0) q35_mtp_policy_note(pol[i], k, ne[j], nullptr, nullptr);
            }
        }
    });
}

int q35_op_tile_weight(q35_engine* e, const uint16_t* w, int N, int K, uint16_t* wt) {
    return guard([&] {
        REQ(e && w && wt && N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0, Q35_ERR_ARG, "bad weight shape");
        HCK(launch_tile(w, N, K, wt, 0, 0, e->st));
    });
}

int q35_op_gemm(q35_engine* e, const uint16_t* wt, int N, int K, const uint16_t* x, int M, uint16_t* y) {
    return guard([&] {
        REQ(e && wt && x && y && M > 0 && N % 16 == 0 && K % 256 == 0 && K <= 4096, Q35_ERR_ARG, "bad gemm shape");
        gemm(e, wt, N, K, M, x, K, y, N);
    });
}

// One GDN decode step of B lanes on caller buffers; y/gnorm (optional) receive the gated
// RMSNorm output as the engine's path for B lanes makes it: whole-head blocks (B > 64) fuse it
// into the recurrence's epilogue, column-sliced blocks (B <= 64) leave it to the out_proj
// GEMM's A producer (produce_kernel here). form 1: the non-persistent whole-head kernel
// (gdn_kernel<1>, the MTP verify path) instead of the persistent one.
static void op_gdn(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                   const uint16_t* dt_bias, const uint16_t* gnorm, float* S2, float* W2, float* o, uint16_t* y,
                   int B, int form) {
    REQ(e && proj && conv_w && A_log && dt_bias && S2 && W2 && o && B > 0, Q35_ERR_ARG, "bad gdn call");
    REQ(B <= 65536 && (form == 0 || form == 1), Q35_ERR_ARG, "bad gdn call");
    REQ(!y == !gnorm, Q35_ERR_ARG, "y and gnorm go together");
    REQ(!y || B <= e->R, Q35_ERR_CAP, "B exceeds max_rows (the norm staging is engine scratch)");
    // rows b = lanes b (T = 1); per lane two slots: 0 = input state, 1 = output state
    std::vector<int> lanes(B);
    for (int i = 0; i < B; ++i) lanes[i] = i;
    int* dl = dalloc<int>(B);
    copy_sync(e, dl, lanes.data(), B * sizeof(int), hipMemcpyHostToDevice);
    GdnArgs g{};
    g.proj = proj; g.o = o; g.conv_w = conv_w; g.A_log = A_log; g.dt_bias = dt_bias;
    g.S = S2; g.S_lane = 2 * kSLayer; g.S_slot = kSLayer; g.S_layer = 0;
    g.win = W2; g.W_lane = 2 * kWLayer; g.W_slot = kWLayer; g.W_layer = 0;
    g.cur = nullptr; g.nslots = 2; g.ckpt = 0;
    g.lane = dl; g.T = 1; g.nlanes = B;
    const int cs = B <= 8 ? 8 : B <= 32 ? 4 : B <= 64 ? 2 : 1;
    const bool whole = cs == 1 || form == 1;           // whole-head blocks: norm in the epilogue
    if (whole && y) { g.y = y; g.gnorm = gnorm; }
    if (cs == 1 && form == 0) HCK(launch_gdn_persist(g, e->st));
    else HCK(launch_gdn(g, whole ? 1 : cs, e->st));
    if (y && !whole) {
        // the column-sliced path: the out_proj producer's arithmetic, staged to y
        GemmArgs a{};
        a.N = kHidden; a.K = 2048; a.M = B; a.X = o; a.ldx = 2048; a.X2 = proj + kGdnZOff; a.ldx2 = kGdnInRows;
        a.aux_w = gnorm; a.prod = y; a.forms = e->forms;
        HCK(launch_produce(a, kAGatedNorm, e->st));
    }
    HCK(hipStreamSynchronize(e->st));
    HCK(hipFree(dl));
}

int q35_op_gdn_step(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                    const uint16_t* dt_bias, float* S2, float* W2, float* o, int B) {
    return guard([&] { op_gdn(e, proj, conv_w, A_log, dt_bias, nullptr, S2, W2, o, nullptr, B, 0); });
}

int q35_op_gdn_step_norm(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                         const uint16_t* dt_bias, const uint16_t* gnorm, float* S2, float* W2, float* o,
                         uint16_t* y, int B, int form) {
    return guard([&] { op_gdn(e, proj, conv_w, A_log, dt_bias, gnorm, S2, W2, o, y, B, form); });
}

// The allocation-free form of q35_op_gdn_step: no hipMalloc / hipFree and no host copy (the
// lane list is written on the device into the per-GPU `scratch` array); asynchronous on the
// engine stream (q35_sync waits for it). Calls that would overlap on one GPU -- another
// engine's call while this GPU's last one is still running -- are refused (Q35_ERR_STATE).
int q35_op_gdn_step_noalloc(q35_engine* e, const uint16_t* proj, const uint16_t* conv_w, const uint16_t* A_log,
                            const uint16_t* dt_bias, float* S2, float* W2, float* o, int B) {
    return guard([&] {
        REQ(e && proj && conv_w && A_log && dt_bias && S2 && W2 && o && B > 0, Q35_ERR_ARG, "bad gdn call");
        REQ(B <= kNoAllocMaxLanes, Q35_ERR_CAP,
            "B exceeds the allocation-free GDN step's maximum of " + std::to_string(kNoAllocMaxLanes) + " lanes");
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        int* lanes = noalloc_scratch(e->device, e, e->noalloc_ev);
        hipLaunchKernelGGL(iota_kernel, dim3((B + 255) / 256), dim3(256), 0, e->st, lanes, B);
        HCK(hipGetLastError());
        GdnArgs g{};
        g.proj = proj; g.o = o; g.conv_w = conv_w; g.A_log = A_log; g.dt_bias = dt_bias;
        g.S = S2; g.S_lane = 2 * kSLayer; g.S_slot = kSLayer; g.S_layer = 0;
        g.win = W2; g.W_lane = 2 * kWLayer; g.W_slot = kWLayer; g.W_layer = 0;
        g.cur = nullptr; g.nslots = 2; g.ckpt = 0;
        g.lane = lanes; g.T = 1; g.nlanes = B;
        const int cs = B <= 8 ? 8 : B <= 32 ? 4 : B <= 64 ? 2 : 1;
        if (cs == 1) HCK(launch_gdn_persist(g, e->st));
        else HCK(launch_gdn(g, cs, e->st));
        HCK(hipEventRecord(e->noalloc_ev, e->st));
    });
}

int q35_op_gemm_a(q35_engine* e, const uint16_t* wt, int N, int K, int amode, const void* x, int ldx,
                  const void* x2, int ldx2, const uint16_t* aux, int M, uint16_t* y) {
    return guard([&] {
        REQ(e && wt && x && y && M > 0 && N % 16 == 0 && K % 256 == 0 && K <= 4096, Q35_ERR_ARG, "bad gemm shape");
        REQ(amode == kAPlain || amode == kASiluMul || amode == kAGatedNorm || amode == 3 || amode == 5 || amode == 6,
            Q35_ERR_ARG, "amode is 0 .. 3, 5, 6");
        if (amode == 3 || amode == 5 || amode == 6) {
            // plain A through the batched GEMMs with the SwiGLU epilogue (5: Y [M][N/2] =
            // bf16(bf16(silu(X.Wg^T)) * bf16(X.Wu^T)), W = gate rows then up rows), and through the
            // many-row kernel (3: stored, 6: SwiGLU), X tiled into the engine's h staging first
            REQ(K == kHidden && M >= 17 && M <= e->R && ldx == K, Q35_ERR_ARG, "amode 3/5/6: K = 1024, 17 <= M <= max_rows");
            const bool wide = amode != 5;
            const int em = amode == 3 ? kEStore : kESiluMul;
            if (wide) HCK(launch_tile((const uint16_t*)x, M, K, e->h, 0, 0, e->st));
            gemm(e, wt, N, K, M, wide ? e->h : x, K, y, em == kESiluMul ? N / 2 : N, kAPlain, nullptr, 0, nullptr, em,
                 nullptr, wide);
            return;
        }
        REQ(amode == kAPlain || x2, Q35_ERR_ARG, "this producer needs x2");
        REQ(amode != kAGatedNorm || (aux && K % 128 == 0), Q35_ERR_ARG, "gated norm needs its weight");
        REQ(M <= 16 || amode == kAPlain || ((size_t)M * K <= (size_t)e->R * kFF), Q35_ERR_CAP,
            "M x K exceeds the producer staging");
        gemm(e, wt, N, K, M, x, ldx, y, N, amode, x2, ldx2, aux);
    });
}

int q35_op_lm_head_argmax(q35_engine* e, const uint16_t* x, int M, int32_t* tok, float* logits) {
    return guard([&] {
        REQ(e && x && tok && M > 0 && M <= e->R, Q35_ERR_ARG, "bad lm_head call");
        GemmArgs a{};
        a.W = e->E; a.N = kVocab; a.K = kHidden; a.M = M; a.X = x; a.ldx = kHidden; a.forms = e->forms;
        a.logits = logits; a.ldl = kVocab;
        a.part_val = e->pval; a.part_idx = e->pidx; a.ldp = kVocab / 16;
        HCK(launch_gemm(a, kAPlain, kEArgmax, e->st));
        HCK(launch_argmax(e->pval, e->pidx, kVocab / 16, gemm_argmax_partials(a), M, tok, nullptr, e->st));
    });
}

int q35_op_attn_decode(q35_engine* e, q35_state* s, int layer, const int32_t* lanes, const int32_t* pos, int n, int T,
                       const uint16_t* proj, const uint16_t* q_norm, const uint16_t* k_norm, uint16_t* out, int form) {
    return guard([&] {
        REQ(e && s && proj && q_norm && k_norm && out && n > 0 && T > 0, Q35_ERR_ARG, "bad attention call");
        REQ(layer >= 0 && layer < kAttnLayers, Q35_ERR_ARG, "attention layer is 0 .. 5");
        REQ(form >= kAttnAuto && form <= kAttnPrompt, Q35_ERR_ARG, "form is 0 .. 6");
        const int R = n * T;
        REQ(R <= e->R, Q35_ERR_CAP, "rows exceed engine max_rows");
        for (int i = 0; i < n; ++i) {
            const int l = lanes ? lanes[i] : i;
            REQ(l >= 0 && l < s->lanes, Q35_ERR_ARG, "lane out of range");
            const int p = pos ? pos[i] : s->prefix[l];
            REQ(p >= 0 && p + T <= s->cap, Q35_ERR_CAP, "rows past the lane's cache capacity");
            for (int t = 0; t < T; ++t) {
                const int r = i * T + t;
                e->h_tok[r] = 0; e->h_lane[r] = l; e->h_pos[r] = p + t; e->h_slot[r] = p + t;
            }
        }
        stage_rcur(e, s, R);
        upload_rows(e, R);
        AttnArgs a{};
        a.proj = proj; a.q_norm = q_norm; a.k_norm = k_norm;
        a.kc = s->kc; a.vc = s->vc; a.kv_lane = s->kv_lane(); a.kv_layer_off = (long long)layer * 2 * s->capT * 256;
        a.cap = s->capT;
        a.rm.lane = e->rlane; a.rm.pos = e->rpos; a.rm.slot = e->rslot;
        a.q = e->q; a.sc = e->sc; a.sc_ld = e->sc_ld; a.stats = e->stats; a.part = e->part;
        a.max_chunks = (a.cap + 255) / 256;
        REQ(a.max_chunks <= e->max_chunks, Q35_ERR_CAP, "cache capacity exceeds engine max_ctx");
        a.out = out; a.R = R; a.T = T; a.inv_freq = e->inv_freq; a.prompt_flash = e->forms.attn_prompt;
        a.split4 = e->forms.attn_split4; a.fused_pair = e->forms.attn_pair; a.rows_form = e->forms.attn_rows;
        a.force = form;
        REQ(attn_form_ok(a), Q35_ERR_ARG, "this attention form cannot run this shape (rows, rows per lane, capacity)");
        HCK(launch_attn_prep(a, e->st));
        HCK(launch_attn_core(a, e->st));
        HCK(hipStreamSynchronize(e->st));
    });
}

int q35_set_option(q35_engine* e, const char* name, int value) {
    return guard([&] {
        REQ(e && name, Q35_ERR_ARG, "null argument");
        std::string n(name);
        if (n == "layers") {
            REQ(value >= 1 && value <= kLayers, Q35_ERR_ARG, "layers out of range");
            e->n_layers = value;
        } else if (n == "kprof") {
            REQ(value >= 0 && value <= 5, Q35_ERR_ARG, "kprof family out of range");
            HCK(hipStreamSynchronize(e->st));
            e->kprof = value;
            e->kev_used = 0;
        } else if (n == "graph") {
            e->use_graph = value;
        } else if (n == "gdn_chunked") {
            HCK(hipStreamSynchronize(e->st));
            e->gdn_chunked = value ? 1 : 0;
        } else if (n == "prompt_exact") {
            // prompt waves in the decode step's arithmetic: the one-row attention kernels and the
            // recurrent GDN kernel, so a prompt is byte-identical to feeding it token by token
            HCK(hipStreamSynchronize(e->st));
            e->gdn_chunked = value ? 0 : 1;
            e->forms.attn_prompt = value ? 0 : 1;
        } else if (n == "b1_partials" || n == "attn_prompt" || n == "partial_rows" || n == "gemv_tpb" ||
                   n == "gemm_pre" || n == "lmhead_persist" || n == "attn_split4" || n == "gemm_wide" || n == "attn_pair" || n == "attn_rows" || n == "gdn_rows" ||
                   n == "gdn_defer" || n == "mid_partials") {
            // kernel-form switches of this engine: captured steps hold the old forms
            REQ(n != "partial_rows" || value >= 17, Q35_ERR_ARG, "partial_rows must exceed the 16-row batch-1 path");
            REQ(n != "gemv_tpb" || value == 1 || value == 2, Q35_ERR_ARG, "gemv_tpb is 1 or 2");
            REQ(n != "gdn_defer" || (value >= 0 && value <= kMaxDefer), Q35_ERR_ARG, "gdn_defer is 0 .. 4");
            REQ(n != "attn_rows" || (value >= 0 && value <= 2), Q35_ERR_ARG, "attn_rows is 0, 1 or 2");
            HCK(hipStreamSynchronize(e->st));
            if (n == "b1_partials") e->b1_partials = value ? 1 : 0;
            else if (n == "attn_prompt") e->forms.attn_prompt = value ? 1 : 0;
            else if (n == "partial_rows") e->forms.partial_rows = value;
            else if (n == "gemv_tpb") e->forms.gemv_tpb = value;
            else if (n == "gemm_pre") e->forms.gemm_pre = value;
            else if (n == "attn_split4") e->forms.attn_split4 = value ? 1 : 0;
            else if (n == "gemm_wide") e->forms.gemm_wide = value ? 1 : 0;
            else if (n == "attn_pair") e->forms.attn_pair = value ? 1 : 0;
            else if (n == "attn_rows") e->forms.attn_rows = value;
            else if (n == "gdn_rows") e->forms.gdn_rows = value ? 1 : 0;
            else if (n == "gdn_defer") e->forms.gdn_defer = value;
            else if (n == "mid_partials") e->forms.mid_partials = value ? 1 : 0;
            else {
                REQ(value == 0 || value == 1 || value == 3, Q35_ERR_ARG, "lmhead_persist is 0, 1 or 3");
                e->forms.lmhead_persist = value;
            }
            for (auto& kv : e->graphs) hipGraphExecDestroy(kv.second);
            e->graphs.clear();
        } else {
            throw Q35Error(Q35_ERR_ARG, "unknown option " + n);
        }
    });
}

int q35_read_scratch(q35_engine* e, const char* name, void* host, size_t bytes) {
    return guard([&] {
        REQ(e && name && host, Q35_ERR_ARG, "null argument");
        std::string n(name);
        const void* p = nullptr;
        size_t cap = 0;
        const size_t R = e->R;
        if (n == "x") { p = e->x; cap = R * kHidden * 2; }
        else if (n == "h") { p = e->h; cap = R * kHidden * 2; }
        else if (n == "nrm") { p = e->nrm; cap = R * kHidden * 2; }
        else if (n == "delta") { p = e->delta; cap = R * kHidden * 2; }
        else if (n == "proj") { p = e->proj; cap = R * kGdnInRows * 2; }
        else if (n == "o") { p = e->o; cap = R * 2048 * 4; }
        else if (n == "gu") { p = e->gu; cap = R * kGuRows * 2; }
        else if (n == "aout") { p = e->aout; cap = R * 2048 * 2; }
        else if (n == "q") { p = e->q; cap = R * kNq * 256 * 4; }
        else throw Q35Error(Q35_ERR_ARG, "unknown scratch " + n);
        REQ(bytes <= cap, Q35_ERR_ARG, "read exceeds scratch size");
        HCK(hipStreamSynchronize(e->st));
        copy_sync(e, host, p, bytes, hipMemcpyDeviceToHost);
    });
}

int q35_kprof_read(q35_engine* e, float* total_ms, int* launches) {
    return guard([&] {
        REQ(e && total_ms && launches, Q35_ERR_ARG, "null argument");
        HCK(hipStreamSynchronize(e->st));
        float tot = 0.f;
        for (size_t i = 0; i < e->kev_used; ++i) {
            float ms = 0.f;
            HCK(hipEventElapsedTime(&ms, e->kev[i].first, e->kev[i].second));
            tot += ms;
        }
        *total_ms = tot;
        *launches = (int)e->kev_used;
        e->kev_used = 0;
    });
}

int q35_sync(q35_engine* e) {
    return guard([&] { REQ(e, Q35_ERR_ARG, "null engine"); HCK(hipStreamSynchronize(e->st)); });
}
int q35_timer_begin(q35_engine* e) {
    return guard([&] { REQ(e, Q35_ERR_ARG, "null engine"); HCK(hipEventRecord(e->ev0, e->st)); });
}
int q35_timer_end(q35_engine* e, float* ms) {
    return guard([&] {
        REQ(e && ms, Q35_ERR_ARG, "null argument");
        HCK(hipEventRecord(e->ev1, e->st));
        HCK(hipEventSynchronize(e->ev1));
        HCK(hipEventElapsedTime(ms, e->ev0, e->ev1));
    });
}

}  // extern "C"
