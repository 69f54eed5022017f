// Adaptive speculation depth (the reference's mtpadapt::Tracker, engine/mtp_adaptive.h:1-254):
// per request, the depth of the next MTP round -- k = 2, k = 1, or 0 (plain steps from then on) --
// decided from what the request's own rounds emitted, with no device traffic of its own.
//
// The rule, as the reference states it: the estimate is emitted tokens per step-equivalent
// over the last 32 rounds (a ratio of two tallies; each round billed at the measured cost of its
// own depth in plain steps); after 16 rounds at k = 2 an estimate below 0.95 demotes to k = 1,
// after 24 rounds at k = 1 an estimate below 0.90 abandons speculation for good. The window
// clears on every change, there is no re-promotion, so a request changes depth at most twice.
// Plain steps are never fed to the tracker.
#include <cstring>
#include <new>
#include <string>

#include "../../include/q35.h"

void q35_set_error(const char* msg);   // q35_engine.cpp: the text q35_last_error() reports

namespace {
constexpr int kWindow = 32;              // engine/mtp_adaptive.h kWindowRounds
constexpr int kMinObserve = 16;          // kMinObserveRounds (k = 2 -> 1)
constexpr int kMinObserveAbandon = 24;   // kMinObserveBeforeAbandon (k = 1 -> plain)
constexpr double kDemote = 0.95, kAbandon = 0.90;
constexpr double kCostK1 = 1.58, kCostK2 = 1.90;   // the reference's round / step midpoints
int fail(int code, const char* msg) {
    q35_set_error(msg);
    return code;
}
}  // namespace

struct q35_mtp_policy {
    int k = 2, ceiling = 2, head = 0, count = 0, changes = 0;
    double cost1 = kCostK1, cost2 = kCostK2;
    double emit[kWindow] = {0.0}, cost[kWindow] = {0.0};
    long long rounds[3] = {0, 0, 0};
    double all_emit = 0.0, all_cost = 0.0;

    double round_cost(int kr) const { return kr >= 2 ? cost2 : cost1; }
    double est() const {
        double e = 0.0, c = 0.0;
        for (int i = 0; i < count; ++i) { e += emit[i]; c += cost[i]; }
        return c > 0.0 ? e / c : 0.0;
    }
};

extern "C" {

int q35_mtp_policy_create(int start_k, double cost_k1, double cost_k2, q35_mtp_policy** out) {
    if (!out) return fail(Q35_ERR_ARG, "q35_mtp_policy_create: null output");
    if (start_k < 0 || start_k > 2) return fail(Q35_ERR_ARG, "q35_mtp_policy_create: start_k is 0, 1 or 2");
    auto* p = new (std::nothrow) q35_mtp_policy();
    if (!p) return fail(Q35_ERR_STATE, "q35_mtp_policy_create: out of host memory");
    p->k = p->ceiling = start_k;
    if (cost_k1 > 0.0) p->cost1 = cost_k1;
    if (cost_k2 > 0.0) p->cost2 = cost_k2;
    *out = p;
    return Q35_OK;
}

int q35_mtp_policy_free(q35_mtp_policy* p) {
    delete p;
    return Q35_OK;
}

int q35_mtp_policy_k(const q35_mtp_policy* p, int32_t* k) {
    if (!p || !k) return fail(Q35_ERR_ARG, "q35_mtp_policy_k: null argument");
    *k = p->k;
    return Q35_OK;
}

int q35_mtp_policy_note(q35_mtp_policy* p, int k_round, int emitted, int32_t* change, double* est) {
    if (!p) return fail(Q35_ERR_ARG, "q35_mtp_policy_note: null policy");
    if (k_round < 0 || k_round > 2 || emitted < 0)
        return fail(Q35_ERR_ARG, "q35_mtp_policy_note: k_round is 0 .. 2 and emitted >= 0");
    if (change) change[0] = change[1] = change[2] = -1;
    p->rounds[k_round]++;
    if (p->k == 0) {                                   // abandoned: sticky
        if (est) *est = p->est();
        return Q35_OK;
    }
    const double c = p->round_cost(k_round);
    p->emit[p->head] = emitted;
    p->cost[p->head] = c;
    p->head = (p->head + 1) % kWindow;
    if (p->count < kWindow) p->count++;
    p->all_emit += emitted;
    p->all_cost += c;
    const double e = p->est();
    if (est) *est = e;
    if (p->count < (p->k >= 2 ? kMinObserve : kMinObserveAbandon)) return Q35_OK;
    int to = p->k;
    if (p->k >= 2 && e < kDemote) to = p->k - 1;
    else if (p->k == 1 && e < kAbandon) to = 0;
    if (to == p->k) return Q35_OK;
    if (change) { change[0] = p->k; change[1] = to; change[2] = p->count; }
    p->k = to;
    p->changes++;
    p->head = 0;
    p->count = 0;
    return Q35_OK;
}

}  // extern "C"
