// Per-kernel timing with HIP events on the launch stream.
//
// While profiling is enabled every launch made through FEQ_LAUNCH is
// bracketed by two events recorded on the kernel's own stream; the summary
// call waits for the recorded events and aggregates elapsed time per kernel
// name.  Off by default: a disabled ProfScope costs one branch.  The state is
// process-global and not thread-safe (profile from one host thread).
#include "feq_internal.h"

#include <cstring>
#include <vector>

namespace feq {
namespace {

struct Rec {
    const char* name;
    hipEvent_t a, b;
};

std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_pool;
bool g_on = false;

hipEvent_t take_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

ProfScope::ProfScope(const char* name, hipStream_t s) : name_(name), s_(s), a_(nullptr) {
    if (!g_on) return;
    a_ = take_event();
    if (a_ && hipEventRecord(a_, s_) != hipSuccess) {
        g_pool.push_back(a_);
        a_ = nullptr;
    }
}

ProfScope::~ProfScope() {
    if (!a_) return;
    hipEvent_t b = take_event();
    if (!b || hipEventRecord(b, s_) != hipSuccess) {
        if (b) g_pool.push_back(b);
        g_pool.push_back(a_);
        return;
    }
    g_recs.push_back({name_, a_, b});
}

}  // namespace feq

using namespace feq;

extern "C" int feq_profile_enable(int on) {
    g_on = on != 0;
    return FEQ_OK;
}

extern "C" int feq_profile_summary(char* buf, size_t len) {
    struct Agg {
        const char* name;
        int calls;
        double ms;
    };
    std::vector<Agg> agg;
    int rc = FEQ_OK;
    for (const Rec& r : g_recs) {
        float ms = 0.0f;
        if (rc == FEQ_OK) {
            hipError_t e = hipEventSynchronize(r.b);
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
            if (e != hipSuccess) rc = fail(FEQ_ERR_HIP, "event timing failed: %s", hipGetErrorString(e));
        }
        size_t k = 0;
        while (k < agg.size() && std::strcmp(agg[k].name, r.name) != 0) ++k;
        if (k == agg.size()) agg.push_back({r.name, 0, 0.0});
        agg[k].calls += 1;
        agg[k].ms += ms;
        g_pool.push_back(r.a);
        g_pool.push_back(r.b);
    }
    g_recs.clear();
    if (rc != FEQ_OK) return rc;
    size_t used = 0;
    if (buf && len) buf[0] = '\0';
    for (const Agg& a : agg) {
        char line[256];
        const int n = snprintf(line, sizeof(line), "%s\t%d\t%.6f\n", a.name, a.calls, a.ms);
        if (!buf || used + n + 1 > len) return fail(FEQ_ERR_INVALID, "summary buffer too small");
        std::memcpy(buf + used, line, n + 1);
        used += n;
    }
    return FEQ_OK;
}
