// tune.cpp -- the dispatcher's tunable parameters.
//
// Every choice the planners can be steered in (kernel families that can be
// switched off, forced tile configurations, split counts, launch shapes) has
// one entry here with its default.  The shipped library takes them from this
// table only: a process changes one explicitly with dnnopt_hip_set_tunable()
// (the tests of the alternative code paths and tuning runs do), never by
// inheriting an environment variable.  A build with -DDNNOPT_TUNING=1 also
// seeds the table once, at its first use, from DNNOPT_<NAME> environment
// variables, for sweeps that drive an unmodified program.
#include <atomic>
#include <climits>
#include <mutex>
#include <stdlib.h>

#include "dnnopt_hip.h"
#include "host.h"

namespace dnnopt_hip {

namespace {

struct TuneDef {
    const char* env;  // DNNOPT_<NAME> (tuning builds only)
    int dflt;
    bool flag;        // parsed as a switch: "0" turns it off
    int lo = 1;       // smallest value the environment may set (not for switches)
};

// Indexed by Tunable (host.h); values are documented there.
constexpr TuneDef kDefs[kTuneCount] = {
    {"DNNOPT_Q8B", 1, true},           {"DNNOPT_KOUTER", 1, true},
    {"DNNOPT_KOUTER_WGS_PER_CU", 1, false}, {"DNNOPT_WAVES_PER_CU", 8, false},
    {"DNNOPT_SKINNY_NW", 0, false},    {"DNNOPT_SKINNY_WGS_PER_CU", 1, false},
    {"DNNOPT_MAX_SPLITS", 256, false}, {"DNNOPT_SPLIT_REDUCE", 1, false, 0},
    {"DNNOPT_SKINNY_WGS", 0, false},   {"DNNOPT_TILE_SPLITS", 0, false},
    {"DNNOPT_TILE_CFG", 0, false},     {"DNNOPT_TILE_TICKET", 0, false},
    {"DNNOPT_S8_CFG", -1, false, 0},      {"DNNOPT_S8_ROWDOT", 1, true},
    {"DNNOPT_S8_SPLITS", 0, false},    {"DNNOPT_ROWDOT_KW", 0, false},
    {"DNNOPT_TALL_RT", 0, false},      {"DNNOPT_TALL_WGS_PER_CU", 1, false},
    {"DNNOPT_TALL", 1, true},          {"DNNOPT_WIDE", 0, true},
};

std::atomic<int> g_val[kTuneCount];
std::once_flag g_init;

void init_table() {
    for (int i = 0; i < kTuneCount; ++i) {
        int v = kDefs[i].dflt;
#if DNNOPT_TUNING
        // A whole decimal integer only; anything else leaves the default.
        const char* e = getenv(kDefs[i].env);
        char* end = nullptr;
        const long x = e && *e ? strtol(e, &end, 10) : 0;
        if (e && *e && end && *end == '\0' && x >= INT_MIN && x <= INT_MAX) {
            if (kDefs[i].flag) v = x != 0 ? 1 : 0;
            else if (x >= kDefs[i].lo) v = (int)x;
        }
#endif
        g_val[i].store(v, std::memory_order_relaxed);
    }
}

}  // namespace

int tunable(Tunable t) {
    std::call_once(g_init, init_table);
    return g_val[t].load(std::memory_order_relaxed);
}

int tunable_default(Tunable t) { return kDefs[t].dflt; }

}  // namespace dnnopt_hip

extern "C" int dnnopt_hip_set_tunable(int key, int value, int* previous) {
    using namespace dnnopt_hip;
    if (key < 0 || key >= kTuneCount) return DNNOPT_ERR_INVALID_ARG;
    std::call_once(g_init, init_table);
    const int old = g_val[key].exchange(value, std::memory_order_relaxed);
    if (previous) *previous = old;
    return DNNOPT_OK;
}

extern "C" int dnnopt_hip_get_tunable(int key, int* value) {
    using namespace dnnopt_hip;
    if (key < 0 || key >= kTuneCount || !value) return DNNOPT_ERR_INVALID_ARG;
    *value = tunable(static_cast<Tunable>(key));
    return DNNOPT_OK;
}
