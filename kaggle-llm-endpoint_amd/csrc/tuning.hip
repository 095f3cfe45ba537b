// The launch-plan override table behind mi_tuning_set / mi_tuning_reset (tuning.h).  Host code only.
#include <limits.h>
#include <string.h>

#include <atomic>

#include "mi355moe.h"
#include "tuning.h"

namespace mi {
namespace {

constexpr int kUnset = INT_MIN;

struct Entry {
    const char *name;
    Knob knob;
};

// The names mi_tuning_set accepts (the enum's order).
const Entry kNames[] = {
    {"S1", kTuneS1}, {"S1_RTW", kTuneS1Rtw}, {"S1_AL", kTuneS1Al},
    {"S2", kTuneS2}, {"S2_RTW", kTuneS2Rtw}, {"S2_AL", kTuneS2Al},
    {"FS1", kTuneFS1}, {"FS1_RTW", kTuneFS1Rtw}, {"FS1_AL", kTuneFS1Al},
    {"FS2", kTuneFS2}, {"FS2_RTW", kTuneFS2Rtw}, {"FS2_AL", kTuneFS2Al},
    {"SMV", kTuneSMV}, {"SMV_RTW", kTuneSMVRtw}, {"SMV_AL", kTuneSMVAl},
    {"MS1", kTuneMS1}, {"MS1_RTW", kTuneMS1Rtw}, {"MS2", kTuneMS2}, {"MS2_RTW", kTuneMS2Rtw}, {"MGMAX", kTuneMGMax},
    {"CS1", kTuneCS1}, {"CS1_RTW", kTuneCS1Rtw}, {"CS2", kTuneCS2}, {"CS2_RTW", kTuneCS2Rtw},
    {"CUSTREAM", kTuneCustream}, {"CUMULTI", kTuneCumulti}, {"PERSIST_ABOVE", kTunePersistAbove},
    {"FUSE_SWIGLU", kTuneFuseSwiglu}, {"CU_FORM_H", kTuneCuFormH}, {"SPIN_LIMIT", kTuneSpinLimit},
    {"CU_COMBINE", kTuneCuCombine},
    {"I8S", kTuneI8S}, {"I8_WAVES", kTuneI8Waves}, {"I8_FUSE", kTuneI8Fuse},
};
static_assert(sizeof(kNames) / sizeof(kNames[0]) == kTuneCount, "every knob has a name");

std::atomic<int> g_value[kTuneCount];
std::atomic<int> g_any{0};       // any override set (the common case, none, costs one load)

struct Init {
    Init() {
        for (auto &v : g_value) v.store(kUnset, std::memory_order_relaxed);
    }
} g_init;

}  // namespace

int tuning(Knob k, int dflt) {
    if (!g_any.load(std::memory_order_relaxed)) return dflt;
    const int v = g_value[k].load(std::memory_order_relaxed);
    return v == kUnset ? dflt : v;
}

}  // namespace mi

extern "C" int mi_tuning_set(const char *name, int32_t value) {
    if (!name || value == mi::kUnset) return MI_ERR_ARG;
    for (const auto &e : mi::kNames)
        if (strcmp(e.name, name) == 0) {
            mi::g_value[e.knob].store(value, std::memory_order_relaxed);
            mi::g_any.store(1, std::memory_order_relaxed);
            return MI_OK;
        }
    return MI_ERR_ARG;
}

extern "C" void mi_tuning_reset(void) {
    for (auto &v : mi::g_value) v.store(mi::kUnset, std::memory_order_relaxed);
    mi::g_any.store(0, std::memory_order_relaxed);
}
