// Launch-plan overrides for tests and measurements.  The library reads no environment variables: every plan uses
// its built-in defaults unless a caller has set an override through mi_tuning_set (include/mi355moe.h), an explicit
// process-wide hook meant for tests and measurement runs, never for production calls.
#pragma once

namespace mi {

// One entry per override; a choose_shape family is three consecutive entries: the split count S, then _RTW and _AL.
enum Knob : int {
    kTuneS1, kTuneS1Rtw, kTuneS1Al,          // grouped decode, gate/up: splits, row tiles per wavefront, alignment
    kTuneS2, kTuneS2Rtw, kTuneS2Al,          // grouped decode, down
    kTuneFS1, kTuneFS1Rtw, kTuneFS1Al,       // one-launch decode, gate/up tasks
    kTuneFS2, kTuneFS2Rtw, kTuneFS2Al,       // one-launch decode, down tasks
    kTuneSMV, kTuneSMVRtw, kTuneSMVAl,       // matvec
    kTuneMS1, kTuneMS1Rtw, kTuneMS2, kTuneMS2Rtw, kTuneMGMax,   // CU-balanced multi-token launches
    kTuneCS1, kTuneCS1Rtw, kTuneCS2, kTuneCS2Rtw,               // CU-balanced one-token launches
    kTuneCustream, kTuneCumulti, kTunePersistAbove, kTuneFuseSwiglu, kTuneCuFormH, kTuneSpinLimit, kTuneCuCombine,
    kTuneI8S, kTuneI8Waves, kTuneI8Fuse,
    kTuneCount
};

// The override of `k`, or `dflt` when none is set.
int tuning(Knob k, int dflt);

}  // namespace mi
