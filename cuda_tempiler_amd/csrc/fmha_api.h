// fmha_api.h -- host interface of the causal FMHA forward (implementation: fmha.hip, kernel:
// tempo/plugins/gfx950/skeletons/fmha_fwd/kernel.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "tempo_gfx950.h"

namespace tempo_fmha {
bool applicable(const TempoFmhaParams& p);
hipError_t launch(const TempoFmhaParams& p, hipStream_t s);
}  // namespace tempo_fmha
