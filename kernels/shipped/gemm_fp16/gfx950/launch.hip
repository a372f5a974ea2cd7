// launch.hip -- the one translation unit of the shipped gemm_fp16 for gfx950.  The generated
// ladder (dispatch.inc) becomes the body of launch() here, so the kernels are instantiated
// exactly once (reference: kernels/shipped/gemm_fp16/sm_70/launch.cu:5-22).
//
// Build (host tree): hipcc -O3 -std=c++17 --offload-arch=gfx950
//                    -Xclang -target-feature -Xclang -packed-fp32-ops -c launch.hip
#include "launch.h"

namespace tempo {
namespace gen {

hipError_t launch_with(const GemmParams& p, hipStream_t s, const Workspace& w) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return call_row(fn, p, s, w);
#define TEMPO_FALLBACK_ROW return hipErrorInvalidConfiguration;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

hipError_t launch(const GemmParams& p, hipStream_t s) {
  Workspace w;
  w.pool = true;
  return launch_with(p, s, w);
}

size_t workspace_bytes(const GemmParams& p) {
  size_t need = 0;
  Workspace w;
  w.need = &need;
  return launch_with(p, nullptr, w) == hipSuccess ? need : 0;
}

const char* route(const GemmParams& p) {
  if (!applicable(p)) return nullptr;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return tag;
#define TEMPO_FALLBACK_ROW return nullptr;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

hipError_t launch_gate_up(const GemmParams& p, hipStream_t s) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
  const Workspace w{};
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return call_row(fn, p, s, w);
#define TEMPO_FALLBACK_ROW return hipErrorInvalidConfiguration;
#include "dispatch_gate_up.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

const char* route_gate_up(const GemmParams& p) {
  if (!applicable(p)) return nullptr;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return tag;
#define TEMPO_FALLBACK_ROW return nullptr;
#include "dispatch_gate_up.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

}  // namespace gen
}  // namespace tempo
