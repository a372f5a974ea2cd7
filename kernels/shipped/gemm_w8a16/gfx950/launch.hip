// launch.hip -- the one translation unit of the shipped gemm_w8a16 for gfx950.  The generated
// ladder (dispatch.inc) becomes the body of launch() here, so the kernels are instantiated
// exactly once (pattern of kernels/shipped/gemm_fp16/sm_70/launch.cu:5-22).
//
// Build (host tree): hipcc -O3 -std=c++17 --offload-arch=gfx950
//                    -Xclang -target-feature -Xclang -packed-fp32-ops -c launch.hip
#include "launch.h"

namespace tempo {
namespace gen8 {

hipError_t launch_with(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return call_row(fn, p, s, w);
#define TEMPO_FALLBACK_ROW return hipErrorInvalidConfiguration;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

hipError_t launch(const W8A16Params& p, hipStream_t s) {
  Workspace w;
  w.pool = true;
  return launch_with(p, s, w);
}

size_t workspace_bytes(const W8A16Params& p) {
  size_t need = 0;
  Workspace w;
  w.need = &need;
  return launch_with(p, nullptr, w) == hipSuccess ? need : 0;
}

const char* route(const W8A16Params& p) {
  if (!applicable(p)) return nullptr;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return tag;
#define TEMPO_FALLBACK_ROW return nullptr;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

hipError_t launch_gate_up(const W8A16Params& p, hipStream_t s) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
  const Workspace w{};
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return call_row(fn, p, s, w);
#define TEMPO_FALLBACK_ROW return hipErrorInvalidConfiguration;
#include "dispatch_gate_up.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

const char* route_gate_up(const W8A16Params& p) {
  if (!applicable(p)) return nullptr;
#define TEMPO_ROW(band, fit, fn, tag) \
  if ((band) && (fit)) return tag;
#define TEMPO_FALLBACK_ROW return nullptr;
#include "dispatch_gate_up.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

}  // namespace gen8
}  // namespace tempo
