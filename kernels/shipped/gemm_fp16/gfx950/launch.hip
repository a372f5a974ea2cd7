// launch.hip -- the one translation unit of the shipped gemm_fp16 for gfx950.  The generated
// ladder (dispatch.inc) becomes the body of launch() here, so the kernels are instantiated
// exactly once (reference: kernels/shipped/gemm_fp16/sm_70/launch.cu:5-22).
//
// Build (host tree): hipcc -O3 -std=c++17 --offload-arch=gfx950
//                    -Xclang -target-feature -Xclang -packed-fp32-ops -c launch.hip
#include <mutex>

#include "launch.h"

namespace tempo {
namespace gen {

hipError_t workspace(float** partials, unsigned** counters) {
  static std::mutex mu;
  static void* ws[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!ws[dev]) {
    const size_t bytes = kWsPartialBytes + kWsCounterCount * sizeof(unsigned);
    void* p = nullptr;
    e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return e;
    // counters must start at zero; every completed call leaves them at zero again
    e = hipMemset(static_cast<char*>(p) + kWsPartialBytes, 0, kWsCounterCount * sizeof(unsigned));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      (void)hipFree(p);
      return e;
    }
    ws[dev] = p;
  }
  *partials = static_cast<float*>(ws[dev]);
  *counters = reinterpret_cast<unsigned*>(static_cast<char*>(ws[dev]) + kWsPartialBytes);
  return hipSuccess;
}

hipError_t launch(const GemmParams& p, hipStream_t s) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
#define TEMPO_ROW(band, fit, fn, tag) \
  if (band) return (fit) ? fn(p, s) : hipErrorInvalidConfiguration;
#define TEMPO_FALLBACK_ROW return hipErrorInvalidConfiguration;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

const char* route(const GemmParams& p) {
  if (!applicable(p)) return nullptr;
#define TEMPO_ROW(band, fit, fn, tag) \
  if (band) return (fit) ? tag : nullptr;
#define TEMPO_FALLBACK_ROW return nullptr;
#include "dispatch.inc"
#undef TEMPO_ROW
#undef TEMPO_FALLBACK_ROW
}

}  // namespace gen
}  // namespace tempo
