// tune_harness.hip -- measuring harness of the variant driver (tempo/plugins/gfx950/tune.py).
//
// Reference pattern: tempo/plugins/sm70/skeletons/gemm_hmma884/harness.cu:35-103,161-268 (a table
// of candidate instantiations, gate before stopwatch).  Here the harness is a shared library and
// the gate and the stopwatch live in tune.py (torch for device memory and HIP events); this file
// only instantiates the candidates and exposes them through a C ABI.
//
// Built by tune.py from one delivery's own launchers, so a candidate runs exactly the code a
// ladder row would run:
//   hipcc ... -DTEMPO_NS=gen -DTEMPO_PARAMS=GemmParams -I <plan dir> -I <delivery dir> -c
//         tune_harness.hip
// <plan dir>/cands.inc holds one TEMPO_CAND(id, "tag", fit, (launcher)) per candidate, written by
// tune.py with the delivery's own gen_dispatch.py (the same launcher expressions and fit
// predicates as dispatch.inc); the prefill kinds' launchers are instantiated by a second
// translation unit of the plan (cands_prefill.inc) built with their scheduler flag.
//
// C ABI (P = the delivery's POD params, the layout of TempoGemmParams / TempoW8A16Params):
//   int         tempo_tune_count(void)
//   int         tempo_tune_id(int i)            candidate id of table entry i
//   const char* tempo_tune_tag(int i)
//   int         tempo_tune_fits(int i, const P* p)
//   int         tempo_tune_launch(int i, const P* p, void* stream)   hipError_t; workspace from the
//                                                                   delivery's pool
//   size_t      tempo_tune_workspace(int i, const P* p)
//   int         tempo_tune_mfma_peak(int waves_per_simd, int iters, float* us_out, void* stream)
//                 MFMA-only throughput probe (operands in registers, no memory traffic)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

#ifndef TEMPO_NS
#error "TEMPO_NS (the delivery's namespace) must be defined"
#endif

namespace tempo {
namespace TEMPO_NS {
namespace tune {

using P = TEMPO_PARAMS;
struct Cand {
  int id;
  const char* tag;
  bool (*fits)(const P&);
  hipError_t (*run)(const P&, hipStream_t, const Workspace&);
};

#define TEMPO_CAND(id, tag, fit, fn)                                                        \
  Cand{id, tag, [](const P& p) -> bool { return (fit); },                                   \
       [](const P& p, hipStream_t s, const Workspace& w) -> hipError_t {                    \
         return call_row(fn, p, s, w);                                                      \
       }},

static const Cand kCands[] = {
#include "cands.inc"
};
#undef TEMPO_CAND

constexpr int kCount = sizeof(kCands) / sizeof(kCands[0]);

// MFMA-only probe: 4 independent 16x16x32 accumulator chains per wave, `iters` rounds, operands
// in registers; the sum is stored so the work cannot be removed.
__global__ __launch_bounds__(256) void k_mfma_peak(float* out, int iters, float seed) {
  f32x4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[c][v] = 0.f;
  f16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(seed * (float)(threadIdx.x + i));
    b[i] = (_Float16)(seed * (float)(i - (int)threadIdx.x));
  }
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) s += acc[c][v];
  out[(long)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace tune
}  // namespace TEMPO_NS
}  // namespace tempo

using tempo::TEMPO_NS::tune::kCands;
using tempo::TEMPO_NS::tune::kCount;
using TuneP = tempo::TEMPO_NS::tune::P;

extern "C" {

int tempo_tune_count(void) { return kCount; }

int tempo_tune_id(int i) { return (i >= 0 && i < kCount) ? kCands[i].id : -1; }

const char* tempo_tune_tag(int i) { return (i >= 0 && i < kCount) ? kCands[i].tag : ""; }

int tempo_tune_fits(int i, const TuneP* p) {
  if (i < 0 || i >= kCount || !p) return 0;
  return tempo::TEMPO_NS::applicable(*p) && kCands[i].fits(*p) ? 1 : 0;
}

int tempo_tune_launch(int i, const TuneP* p, void* stream) {
  if (!tempo_tune_fits(i, p)) return (int)hipErrorInvalidConfiguration;
  tempo::TEMPO_NS::Workspace w;
  w.pool = true;
  return (int)kCands[i].run(*p, static_cast<hipStream_t>(stream), w);
}

size_t tempo_tune_workspace(int i, const TuneP* p) {
  if (!tempo_tune_fits(i, p)) return 0;
  size_t need = 0;
  tempo::TEMPO_NS::Workspace w;
  w.need = &need;
  return kCands[i].run(*p, nullptr, w) == hipSuccess ? need : 0;
}

// grid = 256 CUs x 4 SIMDs x waves_per_simd waves of 64 lanes (4 waves per workgroup) -- four
// rounds of them, so the part is busy long enough to time.
int tempo_tune_mfma_peak(int waves_per_simd, int iters, float* us_out, float* scratch,
                         void* stream) {
  if (waves_per_simd < 1 || waves_per_simd > 8 || iters < 1 || !us_out || !scratch)
    return (int)hipErrorInvalidValue;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = 256 * waves_per_simd * 4;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    return (int)hipErrorUnknown;
  hipLaunchKernelGGL(tempo::TEMPO_NS::tune::k_mfma_peak, dim3(grid), dim3(256), 0, s, scratch,
                     iters, 1e-3f);
  (void)hipEventRecord(e0, s);
  hipLaunchKernelGGL(tempo::TEMPO_NS::tune::k_mfma_peak, dim3(grid), dim3(256), 0, s, scratch,
                     iters, 1e-3f);
  (void)hipEventRecord(e1, s);
  hipError_t e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  *us_out = ms * 1e3f;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return (int)e;
}

}  // extern "C"
