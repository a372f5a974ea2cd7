// launch_prefill.h -- the launchers of the interleaved prefill kernel (k_gemm_ilv8): template
// definitions, instantiated by launch_prefill.hip for the ladder's rows (prefill.inc) -- or by
// any other translation unit built with the same scheduler flag (the plugin's tuning
// harness instantiates its candidates from this header).
#pragma once
#include "launch.h"

namespace tempo {
namespace gen8 {

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int BFMT, int SPLIT>
static void run_ilv8(const W8A16Params& p, hipStream_t s, dim3 grid, float* ws, int splits) {
  hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, BFMT, SPLIT>), grid,
                     dim3(WM * WN * 64), 0, s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale,
                     p.zero, p.C, p.M, p.N, p.K, p.lda, p.ldw, p.ldc, ws, splits);
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int SW, int MINKT>
hipError_t launch_ilv8(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const int splits = split_count(nm * nn, p.K / BK, SW, MINKT);
  const size_t bytes = splits > 1 ? (size_t)splits * p.M * p.N * sizeof(float) : 0;
  if (w.need) {
    *w.need = bytes;
    return hipSuccess;
  }
  if (splits == 1) {
    if (p.fmt == 1)
      run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1, 0>(p, s, dim3(nm * nn), nullptr, 1);
    else
      run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2, 0>(p, s, dim3(nm * nn), nullptr, 1);
    return hipGetLastError();
  }
  float* ws = workspace_for(w, bytes, s);
  if (!ws) return hipErrorOutOfMemory;
  const dim3 grid(nm * nn * splits);
  if (p.fmt == 1)
    run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1, 1>(p, s, grid, ws, splits);
  else
    run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2, 1>(p, s, grid, ws, splits);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_reduce(ws, splits, p.M, p.N, p.C, p.ldc, s);
}

// Fused gate/up (EPI = 1): p.N is the output width; Wq, scale and zero hold 2N rows (gate, then
// up); each tile covers BN/2 output columns.  No split-K, no workspace.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv8_gu(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  const dim3 grid(((p.M + BM - 1) / BM) * (p.N / (BN / 2))), blk(WM * WN * 64);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1, 0, 1>), grid,
                       blk, 0, s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C,
                       p.M, p.N, p.K, p.lda, p.ldw, p.ldc, static_cast<float*>(nullptr), 1);
  else
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2, 0, 1>), grid,
                       blk, 0, s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C,
                       p.M, p.N, p.K, p.lda, p.ldw, p.ldc, static_cast<float*>(nullptr), 1);
  return hipGetLastError();
}

}  // namespace gen8
}  // namespace tempo
