// launch_prefill.h -- the launchers of the interleaved prefill kernel (k_gemm_ilv): template
// definitions, instantiated by launch_prefill.hip for the ladder's rows (prefill.inc) -- or by
// any other translation unit built with the same scheduler flag (the plugin's tuning
// harness instantiates its candidates from this header).
#pragma once
#include "launch.h"

namespace tempo {
namespace gen {

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int SW, int MINKT>
hipError_t launch_ilv(const GemmParams& p, hipStream_t s, const Workspace& w) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const int splits = split_count(nm * nn, p.K / BK, SW, MINKT);
  const size_t bytes = splits > 1 ? (size_t)splits * p.M * p.N * sizeof(float) : 0;
  if (w.need) {
    *w.need = bytes;
    return hipSuccess;
  }
  const dim3 blk(WM * WN * 64);
  if (splits == 1) {
    hipLaunchKernelGGL((k_gemm_ilv<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 0>),
                       dim3(nm * nn), blk, 0, s, p.A, p.B, p.C, p.M, p.N, p.K, p.lda, p.ldb,
                       p.ldc, static_cast<float*>(nullptr), 1, p.N);
    return hipGetLastError();
  }
  hipError_t werr = hipSuccess;
  float* ws = workspace_for(w, bytes, s, &werr);
  if (!ws) return werr;
  hipLaunchKernelGGL((k_gemm_ilv<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1>),
                     dim3(nm * nn * splits), blk, 0, s, p.A, p.B, p.C, p.M, p.N, p.K, p.lda, p.ldb,
                     p.ldc, ws, splits, p.N);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_reduce(ws, splits, p.M, p.N, p.C, p.ldc, s);
}

// Fused gate/up (EPI = 1): p.N is the output width and B holds 2N rows (gate, then up); each
// tile covers BN/2 output columns.  No split-K, no workspace.  `up`: the row of the first up row
// relative to B (p.N for a launch over all output columns).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv_gu_part(const GemmParams& p, hipStream_t s, int up) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / (BN / 2);
  hipLaunchKernelGGL((k_gemm_ilv<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 0, 1>),
                     dim3(nm * nn), dim3(WM * WN * 64), 0, s, p.A, p.B, p.C, p.M, p.N, p.K, p.lda,
                     p.ldb, p.ldc, static_cast<float*>(nullptr), 1, up);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv_gu(const GemmParams& p, hipStream_t s, const Workspace& w) {
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  return launch_ilv_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(p, s, p.N);
}

// The fused gate/up row with the output columns in two parts: where the last round of tiles
// (BN/2 output columns each) is at most a quarter full, the whole rounds run on the leading
// columns and the remaining columns on TBM x TBN/2-column tiles -- four or more times as many --
// as a launch of their own; both parts read their up rows p.N rows past their gate rows.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES>
hipError_t launch_ilv_gu_tail(const GemmParams& p, hipStream_t s, const Workspace& w) {
  static_assert(BN % TBN == 0 && (BM * BN) / (TBM * TBN) >= 4, "tail tiles of a quarter or less");
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  constexpr int CUS = 256, BNO = BN / 2;
  const int nm = (p.M + BM - 1) / BM, nn = p.N / BNO;
  const int tiles = nm * nn, whole = tiles / CUS * CUS;
  if (whole == 0 || whole % nm || whole / nm == nn || 4 * (tiles - whole) > CUS)
    return launch_ilv_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(p, s, p.N);
  const int n0 = whole / nm * BNO;
  GemmParams a = p, b = p;
  a.N = n0;
  b.N = p.N - n0;
  b.B = p.B + (long)n0 * p.ldb;
  b.C = p.C + n0;
  const hipError_t e = launch_ilv_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(a, s, p.N);
  if (e != hipSuccess) return e;
  return launch_ilv_gu_part<TBM, TBN, TBK, TWM, TWN, TSTAGES, GROUP, XCD, RSP>(b, s, p.N);
}

}  // namespace gen
}  // namespace tempo
