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
                     p.zero, p.C, p.M, p.N, p.K, p.lda, p.ldw, p.ldc, ws, splits, p.N);
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
  hipError_t werr = hipSuccess;
  float* ws = workspace_for(w, bytes, s, &werr);
  if (!ws) return werr;
  const dim3 grid(nm * nn * splits);
  if (p.fmt == 1)
    run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1, 1>(p, s, grid, ws, splits);
  else
    run_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2, 1>(p, s, grid, ws, splits);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_reduce(ws, splits, p.M, p.N, p.C, p.ldc, s);
}

// N in two parts, for grids whose last round of BM x BN tiles is at most a quarter full (1088
// tiles of 256 x 256 at (2048, 34816): four rounds and 64 tiles; 272 tiles of 128 x 128 at
// (128, 34816): one round and 16): the whole rounds run as they are on the leading columns, and
// the remaining columns run as a launch of their own on TBM x TBN tiles -- four or more times as
// many of them (no split), or split-K towards TSW workgroups.  ilv8_tail_cols (launch.h) gives
// the split.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES, int TSW, int TMINKT>
hipError_t launch_ilv8_tail(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  static_assert(BN % TBN == 0 && (TSW > 0 || (BM * BN) / (TBM * TBN) >= 4),
                "tail tiles: a quarter of the size or less, or split-K");
  const int n0 = ilv8_tail_cols<BM, BN>(p);
  W8A16Params a = p, b = p;
  a.N = n0;
  b.N = p.N - n0;
  b.Wq = static_cast<const uint8_t*>(p.Wq) + (long)n0 * p.ldw;
  b.scale = p.scale + (p.fmt == 1 ? (long)n0 : (long)n0 * (p.K / p.group));
  b.zero = p.zero ? p.zero + (long)n0 * (p.K / p.group) : nullptr;
  b.C = p.C + n0;
  if (w.need) {  // the tail's split-K workspace, if any
    if (n0 == 0) *w.need = 0;
    else return launch_ilv8<TBM, TBN, TBK, TWM, TWN, TSTAGES, GROUP, XCD, RSP, TSW, TMINKT>(b, s, w);
    return hipSuccess;
  }
  if (n0 == 0) return launch_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 0, 0>(p, s, w);
  const hipError_t e = launch_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 0, 0>(a, s, w);
  if (e != hipSuccess) return e;
  return launch_ilv8<TBM, TBN, TBK, TWM, TWN, TSTAGES, GROUP, XCD, RSP, TSW, TMINKT>(b, s, w);
}

// Fused gate/up (EPI = 1): p.N is the output width; Wq, scale and zero hold 2N rows (gate, then
// up); each tile covers BN/2 output columns.  No split-K, no workspace.  `up`: the row of the
// first up row relative to Wq (p.N for a launch over all output columns).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv8_gu_part(const W8A16Params& p, hipStream_t s, int up) {
  const dim3 grid(((p.M + BM - 1) / BM) * (p.N / (BN / 2))), blk(WM * WN * 64);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1, 0, 1>), grid,
                       blk, 0, s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C,
                       p.M, p.N, p.K, p.lda, p.ldw, p.ldc, static_cast<float*>(nullptr), 1, up);
  else
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2, 0, 1>), grid,
                       blk, 0, s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C,
                       p.M, p.N, p.K, p.lda, p.ldw, p.ldc, static_cast<float*>(nullptr), 1, up);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv8_gu(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  return launch_ilv8_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(p, s, p.N);
}

// The fused gate/up row with the output columns in two parts, as launch_ilv8_tail (unsplit
// tail tiles): the whole rounds of BM x BN/2-column tiles, then the remaining columns on
// TBM x TBN/2-column tiles; both parts read their up rows p.N rows past their gate rows.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES, int TSW, int TMINKT>
hipError_t launch_ilv8_gu_tail(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  static_assert(TSW == 0 && BN % TBN == 0 && (BM * BN) / (TBM * TBN) >= 4,
                "unsplit tail tiles of a quarter of the size or less");
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  const int n0 = ilv8_tail_cols<BM, BN / 2>(p);
  if (n0 == 0) return launch_ilv8_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(p, s, p.N);
  W8A16Params a = p, b = p;
  a.N = n0;
  b.N = p.N - n0;
  b.Wq = static_cast<const uint8_t*>(p.Wq) + (long)n0 * p.ldw;
  b.scale = p.scale + (p.fmt == 1 ? (long)n0 : (long)n0 * (p.K / p.group));
  b.zero = p.zero ? p.zero + (long)n0 * (p.K / p.group) : nullptr;
  b.C = p.C + n0;
  const hipError_t e = launch_ilv8_gu_part<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP>(a, s, p.N);
  if (e != hipSuccess) return e;
  return launch_ilv8_gu_part<TBM, TBN, TBK, TWM, TWN, TSTAGES, GROUP, XCD, RSP>(b, s, p.N);
}

}  // namespace gen8
}  // namespace tempo
