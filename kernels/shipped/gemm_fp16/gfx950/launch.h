// launch.h -- kernel/framework boundary of the shipped gemm_fp16 for gfx950.
//
// Plain POD and pointers only, no framework type (reference:
// kernels/shipped/gemm_fp16/sm_70/launch.cuh:5-8,20-26).  The call is asynchronous on the
// given stream, never synchronises, and the caller owns every buffer.  A shape the ladder
// does not cover returns hipErrorInvalidConfiguration: "take your own path" (dispatch.inc).
//
// Split-K rows (narrow N, long K) add fp32 partial sums of the k ranges in a workspace and reduce
// them with a second kernel on the same stream.  launch() takes that workspace from the
// delivery's pool -- one buffer per (device, stream), allocated on first use and grown when a
// larger shape needs it (hipMalloc; the old buffer is freed after a stream synchronise) -- so
// calls on different streams stay independent, and calls on one stream are ordered by it.
// launch_with() takes the caller's workspace instead and never allocates; no other row touches a
// workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel.hip"

namespace tempo {
namespace gen {

struct GemmParams {
  const _Float16* A;  // [M][lda], k contiguous
  const _Float16* B;  // [N][ldb], k contiguous (C = A . B^T)
  _Float16* C;        // [M][ldc]
  int M, N, K;
  int lda, ldb, ldc;  // row strides in elements
};

// k split of the streaming kernel: waves per workgroup (each takes one contiguous k chunk, the
// workgroup reduces through LDS).  Aim for about 8 waves per CU over the machine's 256 CUs,
// at most 8 waves per workgroup, every chunk a whole number of pipeline stages.
inline void stream_split(int N, int K, int R, int U, int* S_out, int* chunk_out) {
  const int slabs = N / (16 * R);
  const int stages = K / (64 * U);
  int S = (2048 + slabs - 1) / slabs;
  if (S > 8) S = 8;
  if (S > stages) S = stages;
  if (S < 1) S = 1;
  const int per = (stages + S - 1) / S;  // stages per wave
  S = (stages + per - 1) / per;
  *S_out = S;
  *chunk_out = per * 64 * U;
}

// Activations staged in LDS (ALDS rows) only while M*(2K+16) bytes stay within this budget.
constexpr size_t kStreamActLds = 96 * 1024;

// EPI = 1: fused gate/up epilogue -- p.N is the output width, B holds 2N rows (gate, then up)
// and C = silu(A.B[0..N)^T) * (A.B[N..2N)^T); each wave carries 2R row groups.
template <int MB, int R, int U, int ALDS, int EPI = 0>
inline hipError_t launch_stream(const GemmParams& p, hipStream_t s) {
  constexpr int RR = EPI ? 2 * R : R;
  StreamArgs a;
  a.A = p.A;
  a.B = p.B;
  a.scale = nullptr;
  a.zero = nullptr;
  a.C = p.C;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.lda = p.lda;
  a.ldb = p.ldb;
  a.ldc = p.ldc;
  a.group = 0;
  a.up = EPI ? p.N : 0;
  stream_split(p.N, p.K, R, U, &a.S, &a.chunk);
  const dim3 grid(p.N / (16 * R)), blk(64 * a.S);
  const size_t red = a.S > 1 ? (size_t)a.S * RR * MB * 64 * 16 : 0;
  const size_t act = (size_t)p.M * (2 * (size_t)p.K + 16);
  if (ALDS && act <= kStreamActLds)
    hipLaunchKernelGGL((k_stream<MB, R, U, 0, 1, EPI>), grid, blk, act + red, s, a);
  else
    hipLaunchKernelGGL((k_stream<MB, R, U, 0, 0, EPI>), grid, blk, red, s, a);
  return hipGetLastError();
}

// k-chunks of the shared-activation kernel: about 2048 waves over the part, at most TPB/64 waves
// per workgroup (TPB = the kernel's launch bound), the stage count divisible by the chunk count, and the activation rings of every
// chunk plus the reduction within the 160 KiB of LDS.
// RR: row groups per wave (2R with the fused gate/up epilogue; 0 = R).
inline void shared_split(int N, int K, int MB, int R, int U, int SN, int TPB, int* SK_out,
                         int* chunk_out, size_t* lds_out, int RR = 0) {
  if (RR == 0) RR = R;
  const int stages = K / (64 * U);
  const int wgs = N / (16 * R * SN);
  int SK = (2048 + wgs * SN - 1) / (wgs * SN);
  if (SK > TPB / 64 / SN) SK = TPB / 64 / SN;
  if (SK < 1) SK = 1;
  const size_t stage = (size_t)16 * MB * 128 * U;
  auto lds = [&](int sk) {
    return (size_t)sk * 2 * stage + (sk > 1 ? (size_t)SN * sk * RR * MB * 1024 : 0);
  };
  while (SK > 1 && (stages % SK != 0 || lds(SK) > 160 * 1024)) --SK;
  *SK_out = SK;
  *chunk_out = stages / SK * 64 * U;
  *lds_out = lds(SK);
}

template <int MB, int R, int U, int SN, int TPB, int EPI = 0>
inline hipError_t launch_shared(const GemmParams& p, hipStream_t s) {
  StreamArgs a;
  a.A = p.A;
  a.B = p.B;
  a.scale = nullptr;
  a.zero = nullptr;
  a.C = p.C;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.lda = p.lda;
  a.ldb = p.ldb;
  a.ldc = p.ldc;
  a.group = 0;
  a.up = EPI ? p.N : 0;
  size_t lds = 0;
  // EPI: the slab waves pair up (gate, up), so the work is that of the plain kernel over 2N rows
  const int rows = EPI ? 2 * p.N : p.N;
  shared_split(rows, p.K, MB, R, U, SN, TPB, &a.S, &a.chunk, &lds);
  const dim3 grid(rows / (16 * R * SN)), blk(64 * SN * a.S);
  hipLaunchKernelGGL((k_stream_sh<MB, R, U, 0, SN, TPB, EPI>), grid, blk, lds, s, a);
  return hipGetLastError();
}

// k split of the line kernel (k_stream_line): `wgs` workgroups of SN slab waves, each split
// into S k chunks of whole 128-k steps -- about `waves` waves over the part, at most `tpb`
// threads per workgroup (the kernel's launch bound), equal chunks when the slab waves share the activation ring (SN > 1:
// they pass the same barriers), the workgroup's rings (+ the fmt 2 metadata and the reduction)
// within the 160 KiB of LDS.  false: no split fits (the caller's own path).
template <class SL>
inline bool line_split(int wgs, int SN, int K, int waves, int* S_out, int* chunk_out, int* G_out,
                       size_t* lds_out, int tpb = 1024) {
  const int steps = K / 128;
  int S = (waves + wgs * SN - 1) / (wgs * SN);
  if (S > tpb / 64 / SN) S = tpb / 64 / SN;
  if (S > steps) S = steps;
  if (S < 1) S = 1;
  for (;; --S) {
    const int per = (steps + S - 1) / S;  // steps per wave
    const int s2 = (steps + per - 1) / per;
    const size_t lds = SL::lds(s2, per);
    if (lds <= 160 * 1024 && (SN == 1 || steps % s2 == 0)) {
      *S_out = s2;
      *chunk_out = per * 128;
      *G_out = per;
      *lds_out = lds;
      return true;
    }
    if (S == 1) return false;
  }
}

// k slices of the line kernel across workgroups (KS = the most a row allows): the count that
// spreads wgs x ks workgroups most evenly over the part's CUs, each slice a whole number of
// 128-k steps and at least kLineMinSteps of them.  A split pays a partial-sum pass and a second
// launch, so it is taken only when it lifts the evenness (workgroups / whole rounds of
// kLineCus) by at least 0.08 over no split; ties keep fewer slices.
constexpr int kLineCus = 256;  // CUs of the part (MI355X, MI350X)
constexpr int kLineMinSteps = 8;
inline int line_kslices(int wgs, int K, int KS) {
  const int steps = K / 128;
  auto even = [&](int ks) {
    const long w = (long)wgs * ks;
    return (double)w / (double)(((w + kLineCus - 1) / kLineCus) * kLineCus);
  };
  int best = 1;
  for (int ks = 2; ks <= KS; ++ks)
    if (steps % ks == 0 && steps / ks >= kLineMinSteps && even(ks) > even(best) + 1e-9) best = ks;
  return even(best) >= even(1) + 0.08 ? best : 1;
}

// The line kernel (whole-line nontemporal weight stream through per-wave LDS rings).  MB = 0:
// M = 1; MB = 1 / 2: M <= 16 / 32.  SN slab waves of a workgroup share one activation ring.
// EPI = 1: fused gate/up (p.N the output width, B 2N rows).
// KS > 1 (plain epilogue): up to KS k slices across workgroups (line_kslices), their fp32
// partial sums in the workspace `w`, added by k_splitk_reduce on the same stream.
template <int MB, int R, int D, int SN, int WAVES, int EPI, int KS>
inline hipError_t launch_line_impl(const GemmParams& p, hipStream_t s, const Workspace* w) {
  using SL = StreamLine<MB, R, D, 0, EPI, SN>;
  static_assert(KS <= 1 || EPI == 0, "k slices: plain epilogue");
  StreamArgs a;
  a.A = p.A;
  a.B = p.B;
  a.scale = nullptr;
  a.zero = nullptr;
  a.C = p.C;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.lda = p.lda;
  a.ldb = p.ldb;
  a.ldc = p.ldc;
  a.group = 0;
  a.up = EPI ? p.N : 0;
  int G = 0;
  size_t lds = 0;
  const int wgs = p.N / (16 * R * SL::SNO);  // output slabs / per workgroup
  constexpr int TPB = MB >= 4 ? 512 : 1024;  // many activation blocks: 256 VGPRs per lane
  if constexpr (KS > 1) {
    a.ks = line_kslices(wgs, p.K, KS);
    a.kspan = p.K / a.ks;
  }
  if (!line_split<SL>(wgs * a.ks, SN, a.ks > 1 ? a.kspan : p.K, WAVES, &a.S, &a.chunk, &G, &lds,
                      TPB))
    return hipErrorInvalidConfiguration;
  const size_t bytes = a.ks > 1 ? (size_t)a.ks * p.M * p.N * sizeof(float) : 0;
  if (w && w->need) {
    *w->need = bytes;
    return hipSuccess;
  }
  if (a.ks > 1) {
    hipError_t werr = hipSuccess;
    a.part = workspace_for(*w, bytes, s, &werr);
    if (!a.part) return werr;
  }
  hipLaunchKernelGGL((k_stream_line<MB, R, D, 0, EPI, SN, TPB>), dim3(wgs * a.ks),
                     dim3(64 * SN * a.S), lds, s, a, G);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.ks == 1) return e;
  return launch_reduce(a.part, a.ks, p.M, p.N, p.C, p.ldc, s);
}

template <int MB, int R, int D, int SN, int WAVES, int EPI = 0>
inline hipError_t launch_line(const GemmParams& p, hipStream_t s) {
  return launch_line_impl<MB, R, D, SN, WAVES, EPI, 0>(p, s, nullptr);
}

// The line kernel with up to KS k slices across workgroups (a workspace row).
template <int MB, int R, int D, int SN, int WAVES, int KS>
inline hipError_t launch_line_ks(const GemmParams& p, hipStream_t s, const Workspace& w) {
  return launch_line_impl<MB, R, D, SN, WAVES, 0, KS>(p, s, &w);
}

template <int BM, int BN, int BK, int WM, int WN, int MS, int SWZ, int GROUP, int XCD>
inline hipError_t launch_mfma(const GemmParams& p, hipStream_t s) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const dim3 grid(nm * nn), blk(WM * WN * 64);
  hipLaunchKernelGGL((k_gemm<BM, BN, BK, WM, WN, MS, SWZ, GROUP, XCD, 0>), grid, blk, 0, s,
                     p.A, static_cast<const void*>(p.B), static_cast<const _Float16*>(nullptr),
                     static_cast<const uint8_t*>(nullptr), p.C, p.M, p.N, p.K, p.lda, p.ldb,
                     p.ldc, 0);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int SWZ, int GROUP, int XCD, int MS>
inline hipError_t launch_dma(const GemmParams& p, hipStream_t s) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const dim3 grid(nm * nn), blk(WM * WN * 64);
  hipLaunchKernelGGL((k_gemm_dma<BM, BN, BK, WM, WN, STAGES, SWZ, GROUP, XCD, 0, 1, MS>), grid, blk,
                     0, s,
                     p.A, p.B, p.C, p.M, p.N, p.K, p.lda, p.ldb, p.ldc);
  return hipGetLastError();
}

// The interleaved prefill kernel (k_gemm_ilv) lives in its own translation unit,
// launch_prefill.hip, compiled with the register-pressure-minimising scheduler; its launchers
// are instantiated there for the rows of the ladder (prefill.inc, generated from select.py).
// SW > 0: split-K towards SW workgroups, at least MINKT k-tiles per split (split_count).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int SW, int MINKT>
hipError_t launch_ilv(const GemmParams& p, hipStream_t s, const Workspace& w);
// The same kernel with the fused gate/up epilogue (p.N the output width, B 2N rows).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv_gu(const GemmParams& p, hipStream_t s, const Workspace& w);
// That row with the output columns in two parts (whole rounds, then TBM x TBN/2-column tiles).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES>
hipError_t launch_ilv_gu_tail(const GemmParams& p, hipStream_t s, const Workspace& w);

// One dispatch row: launchers without a workspace ignore it (and, asked for their need, report 0).
inline hipError_t call_row(hipError_t (*f)(const GemmParams&, hipStream_t), const GemmParams& p,
                           hipStream_t s, const Workspace& w) {
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  return f(p, s);
}
inline hipError_t call_row(hipError_t (*f)(const GemmParams&, hipStream_t, const Workspace&),
                           const GemmParams& p, hipStream_t s, const Workspace& w) {
  return f(p, s, w);
}

// Applicability predicate.  false = the shape is not covered and the caller must take its own
// path.  Dense row-major operands with 16-byte aligned rows; the band's divisibility is
// checked again by the ladder in dispatch.inc.
inline bool applicable(const GemmParams& p) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0) return false;
  if (p.lda < p.K || p.ldb < p.K || p.ldc < p.N) return false;
  if ((p.K % 8) != 0 || (p.N % 8) != 0) return false;
  if ((p.lda % 8) != 0 || (p.ldb % 8) != 0 || (p.ldc % 4) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.A) % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.B) % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.C) % 8) != 0) return false;
  return true;
}

// Shape dispatcher; body is the generated ladder (dispatch.inc), defined in launch.hip, the
// one translation unit of the delivery.  launch(): split-K rows use the delivery's pool.
hipError_t launch(const GemmParams& p, hipStream_t s);
// The same ladder with the caller's workspace: never allocates; a split-K row whose workspace
// does not fit returns hipErrorOutOfMemory (launching nothing).
hipError_t launch_with(const GemmParams& p, hipStream_t s, const Workspace& w);
// Bytes of workspace the row launch() would run needs for this shape (0: none, or not covered).
size_t workspace_bytes(const GemmParams& p);

// Host-only: tag of the ladder row launch() would run, nullptr when not covered.
const char* route(const GemmParams& p);

// Fused gate/up: C[M][N] = silu(A . B[0..N)^T) * (A . B[N..2N)^T), B with 2N rows of stride ldb
// (the gate rows, then the up rows).  Its own ladder (dispatch_gate_up.inc); not covered ->
// hipErrorInvalidConfiguration, the caller runs the plain GEMM and its own elementwise step.
hipError_t launch_gate_up(const GemmParams& p, hipStream_t s);
const char* route_gate_up(const GemmParams& p);

}  // namespace gen
}  // namespace tempo
