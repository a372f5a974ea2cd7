// launch.h -- kernel/framework boundary of the shipped gemm_w8a16 for gfx950.
//
// POD + pointers only (same discipline as the reference's kernels/shipped/gemm_fp16/sm_70/
// launch.cuh:5-8).  C = fp16_rn(A . deq(Wq)^T) with fp32 accumulation; the weights are
// dequantised in registers, bit-exactly:
//   fmt 1: Wq int8 [N][ldw], scale fp16 [N]                  W = fp16_rn(q * s[n])
//   fmt 2: Wq uint8 [N][ldw], scale fp16 [N][K/group], zero uint8 [N][K/group]
//          W = fp16_rn((q - z) * s)
// Asynchronous on the given stream, never synchronises, caller owns every buffer.  Not covered
// -> hipErrorInvalidConfiguration (take your own path).  Split-K rows (narrow N, long K) add fp32
// partial sums in a workspace: launch() takes it from the delivery's per-(device, stream) pool
// (allocated on first use, grown on demand), launch_with() from the caller and never allocates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "kernel.hip"

namespace tempo {
namespace gen8 {

struct W8A16Params {
  const _Float16* A;      // [M][lda]
  const void* Wq;         // int8 / uint8 [N][ldw]
  const _Float16* scale;  // [N] or [N][K/group]
  const uint8_t* zero;    // nullptr or [N][K/group]
  _Float16* C;            // [M][ldc]
  int M, N, K;
  int lda, ldw, ldc;
  int group;
  int fmt;  // 1 int8 symmetric per-channel, 2 uint8 asymmetric group-wise
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

inline StreamArgs stream_args(const W8A16Params& p) {
  StreamArgs a;
  a.A = p.A;
  a.B = p.Wq;
  a.scale = p.scale;
  a.zero = p.zero;
  a.C = p.C;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.lda = p.lda;
  a.ldb = p.ldw;
  a.ldc = p.ldc;
  a.S = 1;
  a.chunk = p.K;
  a.group = p.fmt == 2 ? p.group : 0;
  a.up = 0;
  return a;
}

// Activations staged in LDS (ALDS rows) only while M*(2K+16) bytes stay within this budget.
constexpr size_t kStreamActLds = 96 * 1024;

// EPI = 1: fused gate/up epilogue -- p.N is the output width; Wq, scale and zero hold 2N rows
// (gate, then up) and C = silu(A.deq(W)[0..N)^T) * (A.deq(W)[N..2N)^T).
template <int MB, int R, int U, int ALDS, int EPI = 0>
inline hipError_t launch_stream(const W8A16Params& p, hipStream_t s) {
  constexpr int RR = EPI ? 2 * R : R;
  StreamArgs a = stream_args(p);
  a.up = EPI ? p.N : 0;
  stream_split(p.N, p.K, R, U, &a.S, &a.chunk);
  const dim3 grid(p.N / (16 * R)), blk(64 * a.S);
  const size_t red = a.S > 1 ? (size_t)a.S * RR * MB * 64 * 16 : 0;
  const size_t act = (size_t)p.M * (2 * (size_t)p.K + 16);
  const bool alds = ALDS && act <= kStreamActLds;
  if (p.fmt == 1) {
    if (alds)
      hipLaunchKernelGGL((k_stream<MB, R, U, 1, 1, EPI>), grid, blk, act + red, s, a);
    else
      hipLaunchKernelGGL((k_stream<MB, R, U, 1, 0, EPI>), grid, blk, red, s, a);
  } else {
    if (alds)
      hipLaunchKernelGGL((k_stream<MB, R, U, 2, 1, EPI>), grid, blk, act + red, s, a);
    else
      hipLaunchKernelGGL((k_stream<MB, R, U, 2, 0, EPI>), grid, blk, red, s, a);
  }
  return hipGetLastError();
}

// k-chunks of the shared-activation kernel (same rule as the gemm_fp16 delivery's): about 2048
// waves over the part, at most TPB/64 waves per workgroup (TPB = the kernel's launch bound), the stage count divisible by the chunk
// count, activation rings of every chunk plus the reduction within the 160 KiB of LDS.
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
inline hipError_t launch_shared(const W8A16Params& p, hipStream_t s) {
  StreamArgs a = stream_args(p);
  a.up = EPI ? p.N : 0;
  size_t lds = 0;
  // EPI: the slab waves pair up (gate, up), so the work is that of the plain kernel over 2N rows
  const int rows = EPI ? 2 * p.N : p.N;
  shared_split(rows, p.K, MB, R, U, SN, TPB, &a.S, &a.chunk, &lds);
  const dim3 grid(rows / (16 * R * SN)), blk(64 * SN * a.S);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_stream_sh<MB, R, U, 1, SN, TPB, EPI>), grid, blk, lds, s, a);
  else
    hipLaunchKernelGGL((k_stream_sh<MB, R, U, 2, SN, TPB, EPI>), grid, blk, lds, s, a);
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

// Tail grid of the line kernel (TL = 1): q whole rounds of SN-slab-wave workgroups, kLineCus per
// round, then one single-wave workgroup per remaining output slab.  It applies when q >= 1, at
// most one slab per CU remains, and a CU holds its q workgroups and one tail at once (LDS: the
// launch's size is the larger of the two bodies'; waves: 16).  EPI = 1 (fused gate/up): the
// workgroups' slab waves pair up (SN/2 output slabs each) and a tail wave carries its output
// slab's gate and up row groups.  The ladder's fit predicate calls line_tail_fits, so a row
// that fits always launches.
constexpr int kLineCus = 256;  // CUs of the part (MI355X, MI350X)
template <int MB, int R, int D, int SN, int EPI = 0>
inline bool line_tail_grid(const W8A16Params& p, int* nbig, int* grid, size_t* lds) {
  if (p.N % (16 * R) || p.K % 128 || p.K > 65536) return false;
  constexpr int SNO = EPI ? SN / 2 : SN;
  const int slabs = p.N / (16 * R);  // output slabs
  const int q = slabs / (kLineCus * SNO);
  const int tail = slabs - q * kLineCus * SNO;
  if (q < 1 || tail > kLineCus) return false;
  const int G = p.K / 128;
  constexpr int TSN = EPI ? 2 : 1;  // waves of a tail workgroup (gate/up: a gate, up pair)
  const size_t L =
      p.fmt == 1 ? std::max(StreamLine<MB, R, D, 1, EPI, SN>::lds(1, G),
                            StreamLine<MB, R, D, 1, EPI, TSN>::lds(1, G))
                 : std::max(StreamLine<MB, R, D, 2, EPI, SN>::lds(1, G),
                            StreamLine<MB, R, D, 2, EPI, TSN>::lds(1, G));
  if ((size_t)(q + 1) * L > 160 * 1024 || (q + 1) * SN > 16) return false;
  *nbig = q * kLineCus;
  *grid = q * kLineCus + tail;
  *lds = L;
  return true;
}
template <int MB, int R, int D, int SN, int EPI = 0>
inline bool line_tail_fits(const W8A16Params& p) {
  int nbig = 0, grid = 0;
  size_t lds = 0;
  return line_tail_grid<MB, R, D, SN, EPI>(p, &nbig, &grid, &lds);
}

// k slices of the line kernel across workgroups (KS = the most a row allows): the count that
// spreads wgs x ks workgroups most evenly over the part's CUs, each slice a whole number of
// 128-k steps and at least kLineMinSteps of them.  A split pays a partial-sum pass and a second
// launch, so it is taken only when it lifts the evenness (workgroups / whole rounds of
// kLineCus) by at least 0.08 over no split; ties keep fewer slices.
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
// EPI = 1: fused gate/up (p.N the output width; Wq, scale and zero hold 2N rows).
// TL = 1: the tail grid above, one k chunk per slab.
// KS > 1 (plain epilogue): up to KS k slices across workgroups (line_kslices), their fp32
// partial sums in the workspace `w`, added by k_splitk_reduce on the same stream.
template <int BFMT, int MB, int R, int D, int SN, int WAVES, int EPI, int TL, int KS = 0>
inline hipError_t launch_line_fmt(const W8A16Params& p, hipStream_t s, const Workspace* w = nullptr) {
  using SL = StreamLine<MB, R, D, BFMT, EPI, SN>;
  static_assert(KS <= 1 || (EPI == 0 && TL == 0), "k slices: plain epilogue, no tail grid");
  StreamArgs a = stream_args(p);
  a.up = EPI ? p.N : 0;
  int G = 0;
  size_t lds = 0;
  int wgs = p.N / (16 * R * SL::SNO);  // output slabs / per workgroup
  constexpr int TPB = MB >= 4 ? 512 : 1024;  // many activation blocks: 256 VGPRs per lane
  if constexpr (TL) {
    static_assert(SN > 1 && (EPI == 0 || SN % 2 == 0), "tail grid: shared activation ring");
    if (!line_tail_grid<MB, R, D, SN, EPI>(p, &a.nbig, &wgs, &lds))
      return hipErrorInvalidConfiguration;
    G = p.K / 128;
  } else {
    if constexpr (KS > 1) {
      a.ks = line_kslices(wgs, p.K, KS);
      a.kspan = p.K / a.ks;
    }
    if (!line_split<SL>(wgs * a.ks, SN, a.ks > 1 ? a.kspan : p.K, WAVES, &a.S, &a.chunk, &G, &lds,
                        TPB))
      return hipErrorInvalidConfiguration;
  }
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
  hipLaunchKernelGGL((k_stream_line<MB, R, D, BFMT, EPI, SN, TPB, TL>), dim3(wgs * a.ks),
                     dim3(64 * SN * a.S), lds, s, a, G);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.ks == 1) return e;
  return launch_reduce(a.part, a.ks, p.M, p.N, p.C, p.ldc, s);
}

template <int MB, int R, int D, int SN, int WAVES, int EPI = 0, int TL = 0>
inline hipError_t launch_line(const W8A16Params& p, hipStream_t s) {
  if (p.fmt == 1) return launch_line_fmt<1, MB, R, D, SN, WAVES, EPI, TL>(p, s);
  return launch_line_fmt<2, MB, R, D, SN, WAVES, EPI, TL>(p, s);
}

// The phase-ordered decode kernel (k_stream_phase; M <= 16 MB, MB = 0: M = 1): one workgroup
// per CU, its 8 waves the k chunks; rwg = N / 256 rows per workgroup (a multiple of 4: NS - 1
// slabs of 16 and a last one of 4 .. 16), K a multiple of 1024.  The fit predicate and the
// launcher share phase_layout, so a row that fits always launches.
// EPI = 1 (fused gate/up): p.N is the output width; a workgroup's cwg = N / 256 output columns
// (a multiple of 4) take its 2 cwg rows, the gate rows and the matching up rows.
template <int MB, int NS, int D, int BFMT, int EPI = 0>
inline bool phase_layout(const W8A16Params& p, PhaseArgs* a, int* lds) {
  using SP = StreamPhase<MB, NS, D, BFMT, EPI>;
  if (p.M > 16 * SP::MBE || (MB == 0 && p.M != 1)) return false;
  if (p.N % SP::CUS || p.K % 1024) return false;
  const int cwg = p.N / SP::CUS, rwg = EPI ? 2 * cwg : cwg;
  if (cwg % 4 || (rwg + 15) / 16 != NS) return false;
  const int G = p.K / 128;
  if (BFMT == 2 && p.group != 128) return false;
  // the workgroups' metadata blocks are copied in 4-byte pieces (rwg % 4 keeps them aligned)
  if (((reinterpret_cast<uintptr_t>(p.scale) | reinterpret_cast<uintptr_t>(p.zero)) % 4) != 0)
    return false;
  if (SP::lds(G, G) > 160 * 1024) return false;
  a->A = p.A;
  a->B = reinterpret_cast<const uint8_t*>(p.Wq);
  a->scale = p.scale;
  a->zero = p.zero;
  a->C = p.C;
  a->M = p.M;
  a->K = p.K;
  a->lda = p.lda;
  a->ldb = p.ldw;
  a->ldc = p.ldc;
  a->rwg = rwg;
  a->cwg = cwg;
  a->up = EPI ? p.N : 0;
  a->G = G;
  a->steps = G;
  a->ks = 1;
  a->N = p.N;
  a->part = nullptr;
  a->stg_off = SP::ring_bytes();
  a->out_off = a->stg_off + SP::stg_bytes(G);
  a->meta_off = a->out_off + SP::out_bytes();
  a->meta_s_off = a->meta_off + SP::meta_z_bytes(G, G);
  *lds = SP::lds(G, G);
  return true;
}
template <int MB, int NS, int D>
inline bool phase_fits(const W8A16Params& p) {
  PhaseArgs a;
  int lds = 0;
  return p.fmt == 1 ? phase_layout<MB, NS, D, 1>(p, &a, &lds) : phase_layout<MB, NS, D, 2>(p, &a, &lds);
}
template <int MB, int NS, int D, int EPI = 0>
inline hipError_t launch_phase(const W8A16Params& p, hipStream_t s) {
  PhaseArgs a;
  int lds = 0;
  if (p.fmt == 1) {
    if (!phase_layout<MB, NS, D, 1, EPI>(p, &a, &lds)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((k_stream_phase<MB, NS, D, 1, EPI>), dim3(StreamPhase<MB, NS, D, 1>::CUS),
                       dim3(64 * StreamPhase<MB, NS, D, 1>::NWV), lds, s, a);
  } else {
    if (!phase_layout<MB, NS, D, 2, EPI>(p, &a, &lds)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((k_stream_phase<MB, NS, D, 2, EPI>), dim3(StreamPhase<MB, NS, D, 2>::CUS),
                       dim3(64 * StreamPhase<MB, NS, D, 2>::NWV), lds, s, a);
  }
  return hipGetLastError();
}
// KS k slices across the workgroups (KSL instantiation): 256 / KS row groups of N / (256 / KS)
// rows (a multiple of 4, NS slabs), K / KS k each in at least 8 steps of 128 (a step or more per
// wave); the slices' fp32 sums in the workspace, added in slice order by k_splitk_reduce.
template <int MB, int NS, int D, int BFMT, int KS>
inline bool phase_ks_layout(const W8A16Params& p, PhaseArgs* a, int* lds) {
  using SP = StreamPhase<MB, NS, D, BFMT, 0, 1>;
  static_assert(SP::CUS % KS == 0, "row groups");
  constexpr int groups = SP::CUS / KS;
  if (p.M > 16 * SP::MBE || (MB == 0 && p.M != 1)) return false;
  if (p.N % groups || p.K % (128 * KS)) return false;
  const int rwg = p.N / groups, S = p.K / (128 * KS), G = p.K / 128;
  if (rwg % 4 || (rwg + 15) / 16 != NS || S < SP::NWV) return false;
  if (BFMT == 2 && p.group != 128) return false;
  if ((reinterpret_cast<uintptr_t>(p.scale) % 4) != 0) return false;  // fmt 1: row-scale block
  if (SP::lds(G, S) > 160 * 1024) return false;
  a->A = p.A;
  a->B = reinterpret_cast<const uint8_t*>(p.Wq);
  a->scale = p.scale;
  a->zero = p.zero;
  a->C = p.C;
  a->M = p.M;
  a->K = p.K;
  a->lda = p.lda;
  a->ldb = p.ldw;
  a->ldc = p.ldc;
  a->rwg = rwg;
  a->cwg = rwg;
  a->up = 0;
  a->G = G;
  a->steps = S;
  a->ks = KS;
  a->N = p.N;
  a->part = nullptr;
  a->stg_off = SP::ring_bytes();
  a->out_off = a->stg_off + SP::stg_bytes(S);
  a->meta_off = a->out_off + SP::out_bytes();
  a->meta_s_off = a->meta_off + SP::meta_z_bytes(G, S);
  *lds = SP::lds(G, S);
  return true;
}
template <int MB, int NS, int D, int KS>
inline bool phase_ks_fits(const W8A16Params& p) {
  PhaseArgs a;
  int lds = 0;
  return p.fmt == 1 ? phase_ks_layout<MB, NS, D, 1, KS>(p, &a, &lds)
                    : phase_ks_layout<MB, NS, D, 2, KS>(p, &a, &lds);
}
template <int MB, int NS, int D, int KS>
inline hipError_t launch_phase_ks(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  PhaseArgs a;
  int lds = 0;
  const bool ok = p.fmt == 1 ? phase_ks_layout<MB, NS, D, 1, KS>(p, &a, &lds)
                             : phase_ks_layout<MB, NS, D, 2, KS>(p, &a, &lds);
  if (!ok) return hipErrorInvalidConfiguration;
  const size_t bytes = (size_t)KS * p.M * p.N * sizeof(float);
  if (w.need) {
    *w.need = bytes;
    return hipSuccess;
  }
  hipError_t werr = hipSuccess;
  a.part = workspace_for(w, bytes, s, &werr);
  if (!a.part) return werr;
  constexpr int CUS = StreamPhase<MB, NS, D, 1, 0, 1>::CUS, NWV = StreamPhase<MB, NS, D, 1, 0, 1>::NWV;
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_stream_phase<MB, NS, D, 1, 0, 1>), dim3(CUS), dim3(64 * NWV), lds, s, a);
  else
    hipLaunchKernelGGL((k_stream_phase<MB, NS, D, 2, 0, 1>), dim3(CUS), dim3(64 * NWV), lds, s, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_reduce(a.part, KS, p.M, p.N, p.C, p.ldc, s);
}

template <int MB, int NS, int D>
inline bool phase_gu_fits(const W8A16Params& p) {
  PhaseArgs a;
  int lds = 0;
  return p.fmt == 1 ? phase_layout<MB, NS, D, 1, 1>(p, &a, &lds)
                    : phase_layout<MB, NS, D, 2, 1>(p, &a, &lds);
}
template <int MB, int NS, int D>
inline hipError_t launch_phase_gu(const W8A16Params& p, hipStream_t s) {
  return launch_phase<MB, NS, D, 1>(p, s);
}

// Row-tiled line kernel (64 < M <= 128): the rows of A in tiles of 16 MB across workgroups, each
// workgroup one row tile x one slab group of 16 R weight rows over the whole K, its S waves
// splitting K (partial sums added through LDS in chunk order) -- no split-K partials in HBM, and
// the activations streamed from L2 per tile instead of per 128-column tile.  Workgroups = row
// tiles x slab groups (the rows' bands choose R so that this makes whole rounds of the part).
// S is the most waves, at most SMAX, whose rings (+ fmt 2 metadata) fit the LDS.
template <int BFMT, int MB, int R, int D, int SMAX>
inline bool line_mt_config(const W8A16Params& p, int* S_out, int* per_out, size_t* lds_out) {
  using SL = StreamLine<MB, R, D, BFMT, 0, 1>;
  if (p.N % (16 * R) || p.K % 128 || p.K > 65536 || p.M <= 0) return false;
  const int steps = p.K / 128;
  for (int S = std::min(SMAX, steps); S >= 1; --S) {
    const int per = (steps + S - 1) / S;  // steps per wave
    const int s2 = (steps + per - 1) / per;
    const size_t lds = SL::lds(s2, per);
    if (lds <= 160 * 1024) {
      *S_out = s2;
      *per_out = per;
      *lds_out = lds;
      return true;
    }
  }
  return false;
}
template <int MB, int R, int D, int SMAX>
inline bool line_mt_fits(const W8A16Params& p) {
  int S = 0, per = 0;
  size_t lds = 0;
  return p.fmt == 1 ? line_mt_config<1, MB, R, D, SMAX>(p, &S, &per, &lds)
                    : line_mt_config<2, MB, R, D, SMAX>(p, &S, &per, &lds);
}
template <int BFMT, int MB, int R, int D, int SMAX>
inline hipError_t launch_line_mt_fmt(const W8A16Params& p, hipStream_t s) {
  int S = 0, per = 0;
  size_t lds = 0;
  if (!line_mt_config<BFMT, MB, R, D, SMAX>(p, &S, &per, &lds)) return hipErrorInvalidConfiguration;
  StreamArgs a = stream_args(p);
  a.S = S;
  a.chunk = per * 128;
  a.mrows = 16 * MB;
  a.mtiles = (p.M + a.mrows - 1) / a.mrows;
  const int groups = p.N / (16 * R);
  hipLaunchKernelGGL((k_stream_line<MB, R, D, BFMT, 0, 1, 64 * SMAX, 0>),
                     dim3(a.mtiles * groups), dim3(64 * S), lds, s, a, per);
  return hipGetLastError();
}
template <int MB, int R, int D, int SMAX>
inline hipError_t launch_line_mt(const W8A16Params& p, hipStream_t s) {
  if (p.fmt == 1) return launch_line_mt_fmt<1, MB, R, D, SMAX>(p, s);
  return launch_line_mt_fmt<2, MB, R, D, SMAX>(p, s);
}

// The line kernel with up to KS k slices across workgroups (a workspace row).
template <int MB, int R, int D, int SN, int WAVES, int KS>
inline hipError_t launch_line_ks(const W8A16Params& p, hipStream_t s, const Workspace& w) {
  if (p.fmt == 1) return launch_line_fmt<1, MB, R, D, SN, WAVES, 0, 0, KS>(p, s, &w);
  return launch_line_fmt<2, MB, R, D, SN, WAVES, 0, 0, KS>(p, s, &w);
}

// The interleaved int8 prefill kernel (k_gemm_ilv8) lives in its own translation unit,
// launch_prefill.hip, compiled with the register-pressure-minimising scheduler; its launchers
// are instantiated there for the rows of the ladder (prefill.inc, generated from select.py).
// SW > 0: split-K towards SW workgroups, at least MINKT k-tiles per split (split_count).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int SW, int MINKT>
hipError_t launch_ilv8(const W8A16Params& p, hipStream_t s, const Workspace& w);
// The same kernel, N in two parts: whole rounds of BM x BN tiles, the rest on TBM x TBN tiles.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES, int TSW, int TMINKT>
hipError_t launch_ilv8_tail(const W8A16Params& p, hipStream_t s, const Workspace& w);
// Columns the whole rounds of such a row take (0: it runs plain).
template <int BM, int BN>
inline int ilv8_tail_cols(const W8A16Params& p) {
  constexpr int CUS = 256;
  const int nm = (p.M + BM - 1) / BM, nn = p.N / BN;
  const int tiles = nm * nn, whole = tiles / CUS * CUS;
  if (whole == 0 || whole % nm || whole / nm == nn || 4 * (tiles - whole) > CUS) return 0;
  return whole / nm * BN;
}
// A FILL row: its BM x BN grid is one round of the part and holds more tiles than 256-row tiles
// would (select.py fill_fits).
template <int BM, int BN>
inline bool ilv8_fill_fits(const W8A16Params& p) {
  constexpr int CUS = 256;
  const int nm = (p.M + BM - 1) / BM;
  return nm * (p.N / BN) <= CUS && nm > (p.M + 255) / 256;
}
// The same kernel with the fused gate/up epilogue (p.N the output width, 2N weight rows), and
// that row with the output columns in two parts.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv8_gu(const W8A16Params& p, hipStream_t s, const Workspace& w);
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int TBM, int TBN, int TBK, int TWM, int TWN, int TSTAGES, int TSW, int TMINKT>
hipError_t launch_ilv8_gu_tail(const W8A16Params& p, hipStream_t s, const Workspace& w);

// One dispatch row: launchers without a workspace ignore it (and, asked for their need, report 0).
inline hipError_t call_row(hipError_t (*f)(const W8A16Params&, hipStream_t), const W8A16Params& p,
                           hipStream_t s, const Workspace& w) {
  if (w.need) {
    *w.need = 0;
    return hipSuccess;
  }
  return f(p, s);
}
inline hipError_t call_row(hipError_t (*f)(const W8A16Params&, hipStream_t, const Workspace&),
                           const W8A16Params& p, hipStream_t s, const Workspace& w) {
  return f(p, s, w);
}

template <int BM, int BN, int BK, int WM, int WN, int MS, int SWZ, int GROUP, int XCD>
inline hipError_t launch_mfma(const W8A16Params& p, hipStream_t s) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const dim3 grid(nm * nn), blk(WM * WN * 64);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_gemm<BM, BN, BK, WM, WN, MS, SWZ, GROUP, XCD, 1>), grid, blk, 0, s,
                       p.A, p.Wq, p.scale, p.zero, p.C, p.M, p.N, p.K, p.lda, p.ldw, p.ldc, 0);
  else
    hipLaunchKernelGGL((k_gemm<BM, BN, BK, WM, WN, MS, SWZ, GROUP, XCD, 2>), grid, blk, 0, s,
                       p.A, p.Wq, p.scale, p.zero, p.C, p.M, p.N, p.K, p.lda, p.ldw, p.ldc,
                       p.group);
  return hipGetLastError();
}

inline bool applicable(const W8A16Params& p) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0) return false;
  if (p.fmt != 1 && p.fmt != 2) return false;
  if (!p.A || !p.Wq || !p.scale || !p.C) return false;
  if (p.fmt == 2 && (!p.zero || p.group != 128 || (p.K % p.group) != 0)) return false;
  if (p.lda < p.K || p.ldw < p.K || p.ldc < p.N) return false;
  if ((p.K % 8) != 0 || (p.N % 8) != 0) return false;
  if ((p.lda % 8) != 0 || (p.ldw % 16) != 0 || (p.ldc % 4) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.A) % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.Wq) % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.C) % 8) != 0) return false;
  return true;
}

hipError_t launch(const W8A16Params& p, hipStream_t s);
const char* route(const W8A16Params& p);
// The same ladder with the caller's workspace: never allocates; a split-K row whose workspace
// does not fit returns hipErrorOutOfMemory (launching nothing).
hipError_t launch_with(const W8A16Params& p, hipStream_t s, const Workspace& w);
// Bytes of workspace the row launch() would run needs for this shape (0: none, or not covered).
size_t workspace_bytes(const W8A16Params& p);

// Fused gate/up: C[M][N] = silu(A . deq(W)[0..N)^T) * (A . deq(W)[N..2N)^T), Wq / scale / zero
// with 2N rows (gate, then up).  Its own ladder (dispatch_gate_up.inc); not covered ->
// hipErrorInvalidConfiguration.
hipError_t launch_gate_up(const W8A16Params& p, hipStream_t s);
const char* route_gate_up(const W8A16Params& p);

// Dequantise a [rows][cols] tile of the weights with the GEMM feeds' own device functions.
inline hipError_t dequant_tile(const W8A16Params& p, int n0, int k0, int rows, int cols,
                               _Float16* out, hipStream_t s) {
  if (!applicable(p) || rows <= 0 || cols <= 0 || (cols % 8) != 0 || (k0 % 8) != 0 || n0 < 0 ||
      k0 < 0 || n0 + rows > p.N || k0 + cols > p.K)
    return hipErrorInvalidValue;
  const StreamArgs a = stream_args(p);
  const int work = rows * (cols / 8);
  const dim3 grid((work + 255) / 256), blk(256);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_dequant_tile<1>), grid, blk, 0, s, a, n0, k0, rows, cols, out);
  else
    hipLaunchKernelGGL((k_dequant_tile<2>), grid, blk, 0, s, a, n0, k0, rows, cols, out);
  return hipGetLastError();
}

}  // namespace gen8
}  // namespace tempo
