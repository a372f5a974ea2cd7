// launch.h -- kernel/framework boundary of the shipped gemm_fp16 for gfx950.
//
// Plain POD and pointers only, no framework type (reference:
// kernels/shipped/gemm_fp16/sm_70/launch.cuh:5-8,20-26).  The call is asynchronous on the
// given stream, never synchronises, and the caller owns every buffer.  A shape the ladder
// does not cover returns hipErrorInvalidConfiguration: "take your own path" (dispatch.inc).
//
// The launcher keeps no state and allocates nothing: concurrent calls on different streams are
// independent.
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

template <int MB, int R, int U, int ALDS>
inline hipError_t launch_stream(const GemmParams& p, hipStream_t s) {
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
  stream_split(p.N, p.K, R, U, &a.S, &a.chunk);
  const dim3 grid(p.N / (16 * R)), blk(64 * a.S);
  const size_t red = a.S > 1 ? (size_t)a.S * R * MB * 64 * 16 : 0;
  const size_t act = (size_t)p.M * (2 * (size_t)p.K + 16);
  if (ALDS && act <= kStreamActLds)
    hipLaunchKernelGGL((k_stream<MB, R, U, 0, 1>), grid, blk, act + red, s, a);
  else
    hipLaunchKernelGGL((k_stream<MB, R, U, 0, 0>), grid, blk, red, s, a);
  return hipGetLastError();
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
// one translation unit of the delivery.
hipError_t launch(const GemmParams& p, hipStream_t s);

// Host-only: tag of the ladder row launch() would run, nullptr when not covered.
const char* route(const GemmParams& p);

}  // namespace gen
}  // namespace tempo
