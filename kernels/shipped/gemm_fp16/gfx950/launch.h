// launch.h -- kernel/framework boundary of the shipped gemm_fp16 for gfx950.
//
// Plain POD and pointers only, no framework type (reference:
// kernels/shipped/gemm_fp16/sm_70/launch.cuh:5-8,20-26).  The call is asynchronous on the
// given stream, never synchronises, and the caller owns every buffer.  A shape the ladder
// does not cover returns hipErrorInvalidConfiguration: "take your own path" (dispatch.inc).
//
// The only state is the split-K workspace of the streaming (decode) kernel: one buffer per
// device, allocated on the first call that needs it and kept for the life of the process.
// Calls that overlap on one device (different streams, same time) must not both take the
// split-K route; calls serialised on one stream are safe.
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

// ---- split-K workspace (streaming kernel only) ---------------------------------------------
constexpr size_t kWsPartialBytes = size_t(32) << 20;  // fp32 partials, S*M*N*4 <= this
constexpr size_t kWsCounterCount = size_t(1) << 16;   // per-slab arrival counters
hipError_t workspace(float** partials, unsigned** counters);  // defined in launch.hip

// Choose the k split for the streaming kernel: enough waves to cover the machine (about 8
// per CU of 256 CUs), chunks of whole pipeline stages, workspace within its fixed size.
inline void stream_split(int M, int N, int K, int R, int U, int* S_out, int* chunk_out) {
  const int slabs = N / (16 * R);
  const int step = 64 * U;
  int S = (2048 + slabs - 1) / slabs;
  const int smax_k = K / 256 > 0 ? K / 256 : 1;  // keep chunks >= 256 k
  if (S > smax_k) S = smax_k;
  if (S < 1) S = 1;
  while (S > 1 && (size_t)S * M * N * 4 > kWsPartialBytes) --S;
  int chunk = (K + S - 1) / S;
  chunk = (chunk + step - 1) / step * step;
  S = (K + chunk - 1) / chunk;
  *S_out = S;
  *chunk_out = chunk;
}

template <int MB, int R, int U>
inline hipError_t launch_stream(const GemmParams& p, hipStream_t s) {
  StreamArgs a;
  a.A = p.A;
  a.B = p.B;
  a.scale = nullptr;
  a.zero = nullptr;
  a.C = p.C;
  a.ws = nullptr;
  a.counters = nullptr;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.lda = p.lda;
  a.ldb = p.ldb;
  a.ldc = p.ldc;
  a.group = 0;
  stream_split(p.M, p.N, p.K, R, U, &a.S, &a.chunk);
  if (a.S > 1) {
    if ((size_t)(p.N / (16 * R)) > kWsCounterCount) return hipErrorInvalidConfiguration;
    const hipError_t e = workspace(&a.ws, &a.counters);
    if (e != hipSuccess) return e;
  }
  const int units = (p.N / (16 * R)) * a.S;
  const dim3 grid((units + 3) / 4), blk(256);
  hipLaunchKernelGGL((k_stream<MB, R, U, 0>), grid, blk, 0, s, a);
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
