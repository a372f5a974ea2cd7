// Tempolator input #1 for gfx950: dense fp16 GEMM written the obvious way.
//
// Not a benchmark and not a candidate: the LOWER MARK the generated kernel is compared against
// ("vs input"), and the source of the operation's declaration.  Same definition as the
// reference's kernels/naive/gemm_fp16.cu:60-68: one thread per output, an fp32 accumulator,
// k strictly in order, acc += a*b fused to one FMA (written as fmaf so the fusion does not
// depend on compiler flags), one round-to-nearest-even conversion to fp16 at the end.
// C = A . B^T with both operands k-contiguous, i.e. torch.nn.functional.linear(x[M,K], W[N,K]).
// ============================================================================================
// TEMPO-OP: gemm
//   dtype: a=fp16 b=fp16 c=fp16 acc=fp32
//   layout: a=k b=k c=n
//   shape: M=* N=* K=*
//   tol_rel_l2: 3e-3
//   coverage: atomic_stamp
//   entry: naive_gemm_fp16
//   signature: (const _Float16* A, const _Float16* B, _Float16* C, int M, int N, int K)
// TEMPO-OP-END
// ============================================================================================
#pragma once
#include <hip/hip_runtime.h>

#ifndef NAIVE_GEMM_TILE
#define NAIVE_GEMM_TILE 16
#endif

__global__ void naive_gemm_fp16(const _Float16* A, const _Float16* B, _Float16* C, int M, int N, int K) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y * blockDim.y + threadIdx.y;
  if (m >= M || n >= N) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k)
    acc = __builtin_fmaf((float)A[(long)m * K + k], (float)B[(long)n * K + k], acc);
  C[(long)m * N + n] = (_Float16)acc;
}

inline hipError_t naive_gemm_fp16_launch(const _Float16* A, const _Float16* B, _Float16* C, int M,
                                         int N, int K, hipStream_t s) {
  constexpr int T = NAIVE_GEMM_TILE;
  const dim3 blk(T, T), grd((N + T - 1) / T, (M + T - 1) / T);
  hipLaunchKernelGGL(naive_gemm_fp16, grd, blk, 0, s, A, B, C, M, N, K);
  return hipGetLastError();
}
