// Tempolator input #2 for gfx950: W8A16 GEMM (fp16 activations, 8-bit weights) written the obvious
// way, in the checkpoint format the production model ships: uint8 weights with an fp16 scale and a
// uint8 zero-point per (output row, 128 consecutive k) -- GPTQ int8 g128 transposed to [N][K]
// (reference bench/gemm_baseline.py:214-232, dense formula :229).
//
// The LOWER MARK for the generated W8A16 kernels and the source of the operation's declaration.
// One thread per output; each weight is dequantised to fp16 exactly once, w = fp16_rn((q - z) * s)
// ((q - z) * s is exact in fp32, so this is one rounding), and then accumulated exactly as the
// naive fp16 GEMM does (kernels/naive/gemm_fp16.hip): fp32 accumulator, k in order, one FMA per
// step, one round-to-nearest-even to fp16 at the end.
// ============================================================================================
// TEMPO-OP: gemm
//   dtype: a=fp16 b=uint8 c=fp16 acc=fp32
//   layout: a=k b=k c=n
//   shape: M=* N=* K=*
//   scale: group128_fp16_zero_u8
//   tol_rel_l2: 3e-3
//   coverage: atomic_stamp
//   entry: naive_gemm_w8a16
//   signature: (const _Float16* A, const void* Wq, const _Float16* S, const uint8_t* Z, _Float16* C, int M, int N, int K, int G, int fmt)
// TEMPO-OP-END
// ============================================================================================
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef NAIVE_GEMM_TILE
#define NAIVE_GEMM_TILE 16
#endif

// fmt 1: int8 weights, S[N] (one scale per row), Z unused.  fmt 2: uint8 weights, S and Z [N][K/G].
__global__ void naive_gemm_w8a16(const _Float16* A, const void* Wq, const _Float16* S,
                                 const uint8_t* Z, _Float16* C, int M, int N, int K, int G, int fmt) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y * blockDim.y + threadIdx.y;
  if (m >= M || n >= N) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    float q, s;
    if (fmt == 1) {
      q = (float)static_cast<const int8_t*>(Wq)[(long)n * K + k];
      s = (float)S[n];
    } else {
      const long g = (long)n * (K / G) + k / G;
      q = (float)static_cast<const uint8_t*>(Wq)[(long)n * K + k] - (float)Z[g];
      s = (float)S[g];
    }
    const _Float16 w = (_Float16)(q * s);
    acc = __builtin_fmaf((float)A[(long)m * K + k], (float)w, acc);
  }
  C[(long)m * N + n] = (_Float16)acc;
}

inline hipError_t naive_gemm_w8a16_launch(const _Float16* A, const void* Wq, const _Float16* S,
                                          const uint8_t* Z, _Float16* C, int M, int N, int K,
                                          int G, int fmt, hipStream_t s) {
  constexpr int T = NAIVE_GEMM_TILE;
  const dim3 blk(T, T), grd((N + T - 1) / T, (M + T - 1) / T);
  hipLaunchKernelGGL(naive_gemm_w8a16, grd, blk, 0, s, A, Wq, S, Z, C, M, N, K, G, fmt);
  return hipGetLastError();
}
