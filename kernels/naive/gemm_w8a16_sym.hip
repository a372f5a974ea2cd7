// Tempolator input #3 for gfx950: the symmetric W8A16 variant -- int8 weights [N][K] with one fp16
// scale per output row, w = fp16_rn(q * s).  The kernel is naive_gemm_w8a16 (gemm_w8a16.hip) with
// fmt = 1; this file only declares the operation, so the recogniser sees int8 weights.
// ============================================================================================
// TEMPO-OP: gemm
//   dtype: a=fp16 b=int8 c=fp16 acc=fp32
//   layout: a=k b=k c=n
//   shape: M=* N=* K=*
//   scale: per_channel_fp16
//   tol_rel_l2: 3e-3
//   coverage: atomic_stamp
//   entry: naive_gemm_w8a16_sym
//   signature: (const _Float16* A, const int8_t* Wq, const _Float16* S, _Float16* C, int M, int N, int K, hipStream_t s)
// TEMPO-OP-END
// ============================================================================================
#pragma once
#include "gemm_w8a16.hip"

inline hipError_t naive_gemm_w8a16_sym(const _Float16* A, const int8_t* Wq, const _Float16* S,
                                       _Float16* C, int M, int N, int K, hipStream_t s) {
  return naive_gemm_w8a16_launch(A, Wq, S, nullptr, C, M, N, K, 0, 1, s);
}
