// gptq.hip -- one-time repack of a GPTQ int8 checkpoint into the layout of the W8A16 kernels.
//
// GPTQ (bits = 8, group G along k, asymmetric) stores, for a linear layer with K inputs and N
// outputs (reference bench/gemm_baseline.py:214-232, the formula of :229):
//   qweight [K/4][N] int32   byte (k % 4) of qweight[k/4][n] is q[k][n]
//   qzeros  [K/G][N/4] int32 byte (n % 4) of qzeros[g][n/4] is z[g][n]
//   scales  [K/G][N] fp16
//   W[k][n] = fp16_rn((q[k][n] - z[k/G][n]) * s[k/G][n])
// The W8A16 kernels take the transposed, unpacked form (format 2): Wq uint8 [N][K], scale fp16
// [N][K/G], zero uint8 [N][K/G] -- the same formula with [n][k] indexing.  The repack is a pure
// byte permutation: no arithmetic touches a weight, so the result is bit-exact by construction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tempo_gfx950.h"

namespace {

constexpr int TK = 128;  // k per tile (32 int32 rows of qweight): one 128-byte line per Wq row
constexpr int TN = 64;   // n per tile
constexpr int RW = TK / 4 + 1;  // words per LDS row (one pad word)

// one 64 x 128 tile: qweight rows [k0/4, k0/4 + 32) x columns [n0, n0 + 64) -> Wq rows n, bytes k
__global__ __launch_bounds__(256) void k_gptq_repack_w(const uint32_t* __restrict__ qw,
                                                       uint8_t* __restrict__ wq, int K, int N) {
  // row n of the tile holds k bytes 0..127 of output row n0 + n; with 33 words per row the byte
  // scatter of one wave hits bank 4c + 33j + r (distinct over its 64 lanes)
  __shared__ uint32_t t[TN * RW];
  uint8_t* tb = reinterpret_cast<uint8_t*>(t);
  const int n0 = blockIdx.x * TN, k0 = blockIdx.y * TK;
  const int tid = threadIdx.x;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = h * 16 + tid / 16, c = tid % 16;  // int32 row r (k = k0 + 4r .. +3), cols 4c..
    const uint4 v = *reinterpret_cast<const uint4*>(qw + (long)(k0 / 4 + r) * N + n0 + 4 * c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        tb[(4 * c + j) * (4 * RW) + 4 * r + b] = (uint8_t)(w[j] >> (8 * b));
  }
  __syncthreads();
  const int n = tid / 4, q = tid % 4;  // row n, bytes 32q .. 32q+31
  const uint32_t* row = t + n * RW + 8 * q;
  uint4* dst = reinterpret_cast<uint4*>(wq + (long)(n0 + n) * K + k0 + 32 * q);
  dst[0] = uint4{row[0], row[1], row[2], row[3]};
  dst[1] = uint4{row[4], row[5], row[6], row[7]};
}

// per (n, g): zero byte and scale, transposed to [N][K/G]
__global__ void k_gptq_repack_meta(const uint32_t* __restrict__ qz, const uint16_t* __restrict__ sc,
                                   uint8_t* __restrict__ z_out, uint16_t* __restrict__ s_out,
                                   int N, int NG) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)N * NG) return;
  const int g = (int)(i / N), n = (int)(i % N);  // reads run along n (coalesced)
  z_out[(long)n * NG + g] = (uint8_t)(qz[(long)g * (N / 4) + n / 4] >> (8 * (n % 4)));
  s_out[(long)n * NG + g] = sc[(long)g * N + n];
}

}  // namespace

extern "C" {

int tempo_gptq_repack_u8(const void* qweight, const void* qzeros, const void* scales, int K,
                         int N, int group, void* wq, void* scale_out, void* zero_out,
                         tempo_stream_t stream) {
  if (!qweight || !qzeros || !scales || !wq || !scale_out || !zero_out)
    return (int)hipErrorInvalidValue;
  if (K <= 0 || N <= 0 || K % TK != 0 || N % TN != 0 || group != 128 || K % group != 0)
    return TEMPO_FALLBACK;
  if ((reinterpret_cast<uintptr_t>(qweight) % 16) != 0 || (reinterpret_cast<uintptr_t>(wq) % 16) != 0)
    return TEMPO_FALLBACK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_gptq_repack_w, dim3(N / TN, K / TK), dim3(256), 0, s,
                     static_cast<const uint32_t*>(qweight), static_cast<uint8_t*>(wq), K, N);
  const int NG = K / group;
  const long total = (long)N * NG;
  hipLaunchKernelGGL(k_gptq_repack_meta, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     static_cast<const uint32_t*>(qzeros), static_cast<const uint16_t*>(scales),
                     static_cast<uint8_t*>(zero_out), static_cast<uint16_t*>(scale_out), N, NG);
  return (int)hipGetLastError();
}

}  // extern "C"
