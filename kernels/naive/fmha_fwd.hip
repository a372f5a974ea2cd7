// Tempolator input #4 for gfx950: attention forward (FMHA) written the obvious way.
//
// The LOWER MARK the shipped k_fmha_fwd is compared against ("vs input") and the source of the
// operation's declaration.  Semantics of the reference's profiled forward: bottom-right causal
// mask, key j visible to query i iff j <= i + (Sk - Sq) (profiled/fwd_ws/fa2_sm70/csrc/
// attn_fwd_cutlass.cu:137, volta_fwd_ws.cuh:863); query head h reads key/value head
// h / (H / Hkv) (attn_fwd_cutlass.cu:193, volta_fwd_ws.cuh:432); LSE in natural-log units,
// max + log(sum) (volta_fwd_ws.cuh:1063).  One thread per (batch, head, query row), two passes
// over the visible keys: the row max of the fp32 scores scale * (q . k_j), then
// sum_j exp(s_j - max) and sum_j exp(s_j - max) * v_j in fp32, each dot product and sum in key
// and d order; O = fp16_rn(acc / sum).  Dense BSHD storage: Q and O [B][Sq][H][D], K and V
// [B][Sk][Hkv][D].
// ============================================================================================
// TEMPO-OP: attention
//   dtype: a=fp16 b=fp16 c=fp16 acc=fp32
//   layout: a=d b=d c=d
//   shape: B=* H=* HKV=* SQ=* SK=* D=* CAUSAL=*
//   tol_rel_l2: 3e-3
//   coverage: atomic_stamp
//   entry: naive_fmha_fwd
//   signature: (const _Float16* Q, const _Float16* K, const _Float16* V, _Float16* O, float* LSE, int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int causal)
// TEMPO-OP-END
// ============================================================================================
#pragma once
#include <hip/hip_runtime.h>

constexpr int NAIVE_FMHA_DMAX = 256;  // head dimensions up to this (the accumulator row)

__global__ void naive_fmha_fwd(const _Float16* Q, const _Float16* K, const _Float16* V, _Float16* O,
                               float* LSE, int B, int H, int Hkv, int Sq, int Sk, int D,
                               float scale, int causal) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)B * H * Sq) return;
  const int i = (int)(t % Sq), h = (int)(t / Sq % H), b = (int)(t / ((long)Sq * H));
  const int hk = h / (H / Hkv);
  const _Float16* q = Q + (((long)b * Sq + i) * H + h) * D;
  const _Float16* kb = K + ((long)b * Sk * Hkv + hk) * D;  // key j at kb + j * Hkv * D
  const _Float16* vb = V + ((long)b * Sk * Hkv + hk) * D;
  long jend = Sk;
  if (causal) {
    jend = (long)i + (Sk - Sq) + 1;
    jend = jend > Sk ? Sk : (jend < 0 ? 0 : jend);
  }
  auto score = [&](long j) {
    const _Float16* kr = kb + j * Hkv * D;
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot = __builtin_fmaf((float)q[d], (float)kr[d], dot);
    return dot * scale;
  };
  float mx = -__builtin_inff();
  for (long j = 0; j < jend; ++j) mx = fmaxf(mx, score(j));
  float acc[NAIVE_FMHA_DMAX];
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  float l = 0.f;
  for (long j = 0; j < jend; ++j) {
    const float p = expf(score(j) - mx);
    l += p;
    const _Float16* vr = vb + j * Hkv * D;
    for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(p, (float)vr[d], acc[d]);
  }
  _Float16* o = O + (((long)b * Sq + i) * H + h) * D;
  for (int d = 0; d < D; ++d) o[d] = (_Float16)(l > 0.f ? acc[d] / l : 0.f);
  if (LSE) LSE[((long)b * H + h) * Sq + i] = l > 0.f ? mx + logf(l) : -__builtin_inff();
}

inline hipError_t naive_fmha_fwd_launch(const _Float16* Q, const _Float16* K, const _Float16* V,
                                        _Float16* O, float* LSE, int B, int H, int Hkv, int Sq,
                                        int Sk, int D, float scale, int causal, hipStream_t s) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || Sq <= 0 || Sk <= 0 || D <= 0 ||
      D > NAIVE_FMHA_DMAX)
    return hipErrorInvalidValue;
  const long rows = (long)B * H * Sq;
  const int blk = 64;
  hipLaunchKernelGGL(naive_fmha_fwd, dim3((unsigned)((rows + blk - 1) / blk)), dim3(blk), 0, s, Q,
                     K, V, O, LSE, B, H, Hkv, Sq, Sk, D, scale, causal);
  return hipGetLastError();
}
