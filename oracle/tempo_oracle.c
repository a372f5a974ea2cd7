/*
 * tempo_oracle.c -- CPU restatement of the reference's arithmetic for the gfx950 hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library, the plugin, or the timed GPU path
 * links or calls this file.  It is loaded by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, and there only as the checker (or as the timed CPU baseline).
 *
 * What each function restates (reference paths are relative to the reference root):
 *   oracle_gemm_f16        kernels/naive/gemm_fp16.cu:60-68   one accumulator per output, float,
 *                          k strictly sequential, acc += a*b contracted to an FMA (nvcc default),
 *                          one RNE rounding to fp16 (__float2half) at the end.
 *   oracle_dequant_sym     BASELINE config 3 closed form: W = fp16_rn(float(q) * float(s[n])).
 *                          Extends tempo/plugins/sm70/skeletons/gemm_w8a16/harness.cu:39-46 (exact
 *                          int8 -> fp16 with no scale) by a per-output-channel scale.
 *   oracle_dequant_asym    bench/gemm_baseline.py:229 `((q - z) * s).half()` with G=128, stored
 *                          [N][K] instead of GPTQ's [K][N]: W = fp16_rn(float(q - z) * float(s)).
 *   oracle_gemm_w8a16      dequant as above, then oracle_gemm_f16 on the dequantised weight
 *                          (bench/gemm_baseline.py:393 `x.float() @ W.float()` -- the fp16 W).
 *   oracle_fmha_fwd        profiled/fwd_ws/fa2_sm70/csrc/attn_fwd_cutlass.cu:137 (off = Sk - Sq,
 *                          bottom-right causal), :193 (kv_head_ratio = H / Hkv),
 *                          volta_fwd_ws.cuh:432 (hkv = h / ratio), :863 (mask q + off < k),
 *                          :1063 (LSE = max + log(l) in natural-log units).  fp32 scores,
 *                          fp32 softmax, fp32 P.V accumulation, fp16 RNE output.
 *   oracle_rel_l2_*        tempo/core/op/oracle.py:114-124 (double accumulation, as in
 *                          tempo/plugins/sm70/skeletons/gemm_hmma884/harness.cu:42-49).
 *   oracle_count_poison    harness.cu:50-57 (cells still holding the 0x7f7f poison).
 *   oracle_spot_fp64       kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:70-79 (fp64 reference
 *                          on sampled cells m=(t*37)%M, n=(t*53)%N, |got-ref|/(|ref|+1e-3)).
 *
 * Pinning (each is a test in tests/test_oracle.py):
 *   f2h/h2f          exhaustive over all 2^32 floats against the F16C hardware converter, and
 *                    all 65536 halves against numpy.
 *   gemm             bit-exact against the ship-probe known-answer inputs (every partial sum is
 *                    exact, so the fp16 result is a closed form computed with Python integers),
 *                    bit-exact against an independent numpy float32 sequential-k emulation
 *                    (fp16*fp16 is exact in fp32, so round(acc + a*b) == fmaf(a, b, acc)), and
 *                    against fp64 matmul within tolerance.
 *   dequant          exhaustive over q (and q, z) against numpy float32 -> float16 casts, plus
 *                    the invariants s = 1 => W = q - z and q = z => W = 0.
 *   fmha             fp64 numpy brute force on small shapes, and invariants (causal row 0 equals
 *                    V[0] when Sq == Sk; a constant K gives the running mean of V).
 *   rel_l2           closed forms (identical -> 0; got = 0 -> 1; got = 2 ref -> 1).
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* fp16 <-> fp32, written from the IEEE-754 binary16 definition (round to nearest, ties to even) */
/* ------------------------------------------------------------------------------------------ */
float oracle_h2f(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t f;
  if (e == 0) {
    if (m == 0) {
      f = s;
    } else {
      int sh = 0;
      while (!(m & 0x400u)) {
        m <<= 1;
        ++sh;
      }
      m &= 0x3ffu;
      f = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
    }
  } else if (e == 31) {
    f = s | 0x7f800000u | (m << 13);
  } else {
    f = s | ((e + 112u) << 23) | (m << 13);
  }
  float x;
  memcpy(&x, &f, 4);
  return x;
}

uint16_t oracle_f2h(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t s = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) /* inf / nan: nan keeps its top payload bits and becomes quiet */
    return (uint16_t)(s | (a > 0x7f800000u ? (0x7e00u | ((a >> 13) & 0x3ffu)) : 0x7c00u));
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                               /* normal binary16 range */
    const uint32_t mant = a & 0x7fffffu;
    uint32_t h = (((a >> 23) - 112u) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exponent */
    return (uint16_t)(s | h);
  }
  if (a < 0x33000000u) return (uint16_t)s; /* below 2^-25: rounds to signed zero */
  {                                        /* subnormal binary16 */
    const uint32_t e = a >> 23;
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e; /* 14..24 */
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(s | h);
  }
}

void oracle_h2f_array(const uint16_t* h, float* f, long n) {
  for (long i = 0; i < n; ++i) f[i] = oracle_h2f(h[i]);
}

void oracle_f2h_array(const float* f, uint16_t* h, long n) {
  for (long i = 0; i < n; ++i) h[i] = oracle_f2h(f[i]);
}

/* Exhaustive self-check of oracle_f2h against the F16C converter over every float bit pattern.
 * Returns the number of mismatches (0 expected).  Independent path: hardware vs. bit arithmetic. */
__attribute__((target("f16c"))) long oracle_check_f2h_exhaustive(int threads) {
  long bad = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for reduction(+ : bad) schedule(static)
#endif
  for (long hi = 0; hi < 65536; ++hi) {
    for (uint32_t lo = 0; lo < 65536u; ++lo) {
      const uint32_t u = ((uint32_t)hi << 16) | lo;
      float x;
      memcpy(&x, &u, 4);
      const uint16_t hw = (uint16_t)_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
      if (hw != oracle_f2h(x)) ++bad;
    }
  }
  return bad;
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

/* ------------------------------------------------------------------------------------------ */
/* GEMM  C[m][n] = fp16_rn( sum_k  float(A[m][k]) * float(B[n][k]) ), k sequential, fmaf.       */
/* kernels/naive/gemm_fp16.cu:60-68.  Vectorised across n only: every output keeps its own    */
/* accumulator and sees the k terms in order 0..K-1, so the result is bit-identical to the     */
/* one-thread-per-output naive kernel.                                                        */
/* ------------------------------------------------------------------------------------------ */
#define OMB 4
#define ONB 16

static void gemm_f32_seq(const float* Af, const float* BT, uint16_t* C, int M, int N, int K,
                         long ldc) {
  const int mblocks = (M + OMB - 1) / OMB;
  const int nblocks = (N + ONB - 1) / ONB;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
#endif
  for (int mb = 0; mb < mblocks; ++mb) {
    for (int nb = 0; nb < nblocks; ++nb) {
      const int m0 = mb * OMB, n0 = nb * ONB;
      const int mr = (M - m0) < OMB ? (M - m0) : OMB;
      const int nr = (N - n0) < ONB ? (N - n0) : ONB;
      if (mr == OMB && nr == ONB) {
        float acc[OMB][ONB];
        for (int i = 0; i < OMB; ++i)
          for (int j = 0; j < ONB; ++j) acc[i][j] = 0.f;
        const float* panel = BT + (long)nb * K * ONB; /* panel nb: [K][ONB] contiguous */
        for (int k = 0; k < K; ++k) {
          const float* b = panel + (long)k * ONB;
          for (int i = 0; i < OMB; ++i) {
            const float a = Af[(long)(m0 + i) * K + k];
#pragma omp simd
            for (int j = 0; j < ONB; ++j) acc[i][j] = fmaf(a, b[j], acc[i][j]);
          }
        }
        for (int i = 0; i < OMB; ++i)
          for (int j = 0; j < ONB; ++j) C[(long)(m0 + i) * ldc + n0 + j] = oracle_f2h(acc[i][j]);
      } else {
        for (int i = 0; i < mr; ++i)
          for (int j = 0; j < nr; ++j) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k)
              acc = fmaf(Af[(long)(m0 + i) * K + k], BT[((long)nb * K + k) * ONB + j], acc);
            C[(long)(m0 + i) * ldc + n0 + j] = oracle_f2h(acc);
          }
      }
    }
  }
}

/* A [M][lda] fp16, B [N][ldb] fp16 (both k-contiguous), C [M][ldc] fp16. */
void oracle_gemm_f16(const uint16_t* A, const uint16_t* B, uint16_t* C, int M, int N, int K,
                     long lda, long ldb, long ldc, int threads) {
  set_threads(threads);
  float* Af = (float*)malloc(sizeof(float) * (size_t)M * K);
  float* BT = NULL;
#ifdef _OPENMP
#pragma omp parallel for
#endif
  for (long m = 0; m < M; ++m)
    for (long k = 0; k < K; ++k) Af[m * K + k] = oracle_h2f(A[m * lda + k]);
  /* pack B[n][k] into column panels BT[nb][k][ONB] (zero-padded past N), so the k walk of
   * one panel is contiguous memory */
  const long nblk = (N + ONB - 1) / ONB;
  BT = (float*)malloc(sizeof(float) * (size_t)nblk * K * ONB);
#ifdef _OPENMP
#pragma omp parallel for collapse(2)
#endif
  for (long nb = 0; nb < nblk; ++nb)
    for (long k0 = 0; k0 < K; k0 += 64) {
      const long k1 = k0 + 64 < K ? k0 + 64 : K;
      for (long j = 0; j < ONB; ++j) {
        const long n = nb * ONB + j;
        for (long k = k0; k < k1; ++k)
          BT[(nb * K + k) * ONB + j] = n < N ? oracle_h2f(B[n * ldb + k]) : 0.f;
      }
    }
  gemm_f32_seq(Af, BT, C, M, N, K, ldc);
  free(Af);
  free(BT);
}

/* ------------------------------------------------------------------------------------------ */
/* Dequantisation closed forms.  The product of an integer with |v| <= 255 (8 bits) and an fp16 */
/* scale (11 significant bits) is exact in fp32, so each weight sees exactly one rounding.     */
/* ------------------------------------------------------------------------------------------ */
void oracle_dequant_sym(const int8_t* q, const uint16_t* s, uint16_t* W, int N, int K,
                        long ldq, long ldw) {
#ifdef _OPENMP
#pragma omp parallel for
#endif
  for (long n = 0; n < N; ++n) {
    const float sc = oracle_h2f(s[n]);
    for (long k = 0; k < K; ++k) W[n * ldw + k] = oracle_f2h((float)q[n * ldq + k] * sc);
  }
}

/* s, z: [N][K/G] row-major (group index fastest).  q, z unsigned. */
void oracle_dequant_asym(const uint8_t* q, const uint16_t* s, const uint8_t* z, uint16_t* W,
                         int N, int K, int G, long ldq, long ldw) {
  const long ng = K / G;
#ifdef _OPENMP
#pragma omp parallel for
#endif
  for (long n = 0; n < N; ++n)
    for (long k = 0; k < K; ++k) {
      const long g = k / G;
      const int d = (int)q[n * ldq + k] - (int)z[n * ng + g];
      W[n * ldw + k] = oracle_f2h((float)d * oracle_h2f(s[n * ng + g]));
    }
}

/* fmt 1 = int8 symmetric per-channel (s [N], z unused); fmt 2 = uint8 asymmetric group-G. */
void oracle_gemm_w8a16(const uint16_t* A, const void* q, const uint16_t* s, const uint8_t* z,
                       uint16_t* C, int M, int N, int K, int G, int fmt, int threads) {
  set_threads(threads);
  uint16_t* W = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)N * K);
  if (fmt == 1)
    oracle_dequant_sym((const int8_t*)q, s, W, N, K, K, K);
  else
    oracle_dequant_asym((const uint8_t*)q, s, z, W, N, K, G, K, K);
  oracle_gemm_f16(A, W, C, M, N, K, K, K, N, threads);
  free(W);
}

/* ------------------------------------------------------------------------------------------ */
/* FMHA forward (fp32 reference).  Strides in elements.  Q [b][i][h][d] addressed as            */
/* b*q_sb + i*q_ss + h*q_sh + d; K, V with (k_sb, k_ss, k_sh); O like Q with o_*; LSE [b][h][i]. */
/* rows == NULL computes every query row; otherwise only rows[0..nrows).                       */
/* ------------------------------------------------------------------------------------------ */
void oracle_fmha_fwd(const uint16_t* Q, const uint16_t* Kt, const uint16_t* V, uint16_t* O,
                     float* LSE, int B, int H, int Hkv, int Sq, int Sk, int D, float scale,
                     int causal, long q_sb, long q_ss, long q_sh, long k_sb, long k_ss, long k_sh,
                     long v_sb, long v_ss, long v_sh, long o_sb, long o_ss, long o_sh,
                     const int* rows, int nrows, int threads) {
  set_threads(threads);
  const int ratio = H / Hkv;
  const long off = (long)Sk - Sq;
  const int nr = rows ? nrows : Sq;
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)Sk);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
#ifdef _OPENMP
#pragma omp for collapse(3) schedule(dynamic, 4)
#endif
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int r = 0; r < nr; ++r) {
          const int i = rows ? rows[r] : r;
          const int hk = h / ratio;
          const uint16_t* q = Q + b * q_sb + (long)i * q_ss + (long)h * q_sh;
          for (int d = 0; d < D; ++d) qf[d] = oracle_h2f(q[d]);
          long jend = Sk;
          if (causal) {
            jend = (long)i + off + 1;
            if (jend > Sk) jend = Sk;
            if (jend < 0) jend = 0;
          }
          float mx = -INFINITY;
          for (long j = 0; j < jend; ++j) {
            const uint16_t* kr = Kt + b * k_sb + j * k_ss + (long)hk * k_sh;
            float dot = 0.f;
            for (int d = 0; d < D; ++d) dot = fmaf(qf[d], oracle_h2f(kr[d]), dot);
            sc[j] = dot * scale;
            if (sc[j] > mx) mx = sc[j];
          }
          for (int d = 0; d < D; ++d) acc[d] = 0.f;
          float l = 0.f;
          for (long j = 0; j < jend; ++j) {
            const float p = expf(sc[j] - mx);
            l += p;
            const uint16_t* vr = V + b * v_sb + j * v_ss + (long)hk * v_sh;
            for (int d = 0; d < D; ++d) acc[d] = fmaf(p, oracle_h2f(vr[d]), acc[d]);
          }
          uint16_t* o = O + b * o_sb + (long)i * o_ss + (long)h * o_sh;
          for (int d = 0; d < D; ++d) o[d] = oracle_f2h(l > 0.f ? acc[d] / l : 0.f);
          if (LSE) LSE[((long)b * H + h) * Sq + i] = l > 0.f ? mx + logf(l) : -INFINITY;
        }
    free(sc);
    free(acc);
    free(qf);
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Gate arithmetic.                                                                           */
/* ------------------------------------------------------------------------------------------ */
double oracle_rel_l2_f16(const uint16_t* got, const uint16_t* ref, long n) {
  double num = 0.0, den = 0.0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : num, den)
#endif
  for (long i = 0; i < n; ++i) {
    const double a = oracle_h2f(got[i]), b = oracle_h2f(ref[i]);
    num += (a - b) * (a - b);
    den += b * b;
  }
  if (den <= 0.0) return NAN;
  return sqrt(num / den);
}

double oracle_rel_l2_f16_f32(const uint16_t* got, const float* ref, long n) {
  double num = 0.0, den = 0.0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : num, den)
#endif
  for (long i = 0; i < n; ++i) {
    const double a = oracle_h2f(got[i]), b = ref[i];
    num += (a - b) * (a - b);
    den += b * b;
  }
  if (den <= 0.0) return NAN;
  return sqrt(num / den);
}

long oracle_count_poison(const uint16_t* c, long n) {
  long bad = 0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : bad)
#endif
  for (long i = 0; i < n; ++i) bad += (c[i] == 0x7f7fu);
  return bad;
}

/* fp64 reference on `cells` sampled outputs; W may be NULL (then B is the fp16 weight).
 * Returns the maximum |got - ref| / (|ref| + 1e-3); *nbad counts cells above tol. */
double oracle_spot_fp64(const uint16_t* A, const uint16_t* B, const uint16_t* C, int M, int N,
                        int K, int cells, double tol, int* nbad) {
  double worst = 0.0;
  int bad = 0;
  for (int t = 0; t < cells; ++t) {
    const long m = ((long)t * 37) % M, n = ((long)t * 53) % N;
    double ref = 0.0;
    for (long k = 0; k < K; ++k)
      ref += (double)oracle_h2f(A[m * K + k]) * (double)oracle_h2f(B[n * K + k]);
    const double got = oracle_h2f(C[m * N + n]);
    const double d = fabs(got - ref) / (fabs(ref) + 1e-3);
    if (d > tol) ++bad;
    if (d > worst || d != d) worst = d;
  }
  if (nbad) *nbad = bad;
  return worst;
}
