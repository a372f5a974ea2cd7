// ship_probe.hip -- proof that the W8A16 delivery alone gives a working launcher.
//
// Built from THIS directory's files only (launch.hip, launch_prefill.hip and this probe, with
// -I pointing here and nowhere else), the way a host tree would vendor the delivery; the
// pattern is the reference's ship probe of its fp16 delivery
// (kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:35-98).
//
// Shapes: one per band of the ladder on the production dense shapes (decode, mid-M, prefill),
// both weight formats.  Inputs are chosen so that every dequantised weight is exact in fp16 and
// every product and partial sum is exact in fp32:
//   A[i]          = ((i % 7) - 3) / 8
//   fmt 1: q[i]   = (i % 9) - 4 (int8),           s[n]    = 1/4
//   fmt 2: q[i]   = 100 + (i % 11) (uint8),       z[n][g] = 103 + (n + g) % 5,   s[n][g] = 1/8
// so C equals the fp16 rounding of the exact sum.  Output poisoned with 0x7f7f first; 64 cells
// (m = 37t % M, n = 53t % N) must equal the fp64 reference bit for bit (and pass the reference's
// |got-ref|/(|ref|+1e-3) <= 3e-3 rule), and no poison may be left anywhere.  Exit 0 = all passed.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "launch.h"

#define CK(x)                                                                        \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) {                                                          \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);          \
      return 2;                                                                      \
    }                                                                                \
  } while (0)

static uint16_t half_bits(_Float16 h) {
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}

int main() {
  struct Shape {
    int M, N, K;
  };
  const Shape shapes[] = {{1, 7168, 5120},     {16, 34816, 5120}, {32, 5120, 17408},
                          {128, 5120, 6144},   {2048, 7168, 5120}, {2048, 1024, 5120}};
  const int G = 128;
  int pass = 0, fail = 0;
  for (int fmt = 1; fmt <= 2; ++fmt) {
    for (const Shape& s : shapes) {
      const size_t na = (size_t)s.M * s.K, nw = (size_t)s.N * s.K, nc = (size_t)s.M * s.N;
      const size_t nmeta = fmt == 1 ? (size_t)s.N : (size_t)s.N * (s.K / G);
      std::vector<_Float16> ha(na), hs(nmeta), hc(nc);
      std::vector<uint8_t> hw(nw), hz(fmt == 2 ? nmeta : 0);
      for (size_t i = 0; i < na; ++i) ha[i] = (_Float16)(((int)(i % 7) - 3) * 0.125f);
      for (size_t i = 0; i < nw; ++i)
        hw[i] = fmt == 1 ? (uint8_t)(int8_t)((int)(i % 9) - 4) : (uint8_t)(100 + i % 11);
      for (size_t i = 0; i < nmeta; ++i) {
        hs[i] = (_Float16)(fmt == 1 ? 0.25f : 0.125f);
        if (fmt == 2) hz[i] = (uint8_t)(103 + (i / (s.K / G) + i % (s.K / G)) % 5);
      }
      auto weight = [&](int n, int k) -> double {
        const size_t i = (size_t)n * s.K + k;
        if (fmt == 1) return (double)(int8_t)hw[i] * 0.25;
        return ((double)hw[i] - (double)hz[(size_t)n * (s.K / G) + k / G]) * 0.125;
      };
      _Float16 *A = nullptr, *S = nullptr, *C = nullptr;
      uint8_t *W = nullptr, *Z = nullptr;
      CK(hipMalloc(&A, na * 2));
      CK(hipMalloc(&W, nw));
      CK(hipMalloc(&S, nmeta * 2));
      CK(hipMalloc(&C, nc * 2));
      if (fmt == 2) CK(hipMalloc(&Z, nmeta));
      CK(hipMemcpy(A, ha.data(), na * 2, hipMemcpyHostToDevice));
      CK(hipMemcpy(W, hw.data(), nw, hipMemcpyHostToDevice));
      CK(hipMemcpy(S, hs.data(), nmeta * 2, hipMemcpyHostToDevice));
      if (fmt == 2) CK(hipMemcpy(Z, hz.data(), nmeta, hipMemcpyHostToDevice));
      CK(hipMemset(C, 0x7f, nc * 2));

      tempo::gen8::W8A16Params p{A, W, S, Z, C, s.M, s.N, s.K, s.K, s.K, s.N,
                                fmt == 2 ? G : 0, fmt};
      const bool app = tempo::gen8::applicable(p);
      const char* row = tempo::gen8::route(p);
      const hipError_t le = tempo::gen8::launch(p, nullptr);
      const hipError_t se = hipDeviceSynchronize();
      double worst = 0.0;
      int bad = 0, wrong_bits = 0;
      size_t poison = 0;
      if (le == hipSuccess && se == hipSuccess) {
        CK(hipMemcpy(hc.data(), C, nc * 2, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < nc; ++i) poison += half_bits(hc[i]) == 0x7f7f;
        for (int t = 0; t < 64; ++t) {
          const int m = (int)(((long)t * 37) % s.M), n = (int)(((long)t * 53) % s.N);
          double ref = 0.0;
          for (int k = 0; k < s.K; ++k) ref += (double)ha[(size_t)m * s.K + k] * weight(n, k);
          const _Float16 got = hc[(size_t)m * s.N + n];
          const double d = fabs((double)got - ref) / (fabs(ref) + 1e-3);
          bad += d > 3e-3;
          worst = d > worst ? d : worst;
          wrong_bits += half_bits(got) != half_bits((_Float16)ref);
        }
      }
      const bool ok = app && le == hipSuccess && se == hipSuccess && bad == 0 &&
                      wrong_bits == 0 && poison == 0;
      printf("fmt=%d M=%-5d N=%-6d K=%-6d row=%-16s launch=%s maxrel=%.3e bad=%d bits=%d "
             "poison=%zu %s\n", fmt, s.M, s.N, s.K, row ? row : "(fallback)",
             hipGetErrorString(le), worst, bad, wrong_bits, poison, ok ? "PASS" : "FAIL");
      ok ? ++pass : ++fail;
      CK(hipFree(A));
      CK(hipFree(W));
      CK(hipFree(S));
      CK(hipFree(C));
      if (Z) CK(hipFree(Z));
      if (se != hipSuccess) {
        printf("ship probe gemm_w8a16/gfx950: context lost, PASS %d / FAIL %d\n", pass, fail + 1);
        return 1;
      }
    }
  }
  printf("ship probe gemm_w8a16/gfx950: PASS %d / FAIL %d\n", pass, fail);
  return fail ? 1 : 0;
}
