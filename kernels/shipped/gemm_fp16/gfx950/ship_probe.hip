// ship_probe.hip -- proof that the delivery alone gives a working launcher.
//
// Built from THIS directory's files only (launch.hip, launch_prefill.hip and this probe, with
// -I pointing here and nowhere else), the way a host tree would vendor the delivery:
//
//   hipcc -O3 -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
//         -I . -c launch.hip; (launch_prefill.hip likewise, plus its tempo:flags line)
//   hipcc ... -I . ship_probe.hip launch.o launch_prefill.o -o ship_probe
//
// It runs the reference's acceptance probe of the shipped path
// (kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:35-98): the six production shapes, inputs
// A[i] = ((i%7)-3)/8 and B[i] = ((i%5)-2)/8, output poisoned with 0x7f7f first, 64 cells
// (m = 37t % M, n = 53t % N) against an fp64 dot product with |got-ref|/(|ref|+1e-3) <= 3e-3.
// Every product of these inputs is a multiple of 1/64 and every partial sum stays far below 2^24
// units of 1/64, so the fp32 accumulation is exact in any order: the probe also demands that the
// 64 cells equal the fp16 rounding of the exact sum bit for bit, and that no poison is left
// anywhere in C.  Exit status 0 = every shape passed.
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
  const Shape shapes[] = {{1, 4096, 3840},   {8, 4096, 3840},    {32, 15360, 3840},
                          {128, 4096, 3840}, {512, 15360, 3840}, {2048, 3840, 15360}};
  int pass = 0, fail = 0;
  for (const Shape& s : shapes) {
    const size_t na = (size_t)s.M * s.K, nb = (size_t)s.N * s.K, nc = (size_t)s.M * s.N;
    std::vector<_Float16> ha(na), hb(nb), hc(nc);
    for (size_t i = 0; i < na; ++i) ha[i] = (_Float16)(((int)(i % 7) - 3) * 0.125f);
    for (size_t i = 0; i < nb; ++i) hb[i] = (_Float16)(((int)(i % 5) - 2) * 0.125f);
    _Float16 *A = nullptr, *B = nullptr, *C = nullptr;
    CK(hipMalloc(&A, na * 2));
    CK(hipMalloc(&B, nb * 2));
    CK(hipMalloc(&C, nc * 2));
    CK(hipMemcpy(A, ha.data(), na * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(B, hb.data(), nb * 2, hipMemcpyHostToDevice));
    CK(hipMemset(C, 0x7f, nc * 2));

    tempo::gen::GemmParams p{A, B, C, s.M, s.N, s.K, s.K, s.K, s.N};
    const bool app = tempo::gen::applicable(p);
    const char* row = tempo::gen::route(p);
    const hipError_t le = tempo::gen::launch(p, nullptr);
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
        for (int k = 0; k < s.K; ++k)
          ref += (double)ha[(size_t)m * s.K + k] * (double)hb[(size_t)n * s.K + k];
        const _Float16 got = hc[(size_t)m * s.N + n];
        const double d = fabs((double)got - ref) / (fabs(ref) + 1e-3);
        bad += d > 3e-3;
        worst = d > worst ? d : worst;
        wrong_bits += half_bits(got) != half_bits((_Float16)ref);  // ref is exact: one rounding
      }
    }
    const bool ok = app && le == hipSuccess && se == hipSuccess && bad == 0 && wrong_bits == 0 &&
                    poison == 0;
    printf("M=%-5d N=%-6d K=%-6d row=%-16s launch=%s maxrel=%.3e bad=%d bits=%d poison=%zu %s\n",
           s.M, s.N, s.K, row ? row : "(fallback)", hipGetErrorString(le), worst, bad,
           wrong_bits, poison, ok ? "PASS" : "FAIL");
    ok ? ++pass : ++fail;
    CK(hipFree(A));
    CK(hipFree(B));
    CK(hipFree(C));
    if (se != hipSuccess) break;  // the context is gone: nothing after this can be trusted
  }
  printf("ship probe gemm_fp16/gfx950: PASS %d / FAIL %d\n", pass, fail);
  return fail ? 1 : 0;
}
