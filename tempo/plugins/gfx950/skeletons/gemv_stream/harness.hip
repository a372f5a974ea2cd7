// harness.hip -- measuring harness of the gemv_stream skeleton (decode regime) on gfx950.
// Reference pattern: tempo/plugins/sm70/skeletons/gemm_w8a16/harness.cu (gate: poison +
// relL2 against a straightforward reference, then timing; JSON lines).
//
// Build: hipcc -O3 -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang
//        -packed-fp32-ops -I<configs dir> -I<skeletons dir> harness.hip -o harness_stream
// Run:   ./harness_stream FMT M N K [iters] [S]
//   FMT 0 fp16 weights, 1 int8 + row scale, 2 uint8 + group-128 scale/zero.
//   S    waves per workgroup (k split); 0 = the launcher's rule.
//
// The reference output comes from a separate dequantise kernel (closed form in float) and the
// naive one-thread-per-output GEMM, so the variant under test shares no device code with it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace tempo {
namespace tune {
#include "common/cdna4.h"
#include "gemv_stream/kernel.hip"
}  // namespace tune
}  // namespace tempo

using namespace tempo::tune;

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      printf("HIPERR %s @%d: %s\n", #x, __LINE__, hipGetErrorString(e_));              \
      exit(2);                                                                         \
    }                                                                                  \
  } while (0)

__device__ unsigned hmix(long i, unsigned seed) {
  unsigned h = (unsigned)i * 2654435761u + seed;
  h ^= h >> 15;
  h *= 2246822519u;
  h ^= h >> 13;
  return h;
}
__global__ void k_fill_h(_Float16* p, long n, unsigned seed, float scale) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = (_Float16)((((float)(hmix(i, seed) & 0xFFFF) / 65535.f) - 0.5f) * scale);
}
__global__ void k_fill_b(uint8_t* p, long n, unsigned seed, int lo, int span) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = (uint8_t)(lo + (int)(hmix(i, seed) % (unsigned)span));
}
// reference dequantisation in float arithmetic (closed forms of the formats)
__global__ void k_deq_ref(int fmt, const void* B, const _Float16* s, const uint8_t* z, _Float16* W,
                          int N, int K) {
  const long n_tot = (long)N * K;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n_tot; i += (long)gridDim.x * blockDim.x) {
    const long n = i / K, k = i % K;
    if (fmt == 0) {
      W[i] = reinterpret_cast<const _Float16*>(B)[i];
    } else if (fmt == 1) {
      W[i] = (_Float16)((float)reinterpret_cast<const int8_t*>(B)[i] * (float)s[n]);
    } else {
      const long g = n * (K / 128) + k / 128;
      W[i] = (_Float16)((float)((int)reinterpret_cast<const uint8_t*>(B)[i] - (int)z[g]) * (float)s[g]);
    }
  }
}
__global__ void k_naive(const _Float16* A, const _Float16* B, _Float16* C, int M, int N, int K) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (m >= M || n >= N) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = __builtin_fmaf((float)A[(long)m * K + k], (float)B[(long)n * K + k], acc);
  C[(long)m * N + n] = (_Float16)acc;
}
__global__ void k_rel(const _Float16* a, const _Float16* b, long n, double* out) {
  double d = 0, r = 0;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const double x = (double)(float)a[i], y = (double)(float)b[i];
    d += (x - y) * (x - y);
    r += y * y;
  }
  atomicAdd(out, d);
  atomicAdd(out + 1, r);
}
__global__ void k_poison_count(const _Float16* a, long n, unsigned long long* o) {
  unsigned long long c = 0;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    if (*reinterpret_cast<const unsigned short*>(a + i) == 0x7f7f) ++c;
  atomicAdd(o, c);
}
__global__ void k_fill_u16(unsigned short* p, long n, unsigned short v) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = v;
}

// the launcher's k-split rule (kernels/shipped/gemm_w8a16/gfx950/launch.h stream_split)
static void split_rule(int N, int K, int R, int U, int* S_out, int* chunk_out, int force_s) {
  const int slabs = N / (16 * R);
  const int stages = K / (64 * U);
  int S = force_s > 0 ? force_s : (2048 + slabs - 1) / slabs;
  if (S > 8) S = 8;
  if (S > stages) S = stages;
  if (S < 1) S = 1;
  const int per = (stages + S - 1) / S;
  S = (stages + per - 1) / per;
  *S_out = S;
  *chunk_out = per * 64 * U;
}

typedef void (*LaunchFn)(StreamArgs, hipStream_t);
struct Arm {
  const char* tag;
  int MB, R, U, BFMT;  // U = k-steps per stage (register kernel) or 1 (ring kernel)
  int D;               // ring depth (LDS-DMA kernel), 0 for the register kernel
  LaunchFn launch;
  int SN = 0;          // shared-activation kernel: slab waves per workgroup (0: other kernels)
  int TPB = 512;       // shared-activation kernel: launch bound
};
template <int MB, int R, int U, int BFMT, int ALDS = 0>
static void launch_arm(StreamArgs a, hipStream_t s) {
  const dim3 grid(a.N / (16 * R)), blk(64 * a.S);
  const size_t lds = (a.S > 1 ? (size_t)a.S * R * MB * 64 * 16 : 0) +
                     (ALDS ? (size_t)a.M * (2 * (size_t)a.K + 16) : 0);
  hipLaunchKernelGGL((k_stream<MB, R, U, BFMT, ALDS>), grid, blk, lds, s, a);
}
template <int MB, int R, int D, int BFMT>
static void launch_arm_dma(StreamArgs a, hipStream_t s) {
  const dim3 grid(a.N / (16 * R)), blk(64 * a.S);
  const size_t lds = stream_dma_lds<MB, R, D, BFMT>(a.S);
  hipLaunchKernelGGL((k_stream_dma<MB, R, D, BFMT>), grid, blk, lds, s, a);
}
template <int MB, int R, int U, int BFMT, int SN, int TPB>
static void launch_arm_sh(StreamArgs a, hipStream_t s) {
  const dim3 grid(a.N / (16 * R * SN)), blk(64 * SN * a.S);
  const size_t lds = StreamSh<MB, U>::lds(SN, a.S, R);
  hipLaunchKernelGGL((k_stream_sh<MB, R, U, BFMT, SN, TPB>), grid, blk, lds, s, a);
}
// k-chunks of the shared kernel: about 2048 waves over the part, at most 8 waves per
// workgroup, the stage count divisible by the chunk count
static void sh_split(int N, int K, int R, int U, int SN, int TPB, int* SK_out, int* chunk_out) {
  const int stages = K / (64 * U);
  const int wgs = N / (16 * R * SN);
  int SK = (2048 + wgs * SN - 1) / (wgs * SN);
  if (SK > TPB / 64 / SN) SK = TPB / 64 / SN;
  if (SK < 1) SK = 1;
  while (stages % SK) --SK;
  *SK_out = SK;
  *chunk_out = stages / SK * 64 * U;
}
#define STREAMS(tag, MB, R, U, F, SN, TPB) \
  Arm{tag, MB, R, U, F, 0, &launch_arm_sh<MB, R, U, F, SN, TPB>, SN, TPB},
#define STREAM(tag, MB, R, U, F) Arm{tag, MB, R, U, F, 0, &launch_arm<MB, R, U, F>},
#define STREAMA(tag, MB, R, U, F) Arm{tag, MB, R, U, F, -1, &launch_arm<MB, R, U, F, 1>},
#define STREAMD(tag, MB, R, D, F) Arm{tag, MB, R, 1, F, D, &launch_arm_dma<MB, R, D, F>},

static const Arm kArms[] = {
#include "configs_stream.inc"
};

// `./harness_stream probe`: streaming-read ceiling through the LDS-DMA ring, 2 GiB rotated,
// for several ring depths and grid sizes.
template <int D>
static void probe_one(const uint8_t* src, long total, int waves, unsigned* out, hipEvent_t e0,
                      hipEvent_t e1) {
  const long per_wave = (total / waves) / 1024 * 1024;
  const int blocks = waves / 4;
  for (int i = 0; i < 3; ++i)
    hipLaunchKernelGGL((k_read_probe<D>), dim3(blocks), dim3(256), 0, 0, src, per_wave, out);
  CK(hipDeviceSynchronize());
  const int it = 10;
  CK(hipEventRecord(e0, 0));
  for (int i = 0; i < it; ++i)
    hipLaunchKernelGGL((k_read_probe<D>), dim3(blocks), dim3(256), 0, 0, src, per_wave, out);
  CK(hipEventRecord(e1, 0));
  CK(hipEventSynchronize(e1));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, e0, e1));
  const double t = ms / it * 1e-3, bytes = (double)per_wave * waves;
  printf("PROBE {\"D\":%d,\"waves\":%d,\"bytes\":%.0f,\"us\":%.1f,\"GBps\":%.0f}\n", D, waves, bytes,
         t * 1e6, bytes / t / 1e9);
  fflush(stdout);
}

static int probe_main() {
  const long total = 2L << 30;
  uint8_t* src;
  unsigned* out;
  CK(hipMalloc(&src, total));
  CK(hipMalloc(&out, 64));
  CK(hipMemset(src, 1, total));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  for (int waves : {2048, 4096, 8192}) {
    probe_one<8>(src, total, waves, out, e0, e1);
    probe_one<16>(src, total, waves, out, e0, e1);
    probe_one<32>(src, total, waves, out, e0, e1);
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "probe") return probe_main();
  const int fmt = argc > 1 ? atoi(argv[1]) : 1;
  const int M = argc > 2 ? atoi(argv[2]) : 1;
  const int N = argc > 3 ? atoi(argv[3]) : 34816;
  const int K = argc > 4 ? atoi(argv[4]) : 5120;
  const int iters = argc > 5 ? atoi(argv[5]) : 50;
  const int force_s = argc > 6 ? atoi(argv[6]) : 0;
  const long nw = (long)N * K, ng = (long)N * (K / 128);
  const int eb = fmt == 0 ? 2 : 1;
  const int nrot = std::max(2, (int)std::ceil(640.0 * 1024 * 1024 / (double)(nw * eb)));
  _Float16 *A, *C, *R, *W, *S;
  uint8_t* Z;
  std::vector<void*> Bs(nrot);
  CK(hipMalloc(&A, (size_t)M * K * 2));
  CK(hipMalloc(&C, (size_t)M * N * 2));
  CK(hipMalloc(&R, (size_t)M * N * 2));
  CK(hipMalloc(&W, (size_t)nw * 2));
  CK(hipMalloc(&S, (size_t)std::max<long>(ng, N) * 2));
  CK(hipMalloc(&Z, (size_t)ng));
  for (int i = 0; i < nrot; ++i) {
    CK(hipMalloc(&Bs[i], (size_t)nw * eb));
    if (fmt == 0)
      hipLaunchKernelGGL(k_fill_h, dim3(2048), dim3(256), 0, 0, (_Float16*)Bs[i], nw, 77u + i, 2.f / sqrtf((float)K));
    else if (fmt == 1)  // int8 uniform in [-127, 127] (two's complement bytes)
      hipLaunchKernelGGL(k_fill_b, dim3(2048), dim3(256), 0, 0, (uint8_t*)Bs[i], nw, 77u + i, -127, 255);
    else
      hipLaunchKernelGGL(k_fill_b, dim3(2048), dim3(256), 0, 0, (uint8_t*)Bs[i], nw, 77u + i, 0, 256);
  }
  hipLaunchKernelGGL(k_fill_h, dim3(256), dim3(256), 0, 0, A, (long)M * K, 11u, 2.f);
  hipLaunchKernelGGL(k_fill_h, dim3(256), dim3(256), 0, 0, S, std::max<long>(ng, N), 5u, 0.01f);
  hipLaunchKernelGGL(k_fill_b, dim3(256), dim3(256), 0, 0, Z, ng, 3u, 100, 57);
  hipLaunchKernelGGL(k_deq_ref, dim3(4096), dim3(256), 0, 0, fmt, Bs[0], S, Z, W, N, K);
  hipLaunchKernelGGL(k_naive, dim3((N + 255) / 256, M), dim3(256), 0, 0, A, W, R, M, N, K);
  CK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  const double bytes = (double)nw * eb + (fmt == 1 ? 2.0 * N : fmt == 2 ? 3.0 * ng : 0.0) +
                       2.0 * M * K + 2.0 * M * N;
  printf("SHAPE {\"fmt\":%d,\"M\":%d,\"N\":%d,\"K\":%d,\"rotate\":%d,\"bytes\":%.0f}\n", fmt, M, N, K, nrot, bytes);
  fflush(stdout);
  for (const Arm& arm : kArms) {
    if (arm.BFMT != fmt || M > 16 * arm.MB || (N % (16 * arm.R)) != 0 || (K % (64 * arm.U)) != 0) continue;
    StreamArgs a;
    a.A = A;
    a.B = Bs[0];
    a.scale = S;
    a.zero = Z;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = K;
    a.ldb = K;
    a.ldc = N;
    a.group = 128;
    split_rule(N, K, arm.R, arm.U, &a.S, &a.chunk, force_s);
    if (arm.SN > 0) {
      if (N % (16 * arm.R * arm.SN)) continue;
      sh_split(N, K, arm.R, arm.U, arm.SN, arm.TPB, &a.S, &a.chunk);
      // activation rings of every k-chunk + the reduction must fit the 160 KiB of LDS
      const size_t stage = (size_t)16 * arm.MB * 128 * arm.U;
      while (a.S > 1 && (size_t)a.S * 2 * stage + (size_t)arm.SN * a.S * arm.R * arm.MB * 1024 >
                            160 * 1024) {
        const int stages = K / (64 * arm.U);
        int sk = a.S - 1;
        while (stages % sk) --sk;
        a.S = sk;
        a.chunk = stages / sk * 64 * arm.U;
      }
    }
    if (arm.D < 0 && (size_t)M * (2 * (size_t)K + 16) > 96 * 1024) continue;  // LDS activations
    if (arm.D > 0) {  // ring kernel: LDS of S waves within 160 KiB; fmt 2 chunk <= 8192 k
      const size_t per_wave = (size_t)arm.D * (arm.R * eb + 2 * arm.MB) * 1024 +
                              (fmt == 2 ? (size_t)arm.R * 16 * 64 * 3 : 0) +
                              (size_t)arm.R * arm.MB * 1024;
      const int steps = K / 64;
      int S = a.S;
      auto fix = [&](int s_) {
        const int per = (steps + s_ - 1) / s_;
        a.S = (steps + per - 1) / per;
        a.chunk = per * 64;
      };
      while (fmt == 2 && (K + S - 1) / S > 8192 && S < 8) ++S;
      fix(S);
      while (a.S > 1 && (size_t)a.S * per_wave > 160 * 1024) fix(a.S - 1);
      if ((size_t)a.S * per_wave > 160 * 1024 || (fmt == 2 && a.chunk > 8192)) continue;
    }
    hipLaunchKernelGGL(k_fill_u16, dim3(256), dim3(256), 0, 0, (unsigned short*)C, (long)M * N, (unsigned short)0x7f7f);
    arm.launch(a, 0);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    unsigned long long* dcnt;
    double* drel;
    CK(hipMalloc(&dcnt, 8));
    CK(hipMalloc(&drel, 16));
    CK(hipMemset(dcnt, 0, 8));
    CK(hipMemset(drel, 0, 16));
    hipLaunchKernelGGL(k_poison_count, dim3(256), dim3(256), 0, 0, C, (long)M * N, dcnt);
    hipLaunchKernelGGL(k_rel, dim3(256), dim3(256), 0, 0, C, R, (long)M * N, drel);
    CK(hipDeviceSynchronize());
    unsigned long long left;
    double h[2];
    CK(hipMemcpy(&left, dcnt, 8, hipMemcpyDeviceToHost));
    CK(hipMemcpy(h, drel, 16, hipMemcpyDeviceToHost));
    CK(hipFree(dcnt));
    CK(hipFree(drel));
    const double rel = h[1] > 0 ? sqrt(h[0] / h[1]) : 1.0;
    if (left || !(rel <= 3e-3)) {
      printf("FAILGATE {\"tag\":\"%s\",\"S\":%d,\"uncovered\":%llu,\"rel\":%.3e}\n", arm.tag, a.S, left, rel);
      fflush(stdout);
      continue;
    }
    for (int i = 0; i < 5; ++i) {
      a.B = Bs[i % nrot];
      arm.launch(a, 0);
    }
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; ++i) {
      a.B = Bs[i % nrot];
      arm.launch(a, 0);
    }
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    const double t = ms / iters;
    printf("CAND {\"tag\":\"%s\",\"fmt\":%d,\"M\":%d,\"N\":%d,\"K\":%d,\"S\":%d,\"us\":%.2f,\"GBps\":%.0f,\"hbm_frac\":%.3f,\"rel\":%.2e}\n",
           arm.tag, fmt, M, N, K, a.S, t * 1e3, bytes / (t * 1e-3) / 1e9, bytes / (t * 1e-3) / 8e12, rel);
    fflush(stdout);
  }
  return 0;
}
