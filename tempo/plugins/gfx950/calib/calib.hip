// gfx950 machine calibration: the probes behind the MEASURED rates of the plugin's rate table.
//
// The reference states its HBM bandwidth as three measured modes, each with its access pattern
// named (pure read / read / copy: tempo/plugins/sm70/__init__.py:110-131), and its loader accepts
// a MEASURED rate only with the card state it was taken on (tempo/plugins/registry.py:67-76).
// These probes take the same three modes on MI355X, plus the matrix-core and LDS rates and the
// engine clock, with kernels of their own:
//
//   hbm_read_pure  every lane loads 16 bytes per access, nontemporal (the line is not kept in the
//                  caches), 8 loads in flight per lane, values folded with xor -- nothing but
//                  the read; two access patterns (a grid-wide stride, and each workgroup
//                  streaming a contiguous share), each mode's rate the faster of the two;
//   hbm_read       the same traffic as fp16 data summed in fp32 (ordinary cached loads): the read
//                  a consuming kernel does;
//   hbm_copy       16-byte load, 16-byte store; bytes counted read + written;
//   mfma           v_mfma_f32_32x32x16_f16 on register operands, 4 independent accumulators per
//                  wave, 2 waves per SIMD;
//   lds            ds_read_b128 without bank conflicts (each half-wave reads 512 contiguous
//                  bytes), 16 reads in flight per lane, up to 8 waves per SIMD;
//   clock          s_memtime (engine clock cycles) against s_memrealtime (constant-rate counter)
//                  over a short spin, one wave per CU.
//
// Buffers are sized by the caller; every kernel checks its sizes on the host (the launchers
// below return hipErrorInvalidValue for a size the grid does not tile exactly), so every access
// is in bounds.  Results are written to plain device arrays the host reads back.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int TPB = 256;
constexpr int UNROLL = 8;

// grid-stride over E 16-byte elements; E is a multiple of UNROLL x (grid threads)
__global__ __launch_bounds__(TPB) void k_read_pure(const u32x4* __restrict__ src, long E,
                                                  unsigned* __restrict__ out) {
  const long T = (long)gridDim.x * TPB;
  const long t = (long)blockIdx.x * TPB + threadIdx.x;
  u32x4 x = {0u, 0u, 0u, 0u};
  for (long i = t; i < E; i += UNROLL * T) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * T);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) x ^= v[u];
  }
  out[t] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

// the same read, each workgroup streaming a contiguous 1/gridDim of the buffer: per iteration a
// workgroup takes 32 KiB (lane t of load u reads element base + u*256 + t), so consecutive
// requests of one CU stay inside a DRAM page; E is a multiple of 2048 x gridDim
__global__ __launch_bounds__(TPB) void k_read_pure_wg(const u32x4* __restrict__ src, long E,
                                                     unsigned* __restrict__ out) {
  const long per = E / gridDim.x;
  const u32x4* p = src + (long)blockIdx.x * per + threadIdx.x;
  u32x4 x = {0u, 0u, 0u, 0u};
  for (long i = 0; i < per; i += UNROLL * TPB) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(p + i + u * TPB);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) x ^= v[u];
  }
  out[(long)blockIdx.x * TPB + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

__global__ __launch_bounds__(TPB) void k_read_sum_wg(const f16x8* __restrict__ src, long E,
                                                    float* __restrict__ out) {
  const long per = E / gridDim.x;
  const f16x8* p = src + (long)blockIdx.x * per + threadIdx.x;
  float acc = 0.f;
  for (long i = 0; i < per; i += UNROLL * TPB) {
    f16x8 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = p[i + u * TPB];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += (float)v[u][j];
  }
  out[(long)blockIdx.x * TPB + threadIdx.x] = acc;
}

__global__ __launch_bounds__(TPB) void k_copy_wg(const u32x4* __restrict__ src,
                                                u32x4* __restrict__ dst, long E) {
  const long per = E / gridDim.x;
  const long b = (long)blockIdx.x * per + threadIdx.x;
  for (long i = 0; i < per; i += UNROLL * TPB) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = src[b + i + u * TPB];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) dst[b + i + u * TPB] = v[u];
  }
}

__global__ __launch_bounds__(TPB) void k_read_sum(const f16x8* __restrict__ src, long E,
                                                 float* __restrict__ out) {
  const long T = (long)gridDim.x * TPB;
  const long t = (long)blockIdx.x * TPB + threadIdx.x;
  float acc = 0.f;
  for (long i = t; i < E; i += UNROLL * T) {
    f16x8 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = src[i + u * T];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += (float)v[u][j];
  }
  out[t] = acc;
}

__global__ __launch_bounds__(TPB) void k_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                             long E) {
  const long T = (long)gridDim.x * TPB;
  const long t = (long)blockIdx.x * TPB + threadIdx.x;
  for (long i = t; i < E; i += UNROLL * T) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = src[i + u * T];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) dst[i + u * T] = v[u];
  }
}

// ITERS x 4 independent 32x32x16 MFMAs per wave; one float per lane is written so the chains
// stay live.  clk[2*blockIdx.x] / [+1] take the wave's engine-clock and constant-clock deltas.
__global__ __launch_bounds__(TPB) void k_mfma(int iters, float seed, float* __restrict__ out,
                                             long long* __restrict__ clk) {
  f16x8v a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)(seed * (float)(threadIdx.x + j));
    b[j] = (_Float16)(seed * (float)(threadIdx.x - j));
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  const long long m0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
  }
  const long long m1 = clock64(), r1 = wall_clock64();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  out[(long)blockIdx.x * TPB + threadIdx.x] = s;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = m1 - m0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// LDS read rate: 16 KiB per workgroup (up to 8 workgroups, 32 waves, per CU), ITERS rounds of
// 16 reads of 16 bytes per lane; lane l of read u reads chunk (c + u*64) % 1024, c advancing by 64
// per round -- each half-wave covers 512 contiguous bytes, all 64 banks once.
// clk[2*blockIdx.x] / [+1]: engine-clock and constant-clock deltas of the read loop (wave 0).
__global__ __launch_bounds__(TPB) void k_lds(int iters, unsigned* __restrict__ out,
                                            long long* __restrict__ clk) {
  __shared__ u32x4 lds[1024];
  for (int i = threadIdx.x; i < 1024; i += TPB) lds[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  u32x4 x = {0u, 0u, 0u, 0u};
  int c = wave * 256 + lane;
  const long long m0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 16; ++u) x ^= lds[(c + u * 64) & 1023];
    c = (c + 1024 + 64) & 1023;
  }
  const long long m1 = clock64(), r1 = wall_clock64();
  out[(long)blockIdx.x * TPB + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = m1 - m0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// one wave per workgroup: a dependent spin of `spin` steps between two clock reads
__global__ __launch_bounds__(64) void k_clock(int spin, long long* __restrict__ clk,
                                             float* __restrict__ sink) {
  float v = (float)threadIdx.x;
  const long long m0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < spin; ++i) v = v * 0.999f + 1.0f;
  const long long m1 = clock64(), r1 = wall_clock64();
  sink[(long)blockIdx.x * 64 + threadIdx.x] = v;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = m1 - m0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// nothing: back-to-back launches of it time the dispatch and completion of a launch alone
__global__ __launch_bounds__(64) void k_empty() {}

}  // namespace

extern "C" {

int calib_empty(int blocks, hipStream_t s) {
  if (blocks <= 0) return hipErrorInvalidValue;
  k_empty<<<blocks, 64, 0, s>>>();
  return hipGetLastError();
}


// Each launcher checks that the grid tiles its buffer exactly before it launches.
int calib_read_pure(const void* src, long bytes, int blocks, void* out, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_read_pure<<<blocks, TPB, 0, s>>>(static_cast<const u32x4*>(src), E,
                                     static_cast<unsigned*>(out));
  return hipGetLastError();
}

// pattern 1: each workgroup streams a contiguous 1/blocks of the buffer
int calib_read_pure_wg(const void* src, long bytes, int blocks, void* out, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_read_pure_wg<<<blocks, TPB, 0, s>>>(static_cast<const u32x4*>(src), E,
                                        static_cast<unsigned*>(out));
  return hipGetLastError();
}

int calib_read_sum_wg(const void* src, long bytes, int blocks, void* out, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_read_sum_wg<<<blocks, TPB, 0, s>>>(static_cast<const f16x8*>(src), E,
                                       static_cast<float*>(out));
  return hipGetLastError();
}

int calib_copy_wg(const void* src, void* dst, long bytes, int blocks, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_copy_wg<<<blocks, TPB, 0, s>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), E);
  return hipGetLastError();
}

int calib_read_sum(const void* src, long bytes, int blocks, void* out, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_read_sum<<<blocks, TPB, 0, s>>>(static_cast<const f16x8*>(src), E, static_cast<float*>(out));
  return hipGetLastError();
}

int calib_copy(const void* src, void* dst, long bytes, int blocks, hipStream_t s) {
  const long E = bytes / 16;
  if (bytes % 16 || blocks <= 0 || E % ((long)UNROLL * blocks * TPB)) return hipErrorInvalidValue;
  k_copy<<<blocks, TPB, 0, s>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), E);
  return hipGetLastError();
}

// out: blocks x 256 floats; clk: 2 x blocks long longs
int calib_mfma(int blocks, int iters, void* out, void* clk, hipStream_t s) {
  if (blocks <= 0 || iters <= 0) return hipErrorInvalidValue;
  k_mfma<<<blocks, TPB, 0, s>>>(iters, 1.0f / 1024.0f, static_cast<float*>(out),
                                static_cast<long long*>(clk));
  return hipGetLastError();
}

// out: blocks x 256 unsigned; clk: 2 x blocks long longs
int calib_lds(int blocks, int iters, void* out, void* clk, hipStream_t s) {
  if (blocks <= 0 || iters <= 0) return hipErrorInvalidValue;
  k_lds<<<blocks, TPB, 0, s>>>(iters, static_cast<unsigned*>(out), static_cast<long long*>(clk));
  return hipGetLastError();
}

// clk: 2 x blocks long longs; sink: blocks x 64 floats
int calib_clock(int blocks, int spin, void* clk, void* sink, hipStream_t s) {
  if (blocks <= 0 || spin <= 0) return hipErrorInvalidValue;
  k_clock<<<blocks, 64, 0, s>>>(spin, static_cast<long long*>(clk), static_cast<float*>(sink));
  return hipGetLastError();
}

// kHz of the constant-rate counter wall_clock64() reads
int calib_wall_clock_khz(int device, int* khz) {
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, device);
}

}  // extern "C"
