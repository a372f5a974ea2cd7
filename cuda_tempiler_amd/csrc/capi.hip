// capi.hip -- extern "C" boundary of libtempo_gfx950.so (declarations: include/tempo_gfx950.h).
//
// Thin by design: it converts the C structs into the shipped deliveries' POD parameters and
// calls their launch(); every kernel decision lives in the deliveries (kernels/shipped/...) and
// the FMHA skeleton.  No framework type crosses this file.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>

#include "tempo_gfx950.h"
#include "gemm_fp16/gfx950/launch.h"
#include "gemm_w8a16/gfx950/launch.h"
#include "naive/gemm_fp16.hip"
#include "naive/gemm_w8a16.hip"
#include "naive/fmha_fwd.hip"
#include "fmha_api.h"

namespace {

using tempo::gen::Mfma;
using tempo::gen::f16x8;

template <int MS>
__global__ void k_probe_layout(float* out) {
  const int l = threadIdx.x;
  constexpr int NACC = Mfma<MS>::NACC;
  for (int pass = 0; pass < 2; ++pass) {
    typename Mfma<MS>::acc_t acc;
    for (int v = 0; v < NACC; ++v) acc[v] = 0.f;
    f16x8 a, b;
    for (int e = 0; e < 8; ++e) {
      a[e] = (_Float16)0.f;
      b[e] = (_Float16)0.f;
    }
    if (l / MS == 0) {  // one k slot (k-group 0, element 0) carries a rank-1 product
      a[0] = (_Float16)(pass == 0 ? (float)(l % MS + 1) : 1.f);
      b[0] = (_Float16)(pass == 0 ? 1.f : (float)(l % MS + 1));
    }
    acc = Mfma<MS>::run(a, b, acc);
    for (int v = 0; v < NACC; ++v) out[(pass * 64 + l) * NACC + v] = acc[v];
  }
}

tempo::gen::GemmParams to_pod(const TempoGemmParams* p) {
  tempo::gen::GemmParams g;
  g.A = static_cast<const _Float16*>(p->A);
  g.B = static_cast<const _Float16*>(p->B);
  g.C = static_cast<_Float16*>(p->C);
  g.M = p->M;
  g.N = p->N;
  g.K = p->K;
  g.lda = p->lda;
  g.ldb = p->ldb;
  g.ldc = p->ldc;
  return g;
}

tempo::gen8::W8A16Params to_pod(const TempoW8A16Params* p) {
  tempo::gen8::W8A16Params g;
  g.A = static_cast<const _Float16*>(p->A);
  g.Wq = p->Wq;
  g.scale = static_cast<const _Float16*>(p->scale);
  g.zero = static_cast<const uint8_t*>(p->zero);
  g.C = static_cast<_Float16*>(p->C);
  g.M = p->M;
  g.N = p->N;
  g.K = p->K;
  g.lda = p->lda;
  g.ldw = p->ldw;
  g.ldc = p->ldc;
  g.group = p->group;
  g.fmt = p->fmt;
  return g;
}

// ---- the allocation-free entry point's scratch ------------------------------------------------
// A file-scope device array: every GPU the library runs on holds its own copy, at its own address,
// from module load until the process ends.  Host code never passes `scratch` itself to a kernel
// (in host code the name is a stand-in, not a device address): the address is looked up once per
// device with hipGetSymbolAddress, with that device current, and kept in scratch_ptr[].
static __device__ __align__(256) unsigned char scratch[TEMPO_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* scratch_ptr[kMaxDevices] = {};
std::mutex scratch_mu;

// The current device's scratch address (nullptr with *err set when it cannot be had).
void* device_scratch(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}

int copy_tag(const char* t, char* tag, int tag_len) {
  if (tag && tag_len > 0) {
    const char* s = t ? t : "";
    std::strncpy(tag, s, (size_t)tag_len - 1);
    tag[tag_len - 1] = '\0';
  }
  return t ? 1 : 0;
}

}  // namespace

extern "C" {

int tempo_abi_version(void) { return 1; }

int tempo_gemm_fp16_applicable(const TempoGemmParams* p) {
  if (!p) return 0;
  return tempo::gen::route(to_pod(p)) != nullptr;
}

int tempo_gemm_fp16_launch(const TempoGemmParams* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  return (int)tempo::gen::launch(to_pod(p), static_cast<hipStream_t>(stream));
}

int tempo_gemm_fp16_launch_ws(const TempoGemmParams* p, void* ws, size_t ws_bytes,
                              tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  tempo::gen::Workspace w;
  w.ptr = ws;
  w.bytes = ws ? ws_bytes : 0;
  w.pool = false;
  return (int)tempo::gen::launch_with(to_pod(p), static_cast<hipStream_t>(stream), w);
}

size_t tempo_gemm_fp16_workspace_bytes(const TempoGemmParams* p) {
  if (!p) return 0;
  return tempo::gen::workspace_bytes(to_pod(p));
}

size_t tempo_gemm_w8a16_workspace_bytes(const TempoW8A16Params* p) {
  if (!p) return 0;
  return tempo::gen8::workspace_bytes(to_pod(p));
}

int tempo_gemm_w8a16_applicable(const TempoW8A16Params* p) {
  if (!p) return 0;
  return tempo::gen8::route(to_pod(p)) != nullptr;
}

int tempo_gemm_w8a16_launch(const TempoW8A16Params* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  return (int)tempo::gen8::launch(to_pod(p), static_cast<hipStream_t>(stream));
}

int tempo_gemm_w8a16_launch_ws(const TempoW8A16Params* p, void* ws, size_t ws_bytes,
                               tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  tempo::gen8::Workspace w;
  w.ptr = ws;
  w.bytes = ws ? ws_bytes : 0;
  w.pool = false;
  return (int)tempo::gen8::launch_with(to_pod(p), static_cast<hipStream_t>(stream), w);
}

int tempo_gemm_w8a16_launch_noalloc(const TempoW8A16Params* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  hipError_t err = hipSuccess;
  tempo::gen8::Workspace w;
  w.ptr = device_scratch(&err);
  if (!w.ptr) return (int)err;
  w.bytes = TEMPO_NOALLOC_SCRATCH_BYTES;
  w.pool = false;  // a row whose workspace exceeds the scratch returns hipErrorOutOfMemory
  return (int)tempo::gen8::launch_with(to_pod(p), static_cast<hipStream_t>(stream), w);
}

int tempo_gemm_fp16_gate_up_launch(const TempoGemmParams* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  return (int)tempo::gen::launch_gate_up(to_pod(p), static_cast<hipStream_t>(stream));
}

int tempo_gemm_w8a16_gate_up_launch(const TempoW8A16Params* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  return (int)tempo::gen8::launch_gate_up(to_pod(p), static_cast<hipStream_t>(stream));
}

int tempo_dequant_tile(const TempoW8A16Params* p, int n0, int k0, int rows, int cols, void* out,
                       tempo_stream_t stream) {
  if (!p || !out) return (int)hipErrorInvalidValue;
  return (int)tempo::gen8::dequant_tile(to_pod(p), n0, k0, rows, cols,
                                        static_cast<_Float16*>(out),
                                        static_cast<hipStream_t>(stream));
}

int tempo_fmha_fwd_applicable(const TempoFmhaParams* p) {
  if (!p) return 0;
  return tempo_fmha::applicable(*p) ? 1 : 0;
}

int tempo_fmha_fwd_launch(const TempoFmhaParams* p, tempo_stream_t stream) {
  if (!p) return (int)hipErrorInvalidValue;
  return (int)tempo_fmha::launch(*p, static_cast<hipStream_t>(stream));
}

int tempo_naive_gemm_fp16_launch(const void* A, const void* B, void* C, int M, int N, int K,
                                 tempo_stream_t stream) {
  if (!A || !B || !C || M <= 0 || N <= 0 || K <= 0) return (int)hipErrorInvalidValue;
  return (int)naive_gemm_fp16_launch(static_cast<const _Float16*>(A),
                                     static_cast<const _Float16*>(B), static_cast<_Float16*>(C),
                                     M, N, K, static_cast<hipStream_t>(stream));
}

int tempo_naive_gemm_w8a16_launch(const TempoW8A16Params* p, tempo_stream_t stream) {
  if (!p || !p->A || !p->Wq || !p->scale || !p->C || p->M <= 0 || p->N <= 0 || p->K <= 0)
    return (int)hipErrorInvalidValue;
  if (p->lda != p->K || p->ldw != p->K || p->ldc != p->N) return (int)hipErrorInvalidValue;
  if (p->fmt == TEMPO_W8_ASYM_U8) {
    if (!p->zero || p->group <= 0 || p->K % p->group != 0) return (int)hipErrorInvalidValue;
  } else if (p->fmt != TEMPO_W8_SYM_I8) {
    return (int)hipErrorInvalidValue;
  }
  return (int)naive_gemm_w8a16_launch(
      static_cast<const _Float16*>(p->A), p->Wq, static_cast<const _Float16*>(p->scale),
      static_cast<const uint8_t*>(p->zero), static_cast<_Float16*>(p->C), p->M, p->N, p->K,
      p->fmt == TEMPO_W8_ASYM_U8 ? p->group : 0, p->fmt, static_cast<hipStream_t>(stream));
}

int tempo_naive_fmha_fwd_launch(const void* Q, const void* K, const void* V, void* O, float* LSE,
                                int B, int H, int Hkv, int Sq, int Sk, int D, float scale,
                                int causal, tempo_stream_t stream) {
  if (!Q || !K || !V || !O) return (int)hipErrorInvalidValue;
  return (int)naive_fmha_fwd_launch(static_cast<const _Float16*>(Q), static_cast<const _Float16*>(K),
                                    static_cast<const _Float16*>(V), static_cast<_Float16*>(O), LSE,
                                    B, H, Hkv, Sq, Sk, D, scale, causal,
                                    static_cast<hipStream_t>(stream));
}

int tempo_probe_mfma_layout(int ms, float* out, tempo_stream_t stream) {
  if (!out) return (int)hipErrorInvalidValue;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ms == 32)
    hipLaunchKernelGGL(k_probe_layout<32>, dim3(1), dim3(64), 0, s, out);
  else if (ms == 16)
    hipLaunchKernelGGL(k_probe_layout<16>, dim3(1), dim3(64), 0, s, out);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

int tempo_route(int op, int M, int N, int K, char* tag, int tag_len) {
  // Host-only: dummy 16-byte-aligned addresses stand in for device pointers (never touched).
  const uintptr_t fake = 0x1000;
  const bool gu = op >= 3 && op <= 5;  // fused gate/up variants of ops 0..2
  const int base = gu ? op - 3 : op;
  if (base == 0) {
    TempoGemmParams p = {(const void*)fake, (const void*)fake, (void*)fake, M, N, K, K, K, N};
    return copy_tag(gu ? tempo::gen::route_gate_up(to_pod(&p)) : tempo::gen::route(to_pod(&p)),
                    tag, tag_len);
  }
  if (base == 1 || base == 2) {
    TempoW8A16Params p = {(const void*)fake, (const void*)fake, (const void*)fake,
                          base == 2 ? (const void*)fake : nullptr, (void*)fake, M, N, K, K, K, N,
                          base == 2 ? 128 : 0, base};
    return copy_tag(gu ? tempo::gen8::route_gate_up(to_pod(&p)) : tempo::gen8::route(to_pod(&p)),
                    tag, tag_len);
  }
  return copy_tag(nullptr, tag, tag_len);
}

}  // extern "C"
