// launch_prefill.hip -- the second translation unit of the shipped gemm_w8a16 for gfx950: the
// interleaved int8 prefill kernel k_gemm_ilv8 and its launchers, instantiated for the ladder rows
// listed in prefill.inc (generated from select.py next to dispatch.inc).
//
// It is a TU of its own because it is built with the register-pressure-minimising pre-RA
// scheduler, which keeps each of the kernel's 256 accumulator tuples in one AGPR range; the
// other kernels of the delivery keep the default scheduler.
//
// Build (host tree): hipcc -O3 -std=c++17 --offload-arch=gfx950
//                    -Xclang -target-feature -Xclang -packed-fp32-ops
//                    -mllvm -amdgpu-sched-strategy=iterative-minreg -c launch_prefill.hip
// The flags line below is read by the library build (cuda_tempiler_amd/build.py):
// tempo:flags -mllvm -amdgpu-sched-strategy=iterative-minreg
#include "launch.h"

namespace tempo {
namespace gen8 {

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP>
hipError_t launch_ilv8(const W8A16Params& p, hipStream_t s) {
  const int nm = (p.M + BM - 1) / BM;
  const int nn = p.N / BN;
  const dim3 grid(nm * nn), blk(WM * WN * 64);
  if (p.fmt == 1)
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 1>), grid, blk, 0,
                       s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C, p.M, p.N,
                       p.K, p.lda, p.ldw, p.ldc);
  else
    hipLaunchKernelGGL((k_gemm_ilv8<BM, BN, BK, WM, WN, STAGES, GROUP, XCD, RSP, 2>), grid, blk, 0,
                       s, p.A, static_cast<const uint8_t*>(p.Wq), p.scale, p.zero, p.C, p.M, p.N,
                       p.K, p.lda, p.ldw, p.ldc);
  return hipGetLastError();
}

#include "prefill.inc"

}  // namespace gen8
}  // namespace tempo
