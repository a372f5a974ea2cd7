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
#include "launch_prefill.h"

namespace tempo {
namespace gen8 {

#include "prefill.inc"

}  // namespace gen8
}  // namespace tempo
