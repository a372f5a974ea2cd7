// fmha.hip -- translation unit of the causal FMHA forward (kernel: the plugin skeleton
// tempo/plugins/gfx950/skeletons/fmha_fwd/kernel.hip, compiled here in its own namespace).
#include "fmha_api.h"

#include <stdint.h>

namespace tempo_fmha {
#include "common/cdna4.h"
#include "fmha_fwd/kernel.hip"

bool applicable(const TempoFmhaParams& p) {
  if (!p.Q || !p.K || !p.V || !p.O) return false;
  if (p.B <= 0 || p.H <= 0 || p.Hkv <= 0 || p.Sq <= 0 || p.Sk <= 0) return false;
  if (p.H % p.Hkv != 0) return false;
  if (p.D != 128 && p.D != 256) return false;
  // d contiguous with 16-byte aligned rows (strides in elements)
  const long s[] = {p.q_ss, p.q_sh, p.q_sb, p.k_ss, p.k_sh, p.k_sb,
                    p.v_ss, p.v_sh, p.v_sb, p.o_ss, p.o_sh, p.o_sb};
  for (long x : s)
    if (x % 8 != 0) return false;
  const uintptr_t ptrs[] = {(uintptr_t)p.Q, (uintptr_t)p.K, (uintptr_t)p.V, (uintptr_t)p.O};
  for (uintptr_t x : ptrs)
    if (x % 16 != 0) return false;
  if ((long)p.Sq * p.q_ss > (1L << 40)) return false;
  if ((long)((p.Sq + 127) / 128) * p.H * p.B >= (1L << 31)) return false;
  // key/value rows of one block are addressed with 32-bit byte offsets from the block's first row
  if (p.k_ss > (1L << 24) || p.v_ss > (1L << 24)) return false;
  return true;
}

template <int D, bool CAUSAL>
static hipError_t run(const TempoFmhaParams& p, hipStream_t s) {
  // one workgroup per (query block, head, batch); the kernel numbers them heaviest causal
  // query block first across all heads and batches
  const int nqb = (p.Sq + fmha::BQ - 1) / fmha::BQ;
  const dim3 grid((unsigned)nqb * p.H * p.B), blk(256);
  const float scale_log2 = p.scale * 1.4426950408889634f;
  hipLaunchKernelGGL((fmha::k_fmha_fwd<D, CAUSAL>), grid, blk, 0, s,
                     static_cast<const _Float16*>(p.Q), static_cast<const _Float16*>(p.K),
                     static_cast<const _Float16*>(p.V), static_cast<_Float16*>(p.O), p.LSE, p.B,
                     p.H, p.Hkv, p.Sq, p.Sk, scale_log2, p.q_sb, p.q_ss, p.q_sh, p.k_sb, p.k_ss,
                     p.k_sh, p.v_sb, p.v_ss, p.v_sh, p.o_sb, p.o_ss, p.o_sh);
  return hipGetLastError();
}

hipError_t launch(const TempoFmhaParams& p, hipStream_t s) {
  if (!applicable(p)) return hipErrorInvalidConfiguration;
  if (p.D == 256) return p.causal ? run<256, true>(p, s) : run<256, false>(p, s);
  return p.causal ? run<128, true>(p, s) : run<128, false>(p, s);
}
}  // namespace tempo_fmha
