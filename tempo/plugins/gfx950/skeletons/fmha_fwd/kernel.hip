// fmha_fwd -- causal / full attention forward for gfx950: O = softmax(scale Q K^T + mask) V.
//
// Semantics (reference, profiled/fwd_ws/fa2_sm70/csrc): bottom-right causal mask, key j visible
// to query i iff j <= i + (Sk - Sq) (attn_fwd_cutlass.cu:137, volta_fwd_ws.cuh:863); GQA maps
// query head h to KV head h / (H / Hkv) (attn_fwd_cutlass.cu:193, volta_fwd_ws.cuh:432); the
// softmax runs in base 2 with scale*log2(e) folded into the scores (attn_fwd_cutlass.cu:660-666)
// and LSE is returned in natural-log units, m*ln2 + ln(l) (volta_fwd_ws.cuh:1063).  fp32 scores,
// fp32 running max/sum, fp16 P and O, fp32 accumulation of P.V.
//
// Mapping onto CDNA4 (one workgroup = 4 waves = BQ = 128 query rows of one (b, h); each wave owns
// 32 rows; key/value blocks of BKV = 64):
//   * S^T = K . Q^T on v_mfma_f32_32x32x16_f16: K rows are the "A" operand, Q rows the "B"
//     operand, so every lane's result registers belong to ONE query row (column = lane % 32) --
//     row max and row sum are in-lane plus one exchange with lane ^ 32.  Q stays in registers
//     for the whole key loop (16 fragments of 8 halves).
//   * O^T = V^T . P^T: P^T is the "B" operand and is taken straight from the S^T accumulators
//     (lane l, k-group l/32 holds exactly the 8 key indices that operand slot needs), so P never
//     touches LDS.  O^T's column is again the query row, so the online-softmax rescale is one
//     per-lane factor for all 128 accumulator registers.
//   * V is staged into LDS as [j/4][d][4] (four consecutive keys of one d contiguous), so the
//     V^T operand (8 keys of one d) is two 8-byte LDS reads; K is staged [j][d] with the 16-byte
//     chunk index XOR-swizzled by row.  Both are double-buffered, register-staged from global.
//   * Causal work is triangular: workgroups are issued heaviest query block first.

namespace fmha {

constexpr int BQ = 128;
constexpr int BKV = 64;
constexpr int WAVES = 4;

template <int DCH>
__device__ __forceinline__ int kswz(int row, int chunk) { return chunk ^ (row & (DCH - 1)); }

template <int D>
struct Smem {
  static constexpr int K_ELEMS = BKV * D;  // [64][D]
  static constexpr int V_ELEMS = BKV * D;  // [16][D][4]
  static constexpr int BYTES = 2 * (K_ELEMS + V_ELEMS) * 2;
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void k_fmha_fwd(
    const _Float16* __restrict__ Q, const _Float16* __restrict__ Kg,
    const _Float16* __restrict__ Vg, _Float16* __restrict__ O, float* __restrict__ LSE, int H,
    int Hkv, int Sq, int Sk, float scale_log2, long q_sb, long q_ss, long q_sh, long k_sb,
    long k_ss, long k_sh, long v_sb, long v_ss, long v_sh, long o_sb, long o_ss, long o_sh) {
  static_assert(D == 128 || D == 256, "head dim 128 or 256");
  constexpr int DCH = D / 8;     // 16-byte chunks per K row
  constexpr int DS = D / 16;     // MFMA k-steps over d
  constexpr int DB = D / 32;     // 32-wide d blocks of O^T
  constexpr int K_IT = BKV * DCH / 256;             // K chunks per thread per block
  constexpr int V_IT = (BKV / 4) * (D / 8) / 256;   // V 4x8 sub-blocks per thread per block

  __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (Smem<D>::K_ELEMS + Smem<D>::V_ELEMS)];
  _Float16* const sK = smem;                                  // [2][64][D] swizzled
  _Float16* const sV = smem + 2 * Smem<D>::K_ELEMS;           // [2][16][D][4]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5;      // k-group / half of the wave
  const int l32 = lane & 31;

  // heaviest query block first (causal work grows with the block index)
  const int nqb = (Sq + BQ - 1) / BQ;
  const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hkv);
  const long off = (long)Sk - Sq;
  const int q0 = qb * BQ;
  const int qi = q0 + wave * 32 + l32;                    // this lane's query row
  const int qrow = min(qi, Sq - 1);

  const _Float16* Qp = Q + b * q_sb + (long)h * q_sh;
  const _Float16* Kp = Kg + b * k_sb + (long)hk * k_sh;
  const _Float16* Vp = Vg + b * v_sb + (long)hk * v_sh;

  // ---- Q fragments: lane supplies row qrow, d in [16s + 8*hl, +8) for s = 0..DS-1 -----------
  f16x8 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = *reinterpret_cast<const f16x8*>(Qp + (long)qrow * q_ss + 16 * s + 8 * hl);

  // ---- key range ---------------------------------------------------------------------------
  long kend = Sk;
  if (CAUSAL) {
    const long last = (long)min(q0 + BQ, Sq) - 1 + off;  // last key any row of the block sees
    kend = last + 1 < Sk ? last + 1 : Sk;
    if (kend < 0) kend = 0;
  }
  const int nkb = (int)((kend + BKV - 1) / BKV);

  // ---- staging registers -------------------------------------------------------------------
  u32x4 rk[K_IT];
  u32x4 rv[V_IT][4];
  auto load_kv = [&](int kb) {
    const int j0 = kb * BKV;
#pragma unroll
    for (int i = 0; i < K_IT; ++i) {
      const int q = tid + i * 256, r = q / DCH, c = q % DCH;
      const int j = min(j0 + r, Sk - 1);
      rk[i] = *reinterpret_cast<const u32x4*>(Kp + (long)j * k_ss + c * 8);
    }
#pragma unroll
    for (int i = 0; i < V_IT; ++i) {
      const int q = tid + i * 256, jq = q / (D / 8), dg = q % (D / 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = min(j0 + 4 * jq + e, Sk - 1);
        rv[i][e] = *reinterpret_cast<const u32x4*>(Vp + (long)j * v_ss + dg * 8);
      }
    }
  };
  auto store_kv = [&](int buf) {
    _Float16* k = sK + buf * Smem<D>::K_ELEMS;
    _Float16* v = sV + buf * Smem<D>::V_ELEMS;
#pragma unroll
    for (int i = 0; i < K_IT; ++i) {
      const int q = tid + i * 256, r = q / DCH, c = q % DCH;
      *reinterpret_cast<u32x4*>(k + r * D + kswz<DCH>(r, c) * 8) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < V_IT; ++i) {
      const int q = tid + i * 256, jq = q / (D / 8), dg = q % (D / 8);
      // transpose 4 keys x 8 d (4 rows of 4 dwords) into 8 d x 4 keys (8 runs of 8 bytes)
      u32x4 o[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // dword w holds d = 2w, 2w+1 of each key row
        const uint32_t a0 = rv[i][0][w], a1 = rv[i][1][w], a2 = rv[i][2][w], a3 = rv[i][3][w];
        // d = 2w   : keys 0..3 low halves ; d = 2w+1 : keys 0..3 high halves
        const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
        o[w] = u32x4{lo01, lo23, hi01, hi23};
      }
      u32x4* dst = reinterpret_cast<u32x4*>(v + ((long)jq * D + dg * 8) * 4);
#pragma unroll
      for (int w = 0; w < 4; ++w) dst[w] = o[w];
    }
  };

  f32x16 acc_o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc_o[i][v] = 0.f;
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  if (nkb > 0) {
    load_kv(0);
    store_kv(0);
  }
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load_kv(kb + 1);
    const _Float16* k = sK + cur * Smem<D>::K_ELEMS;
    const _Float16* v = sV + cur * Smem<D>::V_ELEMS;
    const int j0 = kb * BKV;

    // S^T for two 32-key blocks: lane holds keys j0 + 32*jb + 8g + 4*hl + e (reg 4g+e) of row qi
    f32x16 s[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[jb][r] = 0.f;
      const int kr = jb * 32 + l32;
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const f16x8 kf =
            *reinterpret_cast<const f16x8*>(k + kr * D + kswz<DCH>(kr, 2 * st + hl) * 8);
        s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], s[jb], 0, 0, 0);
      }
    }

    // scale, mask, block row max
    const bool need_mask = (j0 + BKV > Sk) || (CAUSAL && (long)(j0 + BKV - 1) > (long)q0 + off);
    float mx = -__builtin_inff();
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[jb][r] * scale_log2;
        if (need_mask) {
          const int j = j0 + jb * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
          const bool hide = (j >= Sk) || (CAUSAL && (long)j > (long)qi + off);
          x = hide ? -__builtin_inff() : x;
        }
        s[jb][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
    f16x8 pf[4];  // P^T operand fragments for the four 16-key MFMA steps
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[jb][r] - m_use);
        psum += p;
        pf[jb * 2 + (r >> 3)][r & 7] = (_Float16)p;
      }
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[i][r] *= alpha;

    // O^T += V^T . P^T over the 64 keys of this block (4 MFMA k-steps of 16 keys)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // keys of step t for k-group hl: 32*(t/2) + 16*(t%2) + 8*(e/4) + 4*hl + e%4
      const int jq0 = 8 * (t >> 1) + 4 * (t & 1) + hl;  // j/4 of elements 0..3
      const int jq1 = jq0 + 2;                          // j/4 of elements 4..7
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = db * 32 + l32;
        const u32x2 v0 = *reinterpret_cast<const u32x2*>(v + ((long)jq0 * D + d) * 4);
        const u32x2 v1 = *reinterpret_cast<const u32x2*>(v + ((long)jq1 * D + d) * 4);
        const u32x4 vv = {v0[0], v0[1], v1[0], v1[1]};
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(vv), pf[t], acc_o[db], 0, 0, 0);
      }
    }

    if (kb + 1 < nkb) store_kv(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[qi][d] = acc / l; lane holds d = db*32 + 8g + 4*hl + e ----------------------
  if (qi < Sq) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    _Float16* Op = O + b * o_sb + (long)qi * o_ss + (long)h * o_sh;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 o;
        o[0] = (_Float16)(acc_o[db][4 * g + 0] * inv);
        o[1] = (_Float16)(acc_o[db][4 * g + 1] * inv);
        o[2] = (_Float16)(acc_o[db][4 * g + 2] * inv);
        o[3] = (_Float16)(acc_o[db][4 * g + 3] * inv);
        *reinterpret_cast<f16x4*>(Op + db * 32 + 8 * g + 4 * hl) = o;
      }
    if (LSE && hl == 0)
      LSE[((long)b * H + h) * Sq + qi] =
          l_run > 0.f ? m_run * 0.6931471805599453f + __logf(l_run) : -__builtin_inff();
  }
}

}  // namespace fmha
