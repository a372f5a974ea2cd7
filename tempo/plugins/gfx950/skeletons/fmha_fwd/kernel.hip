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
// 32 rows; key/value blocks of BKV2 keys):
//   * S^T = K . Q^T on v_mfma_f32_32x32x16_f16: K rows are the "A" operand, Q rows the "B"
//     operand, so every lane's result registers belong to ONE query row (column = lane % 32) --
//     row max and row sum are in-lane plus one exchange with lane ^ 32.  Q stays in registers
//     for the whole key loop (D/16 fragments of 8 halves).
//   * O^T = V^T . P^T: P^T is the "B" operand and is taken straight from the S^T accumulators
//     (lane l, k-group l/32 holds exactly the 8 key indices that operand slot needs), so P never
//     touches LDS.  O^T's column is again the query row, so the online-softmax rescale is one
//     per-lane factor for all accumulator registers.
//   * K and V blocks are copied global -> LDS with LDS-DMA (global_load_lds_dwordx4), no register
//     staging.  Both are stored in their natural [key][d] order with the 16-byte chunk index
//     XOR-ed by fmha_swz(key % 16), a bit swap of the 4-bit row index chosen so that both read
//     patterns are free of bank conflicts on the 64-bank LDS: the K read (16 rows, one chunk) and
//     the transposed V read (4 rows x 4 consecutive chunks) each land on 16 distinct 16-byte
//     slots of a 256-byte bank window.  The swizzle is applied on the global side (lane l of a
//     DMA instruction writes bytes [16l, 16l+16) of a 1 KiB block and fetches the chunk that
//     belongs there).
//   * The V^T operand (8 keys of one d per lane) is read with ds_read_b64_tr_b16: within each
//     group of 16 lanes, lane j supplies the address of 4 consecutive d of key row (base + j/4),
//     and lane i receives, for e = 0..3, element i%4 of the row supplied by lane 4e + i/4 --
//     i.e. key base+e at d = d0 + i.  Two such reads give the 8 keys of one MFMA k-group.
//   * Rescale threshold: the running max used for the exponentials only moves when some lane's
//     block max exceeds it by more than FMHA_TAU (base-2 units).  Any reference value gives the
//     same softmax (the numerator and l use the same one), exp2 arguments stay <= TAU, and the O
//     rescale is almost never paid.
//   * Causal work is triangular: workgroups are numbered heaviest query block first over ALL
//     heads and batches.

namespace fmha {

constexpr int BQ = 128;  // query rows per workgroup (4 waves x 32)

typedef __attribute__((address_space(3))) void fmha_lds_void_t;
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fmha_h4;
typedef __attribute__((address_space(3))) fmha_h4 fmha_lds_h4;

template <int N>
__device__ __forceinline__ void fmha_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

__device__ __forceinline__ u32x2 fmha_tr_read(const char* p) {
  const fmha_h4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      (fmha_lds_h4*)((__attribute__((address_space(3))) const char*)(p)));
  return __builtin_bit_cast(u32x2, v);
}

constexpr float FMHA_TAU = 8.f;  // log2 of the largest unnormalised probability allowed

// swizzle key of a key row (only its low 4 bits matter): swap the two 2-bit halves
__device__ __forceinline__ int fmha_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// ============================================================================================
// k_fmha_fwd3 -- software-pipelined: the score MFMAs of the NEXT key block overlap the softmax
// of the current one.  Iteration kb computes S(kb+1) = K(kb+1).Q^T on the matrix cores while the
// VALU turns S(kb) into P(kb) (max, exponentials, sums), then O^T += V(kb)^T . P(kb)^T.  K runs
// one block ahead of V: K(kb+2) and V(kb+1) are copied during iteration kb into the slots that
// K(kb) and V(kb-1) left, so the LDS footprint is two K and two V blocks.
// ============================================================================================
// SG = 1 adds sched_group_barrier hints that interleave MFMAs with LDS reads and VALU work
// (measured slower at C5; the shipped instantiation has SG = 0).
template <int D, bool CAUSAL, int BKV2, int SG = 0>
__global__ __launch_bounds__(256, 1) void k_fmha_fwd3(
    const _Float16* __restrict__ Q, const _Float16* __restrict__ Kg,
    const _Float16* __restrict__ Vg, _Float16* __restrict__ O, float* __restrict__ LSE, int B,
    int H, int Hkv, int Sq, int Sk, float scale_log2, long q_sb, long q_ss, long q_sh, long k_sb,
    long k_ss, long k_sh, long v_sb, long v_ss, long v_sh, long o_sb, long o_ss, long o_sh) {
  static_assert(D == 128 || D == 256, "head dim 128 or 256");
  static_assert(BKV2 == 32 || BKV2 == 64, "key block 32 or 64");
  constexpr int WAVES = 4;
  constexpr int NJ = BKV2 / 32;
  constexpr int DCH = D / 8;
  constexpr int DS = D / 16;
  constexpr int DB = D / 32;
  constexpr int RB = D * 2;
  constexpr int ROWS_PER_KB = 1024 / RB;
  constexpr int BLK = BKV2 / ROWS_PER_KB;
  constexpr int BLK_W = BLK / WAVES;
  constexpr int BQW = 32 * WAVES;
  constexpr int TILE_B = BKV2 * RB;
  static_assert(BLK % WAVES == 0, "DMA blocks split over the waves");

  __shared__ __attribute__((aligned(1024))) char smem[4 * TILE_B];  // K[2] then V[2]
  char* const kbuf = smem;
  char* const vbuf = smem + 2 * TILE_B;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  const int nqb = (Sq + BQW - 1) / BQW;
  const int bid = blockIdx.x;
  const int per_qb = H * B;
  const int qb = CAUSAL ? (nqb - 1 - bid / per_qb) : bid / per_qb;
  const int hb = bid % per_qb;
  const int h = hb % H, b = hb / H;
  const int hk = h / (H / Hkv);
  const int off = Sk - Sq;
  const int q0 = qb * BQW;
  const int qi = q0 + wave * 32 + l32;
  const int qrow = min(qi, Sq - 1);

  const _Float16* Qp = Q + b * q_sb + (long)h * q_sh;
  const char* Kp = reinterpret_cast<const char*>(Kg + b * k_sb + (long)hk * k_sh);
  const char* Vp = reinterpret_cast<const char*>(Vg + b * v_sb + (long)hk * v_sh);

  f16x8 qf[DS];
#pragma unroll
  for (int st = 0; st < DS; ++st)
    qf[st] = *reinterpret_cast<const f16x8*>(Qp + (long)qrow * q_ss + 16 * st + 8 * hl);

  int kend = Sk;
  if (CAUSAL) {
    const int last = min(q0 + BQW, Sq) - 1 + off;
    kend = last + 1 < Sk ? last + 1 : Sk;
    if (kend < 0) kend = 0;
  }
  const int nkb = (kend + BKV2 - 1) / BKV2;

  const int rin = lane / DCH, phys = lane % DCH;
  unsigned ksrc[BLK_W], vsrc[BLK_W];
  int drow[BLK_W];
#pragma unroll
  for (int i = 0; i < BLK_W; ++i) {
    const int r = (i * WAVES + wave) * ROWS_PER_KB + rin;
    const int c = phys ^ fmha_swz(r);
    drow[i] = r;
    ksrc[i] = (unsigned)(r * k_ss * 2 + c * 16);
    vsrc[i] = (unsigned)(r * v_ss * 2 + c * 16);
  }
  // one operand block j (K or V) -> its slot j & 1; rows past Sk re-read row Sk-1
  auto copy_block = [&](const char* base, long ss, const unsigned* src, char* slots, int j) {
    char* dst = slots + (j & 1) * TILE_B;
    const int j0 = j * BKV2;
    const char* blk = base + (long)j0 * ss * 2;
    if (j0 + BKV2 <= Sk) {
#pragma unroll
      for (int i = 0; i < BLK_W; ++i)
        __builtin_amdgcn_global_load_lds((void*)(blk + src[i]),
                                         (fmha_lds_void_t*)(dst + (i * WAVES + wave) * 1024), 16,
                                         0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < BLK_W; ++i) {
        const long back = (long)max(0, j0 + drow[i] - (Sk - 1));
        __builtin_amdgcn_global_load_lds((void*)(blk + src[i] - back * ss * 2),
                                         (fmha_lds_void_t*)(dst + (i * WAVES + wave) * 1024), 16,
                                         0, 0);
      }
    }
  };

  const int kkey = fmha_swz(l32);
  int koff[8];
#pragma unroll
  for (int s7 = 0; s7 < 8; ++s7) koff[s7] = l32 * RB + (((2 * s7) | hl) ^ kkey) * 16;
  const int tg = lane >> 4, tj = lane & 15;
  const int tk = 4 * (tg >> 1) + (tj >> 2);
  const int cd = 2 * (tg & 1) + ((tj & 3) >> 1);
  const int half = 8 * (tj & 1);
  int voff0[4], voff1[4];
#pragma unroll
  for (int p4 = 0; p4 < 4; ++p4) {
    voff0[p4] = tk * RB + (((p4 << 2) | cd) ^ fmha_swz(tk)) * 16 + half;
    voff1[p4] = (tk + 8) * RB + (((p4 << 2) | cd) ^ fmha_swz(tk + 8)) * 16 + half;
  }

  f32x16 acc_o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc_o[i][v] = 0.f;
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  // S^T of block j from K slot j & 1 into s (NJ 32-key blocks)
  auto scores = [&](f32x16* s, int j) {
    const char* k = kbuf + (j & 1) * TILE_B;
#pragma unroll
    for (int jb = 0; jb < NJ; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[jb][r] = 0.f;
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const f16x8 kf = *reinterpret_cast<const f16x8*>(k + koff[st & 7] + (st >> 3) * 256 +
                                                         jb * 32 * RB);
        s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], s[jb], 0, 0, 0);
      }
    }
  };
  // softmax, part 1: masked row max of block j (scale > 0 commutes with the max)
  auto softmax_max = [&](f32x16* s, int j) {
    const int j0 = j * BKV2;
    const bool need_mask = (j0 + BKV2 > Sk) || (CAUSAL && j0 + BKV2 - 1 > q0 + off);
    float mx = -__builtin_inff();
#pragma unroll
    for (int jb = 0; jb < NJ; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[jb][r];
        if (need_mask) {
          const int jj = j0 + 32 * jb + 8 * (r >> 2) + 4 * hl + (r & 3);
          const bool hide = (jj >= Sk) || (CAUSAL && jj > qi + off);
          x = hide ? -__builtin_inff() : x;
        }
        s[jb][r] = x;
        mx = fmaxf(mx, x);
      }
    return fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;
  };
  // the (rare) move of the reference value, with the O rescale it implies
  auto move_ref = [&](float mx) {
    const bool move = !(mx - m_run <= FMHA_TAU);
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha =
          (m_new == -__builtin_inff()) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[i][r] *= alpha;
    }
  };
  // softmax, part 2 fused with O^T += V^T . P^T: the 8 probabilities of MFMA k-step t are made
  // right before the step's MFMAs, so the exponentials of step t+1 overlap the MFMAs of step t.
  // Step t, element e <-> key 32(t/2) + 16(t%2) + 8(e/4) + 4*hl + e%4 = S register 8(t%2) + e of
  // 32-key block t/2.
  auto exp_pv = [&](const f32x16* s, int j) {
    const char* v = vbuf + (j & 1) * TILE_B;
    const float m_use = (m_run == -__builtin_inff()) ? 0.f : m_run;
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 2 * NJ; ++t) {
      f16x8 pt;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pv = __builtin_amdgcn_exp2f(
            __builtin_fmaf(s[t >> 1][8 * (t & 1) + e], scale_log2, -m_use));
        psum += pv;
        pt[e] = (_Float16)pv;
      }
      const int rt = 32 * (t >> 1) + 16 * (t & 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 v0 = fmha_tr_read(v + voff0[db & 3] + rt * RB + (db >> 2) * 256);
        const u32x2 v1 = fmha_tr_read(v + voff1[db & 3] + rt * RB + (db >> 2) * 256);
        const u32x4 vv = {v0[0], v0[1], v1[0], v1[1]};
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(vv), pt, acc_o[db], 0, 0, 0);
      }
    }
    psum += __shfl_xor(psum, 32);
    l_run += psum;
  };
  auto sync_top = [&]() {
    asm volatile("" ::: "memory");
    fmha_wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  f32x16 sa[NJ], sb[NJ];
  if (nkb > 0) {
    copy_block(Kp, k_ss, ksrc, kbuf, 0);
    copy_block(Vp, v_ss, vsrc, vbuf, 0);
    if (nkb > 1) copy_block(Kp, k_ss, ksrc, kbuf, 1);
    sync_top();
    scores(sa, 0);
  }
  // iteration kb: K(kb+1), V(kb) resident; copy K(kb+2), V(kb+1); S(kb+1) || max(kb); exp + PV(kb).
  // The scores of a block past the end read a stale K slot and are never used (unconditional so
  // the MFMAs and the max share one scheduling region).
  auto iter = [&](f32x16* cur, f32x16* nxt, int kb) {
    sync_top();
    if (kb + 2 < nkb) copy_block(Kp, k_ss, ksrc, kbuf, kb + 2);
    if (kb + 1 < nkb) copy_block(Vp, v_ss, vsrc, vbuf, kb + 1);
    scores(nxt, kb + 1);
    const float mx = softmax_max(cur, kb);
    if constexpr (SG) {
#pragma unroll
      for (int i = 0; i < NJ * DS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x0002, 2, 0);  // VALU
      }
    }
    move_ref(mx);
    exp_pv(cur, kb);
    if constexpr (SG) {
#pragma unroll
      for (int i = 0; i < 2 * NJ * DB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x0100, 2, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x0002, 3, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x0400, 1, 0);  // transcendental
      }
    }
  };
  int kb = 0;
  for (; kb + 1 < nkb; kb += 2) {
    iter(sa, sb, kb);
    iter(sb, sa, kb + 1);
  }
  if (kb < nkb) iter(sa, sb, kb);

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
