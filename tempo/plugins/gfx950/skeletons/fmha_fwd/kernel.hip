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
//   * K and V blocks are copied global -> LDS with LDS-DMA (buffer_load_dwordx4 ... lds), no
//     register staging.  Both are stored in their natural [key][d] order with the 16-byte chunk index
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

// 16-byte-per-lane buffer load into LDS (MUBUF buffer_load ... lds): lane l's 16 bytes at byte
// offset voff of the raw buffer [base, base + nrec) land at lds + 16 l; reads past nrec return
// zeros.  The MUBUF form, not global_load_lds: the compiler counts a FLAT-encoded LDS copy on
// both counters and then waits for every LDS read with lgkmcnt(0).
__device__ __forceinline__ void fmha_buf_lds16(const void* base, unsigned nrec, void* lds,
                                               unsigned voff) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nrec, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (fmha_lds_void_t*)lds, 16, (int)voff, 0, 0, 0);
}

// ============================================================================================
// k_fmha_fwd -- software-pipelined over 32-key blocks, laid out for one wave per SIMD (the 128 O
// accumulators, Q and the fragments take ~440 registers), where nothing but the wave's own
// instruction order hides a latency.
//
// Iteration kb computes, on the matrix cores, S(kb+1) = K(kb+1).Q^T and O^T += V(kb-1)^T .
// P(kb-1)^T, while the VALU turns S(kb) into P(kb) (row max, exponentials, sums):
//   * the chain of iteration kb is cut into DS chunks fenced with sched_barrier; each chunk
//     holds one score MFMA, one P.V MFMA, the K fragment read KP chunks ahead, the transposed V
//     pair read VP chunks ahead, and one slice of the softmax of block kb (chunk 2: row max,
//     chunk 3: the exchange with lane ^ 32, the others: the exponentials against the running
//     reference, computed speculatively and pinned into their chunk), so the exponentials run
//     in the matrix pipe's shadow;
//   * P(kb) lives in registers until the next iteration consumes it (two P sets, alternating;
//     the scores likewise), so the P.V product of a block runs one iteration after its
//     softmax, interleaved with the next block's scores;
//   * after the chain, the rare move of the reference (ballot): O and l rescaled in place in
//     the accumulator registers -- O then holds P(0..kb-1).V, all relative to the old reference
//     -- and the exponentials of block kb redone against the new one; after the last block
//     one more P.V step (the last block's) runs on its own.
//
// K and V travel by LDS-DMA two blocks at a time, two blocks ahead.  Each operand has four
// block slots (two pairs); K blocks are paired as (2c+1, 2c+2), V blocks as (2c-1, 2c), so both
// pairs held by one slot pair are read by the same two iterations (2c, 2c+1) and are free after
// the second.  Every EVEN iteration kb starts with one wait (this wave's copies, issued two
// iterations earlier, have landed) and one workgroup barrier (everyone's have, and every wave
// is done with the slots about to be refilled), then copies K(kb+3), K(kb+4) and V(kb+1),
// V(kb+2) into the slots the previous two iterations read; odd iterations neither wait nor
// synchronise.  Block j of K lives in slot (j - 1) % 4, block j of V in slot (j + 1) % 4, so
// iteration kb reads slot kb % 4 of both.  One LDS array per slot and a four-iteration loop
// body make every slot a compile-time choice: the compiler's LDS alias scopes then keep the
// reads of one slot from waiting for the copies in flight into another (with one shared array
// every read waited for all outstanding copies).  The four-body loop is written as a counted
// for-loop with a phased tail: a while-loop with a break after every body made the register
// allocator spill Q and the accumulators.
//
// Every sum is taken in a fixed order (the row max and sums, then P.V by key block and, within
// a block, k-step 0 then 1), so results do not depend on the schedule.
// ============================================================================================
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void k_fmha_fwd(
    const _Float16* __restrict__ Q, const _Float16* __restrict__ Kg,
    const _Float16* __restrict__ Vg, _Float16* __restrict__ O, float* __restrict__ LSE, int B,
    int H, int Hkv, int Sq, int Sk, float scale_log2, long q_sb, long q_ss, long q_sh, long k_sb,
    long k_ss, long k_sh, long v_sb, long v_ss, long v_sh, long o_sb, long o_ss, long o_sh) {
  static_assert(D == 128 || D == 256, "head dim 128 or 256");
  constexpr int BKV2 = 32;
  constexpr int WAVES = 4;
  constexpr int DCH = D / 8;
  constexpr int DS = D / 16;   // score MFMAs (k = 16 each) per key block = chunks
  constexpr int DB = D / 32;   // 32-wide d blocks of O
  constexpr int RB = D * 2;
  constexpr int ROWS_PER_KB = 1024 / RB;
  constexpr int BLK = BKV2 / ROWS_PER_KB;
  constexpr int BLK_W = BLK / WAVES;
  constexpr int BQW = 32 * WAVES;
  constexpr int TILE_B = BKV2 * RB;
  constexpr int KP = 4;        // K fragment reads ahead of the chain
  constexpr int VP = 2;        // V pair reads ahead of their P.V MFMA
  constexpr int NX = DS - 4;   // chunks carrying exponentials (chunks 2-3: max, exchange)
  static_assert(DS >= 8 && 2 * DB == DS, "one V pair per chunk");
  static_assert(BLK % WAVES == 0, "DMA blocks split over the waves");

  __shared__ __attribute__((aligned(1024))) char k0s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char k1s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char k2s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char k3s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char v0s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char v1s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char v2s[TILE_B];
  __shared__ __attribute__((aligned(1024))) char v3s[TILE_B];

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
  // block j of one operand into the slot array dst; rows past Sk re-read row Sk-1.  The buffer
  // starts at the block's first row and ends with row Sk-1 (every offset below is inside it;
  // capped at 2^32 - 1: every offset used is below 32 rows x ss x 2 < 2^31).
  auto copy_block = [&](const char* base, long ss, const unsigned* src, char* dst, int j) {
    const int j0 = j * BKV2;
    const char* blk = base + (long)j0 * ss * 2;
    const long span = (long)(Sk - 1 - j0) * ss * 2 + D * 2;
    const unsigned nrec = span < 0xFFFFFFFFL ? (unsigned)span : 0xFFFFFFFFu;
    if (j0 + BKV2 <= Sk) {
#pragma unroll
      for (int i = 0; i < BLK_W; ++i)
        fmha_buf_lds16(blk, nrec, dst + (i * WAVES + wave) * 1024, src[i]);
    } else {
#pragma unroll
      for (int i = 0; i < BLK_W; ++i) {
        const unsigned back = (unsigned)max(0, j0 + drow[i] - (Sk - 1));
        fmha_buf_lds16(blk, nrec, dst + (i * WAVES + wave) * 1024,
                       src[i] - back * (unsigned)(ss * 2));
      }
    }
  };
  auto kslot = [&](auto sl) -> char* {
    constexpr int S4 = decltype(sl)::value % 4;
    if constexpr (S4 == 0) return k0s;
    else if constexpr (S4 == 1) return k1s;
    else if constexpr (S4 == 2) return k2s;
    else return k3s;
  };
  auto vslot = [&](auto sl) -> char* {
    constexpr int S4 = decltype(sl)::value % 4;
    if constexpr (S4 == 0) return v0s;
    else if constexpr (S4 == 1) return v1s;
    else if constexpr (S4 == 2) return v2s;
    else return v3s;
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
  // V pair i of a slot: P.V k-step i / DB, d block i % DB
  auto vread = [&](const char* vr, int i) -> f16x8 {
    const int tt = i / DB, db = i % DB;
    const u32x2 a = fmha_tr_read(vr + voff0[db & 3] + 16 * tt * RB + (db >> 2) * 256);
    const u32x2 c = fmha_tr_read(vr + voff1[db & 3] + 16 * tt * RB + (db >> 2) * 256);
    const u32x4 vv = {a[0], a[1], c[0], c[1]};
    return as_f16x8(vv);
  };

  f32x16 acc_o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc_o[i][v] = 0.f;
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  auto sync_top = [&]() {
    asm volatile("" ::: "memory");
    fmha_wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto exps = [&](const f32x16& s, float m_use, f16x8 (&pt)[2], float& psum, int e0, int e1) {
#pragma unroll
    for (int e = e0; e < e1; ++e) {
      const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], scale_log2, -m_use));
      psum = e == 0 ? pv : psum + pv;
      pt[e >> 3][e & 7] = (_Float16)pv;
    }
  };

  f32x16 sa, sb;
  f16x8 pa[2], pb[2];
  if (nkb > 0) {
    // K(0) -> slot 3, K(1), K(2) -> slots 0, 1; V(0) -> slot 1
    copy_block(Kp, k_ss, ksrc, k3s, 0);
    if (nkb > 1) copy_block(Kp, k_ss, ksrc, k0s, 1);
    if (nkb > 2) copy_block(Kp, k_ss, ksrc, k1s, 2);
    copy_block(Vp, v_ss, vsrc, v1s, 0);
    sync_top();
#pragma unroll
    for (int r = 0; r < 16; ++r) sa[r] = 0.f;
#pragma unroll
    for (int st = 0; st < DS; ++st) {
      const f16x8 kf = *reinterpret_cast<const f16x8*>(k3s + koff[st & 7] + (st >> 3) * 256);
      sa = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], sa, 0, 0, 0);
    }
  }
  // iteration kb (phase T = kb % 4; FIRST: kb = 0): K(kb+1) and V(kb-1) are resident in slot
  // T; an even iteration first waits for its copies of two iterations ago and synchronises,
  // then copies K(kb+3), K(kb+4) -> slots T+2, T+3 and V(kb+1), V(kb+2) -> slots T+2, T+3;
  // S(kb+1) = K(kb+1).Q^T || O += V(kb-1)^T . P(kb-1)^T (ppv) || softmax of S(kb) -> P(kb)
  // (pcur).  The scores of a block past the end read a stale slot and are never used.
  auto iter = [&](auto phase, auto first, f32x16& cur, f32x16& nxt, const f16x8 (&ppv)[2],
                   f16x8 (&pcur)[2], int kb) {
    constexpr int T = decltype(phase)::value;
    constexpr bool FIRST = decltype(first)::value;
    if constexpr (T % 2 == 0) {
      sync_top();
      if (kb + 3 < nkb) copy_block(Kp, k_ss, ksrc, kslot(IC<T + 2>{}), kb + 3);
      if (kb + 4 < nkb) copy_block(Kp, k_ss, ksrc, kslot(IC<T + 3>{}), kb + 4);
      if (kb + 1 < nkb) copy_block(Vp, v_ss, vsrc, vslot(IC<T + 2>{}), kb + 1);
      if (kb + 2 < nkb) copy_block(Vp, v_ss, vsrc, vslot(IC<T + 3>{}), kb + 2);
    }
    const char* const kr = kslot(IC<T>{});
    const char* const vr = vslot(IC<T>{});
    const int j0 = kb * BKV2;
    if ((j0 + BKV2 > Sk) || (CAUSAL && j0 + BKV2 - 1 > q0 + off)) {
      const int lim = (CAUSAL ? min(Sk - 1, qi + off) : Sk - 1) - j0 - 4 * hl;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        cur[r] = (8 * (r >> 2) + (r & 3)) > lim ? -__builtin_inff() : cur[r];
    }
    const float m_use0 = (m_run == -__builtin_inff()) ? 0.f : m_run;
    f16x8 kf[DS];
    f16x8 vf[DS];
    float mx = -__builtin_inff(), mxs = 0.f, psum;
#pragma unroll
    for (int st = 0; st < KP; ++st)
      kf[st] = *reinterpret_cast<const f16x8*>(kr + koff[st & 7] + (st >> 3) * 256);
    if constexpr (!FIRST) {
#pragma unroll
      for (int i = 0; i < VP; ++i) vf[i] = vread(vr, i);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) nxt[r] = 0.f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < DS; ++c) {
      nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], nxt, 0, 0, 0);
      if constexpr (!FIRST)
        acc_o[c % DB] =
            __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[c], ppv[c / DB], acc_o[c % DB], 0, 0, 0);
      if (c + KP < DS)
        kf[c + KP] =
            *reinterpret_cast<const f16x8*>(kr + koff[(c + KP) & 7] + ((c + KP) >> 3) * 256);
      if constexpr (!FIRST) {
        if (c + VP < DS) vf[c + VP] = vread(vr, c + VP);
      }
      if (c == 2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, cur[r]);
      } else if (c == 3) {
        mxs = fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;
      } else {
        exps(cur, m_use0, pcur, psum, 16 * (c - 4) / NX, 16 * (c - 3) / NX);
        asm volatile("" : "+v"(psum), "+v"(pcur[0]), "+v"(pcur[1]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (__builtin_amdgcn_ballot_w64(!(mxs - m_run <= FMHA_TAU)) != 0) {
      const float m_new = fmaxf(m_run, mxs);
      const float alpha =
          (m_new == -__builtin_inff()) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      // the chain's last P.V MFMAs write O: wait states before the accumulators are read
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = acc_o[i][r], tmp;
          asm volatile(
              "v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
              : "+a"(x), "=&v"(tmp)
              : "v"(alpha));
          acc_o[i][r] = x;
        }
      exps(cur, (m_run == -__builtin_inff()) ? 0.f : m_run, pcur, psum, 0, 16);
    }
    l_run += psum + __shfl_xor(psum, 32);
  };
  // the P.V step of the last block (V(nkb-1) in slot nkb % 4)
  auto pv_last = [&](const f16x8 (&pl)[2]) {
    sync_top();
    const int t4 = nkb & 3;
    const char* const vr = t4 == 0 ? v0s : t4 == 1 ? v1s : t4 == 2 ? v2s : v3s;
#pragma unroll
    for (int i = 0; i < DS; ++i)
      acc_o[i % DB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vread(vr, i), pl[i / DB],
                                                             acc_o[i % DB], 0, 0, 0);
  };
  if (nkb > 0) {
    iter(IC<0>{}, IC<1>{}, sa, sb, pb, pa, 0);
    int kb = 1;
    for (; kb + 3 < nkb; kb += 4) {
      iter(IC<1>{}, IC<0>{}, sb, sa, pa, pb, kb);
      iter(IC<2>{}, IC<0>{}, sa, sb, pb, pa, kb + 1);
      iter(IC<3>{}, IC<0>{}, sb, sa, pa, pb, kb + 2);
      iter(IC<0>{}, IC<0>{}, sa, sb, pb, pa, kb + 3);
    }
    // the last 0-3 blocks continue the phase sequence 1, 2, 3
    if (kb < nkb) {
      iter(IC<1>{}, IC<0>{}, sb, sa, pa, pb, kb);
      if (kb + 1 < nkb) {
        iter(IC<2>{}, IC<0>{}, sa, sb, pb, pa, kb + 1);
        if (kb + 2 < nkb) iter(IC<3>{}, IC<0>{}, sb, sa, pa, pb, kb + 2);
      }
    }
    if (nkb & 1) pv_last(pa);
    else pv_last(pb);
  }

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
