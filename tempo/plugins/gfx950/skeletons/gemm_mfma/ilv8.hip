// gemm_mfma/ilv8.hip -- the interleaved prefill GEMM with int8 / uint8 weights (W8A16):
// C = A . deq(W)^T.  Uses the tile machinery of gemm_mfma/kernel.hip (lds_chunk, tile_of,
// s_wait_vm, buf_lds16, buf_lds_n) and the dequantisation of common/cdna4.h.
// ============================================================================================
// k_gemm_ilv8 has the structure of k_gemm_ilv -- 4 waves (wave tiles of 128 x 128, 128 x 64 or
// 64 x 64) on v_mfma_f32_16x16x32_f16, chunked substeps fenced by sched_barrier, buffer LDS-DMA
// copies, the C tile written out through LDS -- with the weight tile travelling as bytes:
//   * A stage holds the fp16 A tile (BM x BK, SWZ2 chunk swizzle of its rows), the weight tile
//     (BN x BK bytes; 16-byte chunk c of row r stored at chunk c ^ wswz(r), wswz = (r / 4) % 4 for
//     64-byte rows and (r / 2) % 8 for 128-byte rows, which makes the 8-byte fragment reads below
//     conflict-free) and, fmt 2, the tile's zero-points and scales (one byte / one half per row,
//     4 bytes apart).  BK = 64: three stages (150 KiB) -- the weight tile is half the size of an
//     fp16 one, so a third stage fits.  BK = 128: every k-tile takes a whole 128-byte line of
//     each weight row, the granularity at which HBM streams near its peak (64-byte pieces of
//     scattered rows stream at about two thirds of the rate); two stages of 64 KiB at BM = 128,
//     BN = 256.  The C tile fits the stages for the epilogue.
//   * Fragments: A as in k_gemm_ilv (ds_read_b128); a weight fragment (16 rows x 32 k) is one
//     8-byte read per lane.  The MFMAs of a substep run block column by block column, and each
//     column's 8 weight bytes are dequantised in registers (cdna4.h dequant8: bit-exact
//     fp16_rn((q - z) s)) one chunk before its TM MFMAs -- so at most two dequantised fragments
//     are live, and the register budget (256 AGPR accumulators + 256 VGPRs) is not exceeded.
//   * fmt 1 (int8, per-channel scale): the wave's 8 row scales are copied into LDS once and held
//     in registers.  fmt 2 (uint8, group-128 zero-point and scale): every stage carries its tile's
//     metadata; the barrier substep of tile kt reads tile kt+1's into a second register set, which
//     becomes current once that substep's own MFMAs (still tile kt's) are issued.  The loop runs
//     one k-tile per iteration (unrolled further, the register allocator split the accumulator
//     chains).
// Requirements (the ladder's fit): N % BN == 0, K % 128 == 0, 16-byte aligned rows, panel byte
// offsets below 2^31.  M is predicated (A rows past M-1 clamped, never stored).
// SPLIT = 1 (split-K), as in k_gemm_ilv: workgroup split sk of split_tile_of takes k-tiles
// [sk*kper, ...), writes its fp32 partial tile to ws[sk][M][N]; k_splitk_reduce rounds the sum.
// A split may start at an odd k-tile: the scale group of k-tile t is t * BK / 128 in every
// stage.
// EPI = 1 (fused gate/up), as in k_gemm_ilv: W (and its scales and zero-points) hold the gate
// rows then, from row `up` on (the full output width), the up rows; a tile covers BN/2 output
// columns with BN/2 gate and the BN/2 matching up rows, and the epilogue writes
// fp16_rn(silu(g) * u) from the two halves of the C image.  (`up` may exceed N: a launch over
// some of the output columns, W and the metadata offset to its first gate row.)
// Build: -mllvm -amdgpu-sched-strategy=iterative-minreg, like k_gemm_ilv (own translation unit).
// ============================================================================================
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP, int BFMT,
          int SPLIT = 0, int EPI = 0>
__global__ __launch_bounds__(WM * WN * 64, 1) void k_gemm_ilv8(
    const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ scale,
    const uint8_t* __restrict__ zero, _Float16* __restrict__ C, int M, int N, int K, int lda,
    int ldw, int ldc, float* __restrict__ ws, int ksplit, int up) {
  using MF = Mfma<16>;
  constexpr int SWZ = 2;
  constexpr int NW = WM * WN;
  constexpr int CPR = BK / 8;                 // 16-byte chunks per A tile row (fp16)
  constexpr int RPB = 1024 / (BK * 2);        // A rows per 1 KiB copy block
  constexpr int R256 = BK * 2 >= 256 ? 1 : 256 / (BK * 2);
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int KS = BK / 32;
  constexpr int A_BLK = BM / RPB / NW;        // A copies per wave per k-tile
  constexpr int WCH = BK / 16;                // 16-byte chunks per weight row
  constexpr int RPW = 1024 / BK;              // weight rows per 1 KiB copy block
  constexpr int B_BLK = BN / RPW / NW;        // W copies (RPW rows x BK bytes each) per wave
  constexpr int M_BLK = BFMT == 2 ? 2 : 0;    // fmt 2: one zero-point and one scale copy
  constexpr int L = A_BLK + B_BLK + M_BLK;    // copies per wave per k-tile
  // metadata slots: every wave copies 64 rows (one byte / half per lane, 4 bytes apart); with
  // BN < 64 NW the waves past BN / 64 copy rows (wave % (BN / 64)) * 64 + lane again into slots
  // nobody reads, so the copy count (and the vmcnt arithmetic) is the same in every wave
  constexpr int MROWS = BN > 64 * NW ? BN : 64 * NW;
  constexpr int ABYTES = BM * BK * 2, BBYTES = BN * BK, MBYTES = BFMT == 2 ? MROWS * 8 : 0;
  constexpr int SBYTES = ABYTES + BBYTES + MBYTES;  // one stage
  constexpr int NMF = TM * TN;
  constexpr int RSPAN = RSP > 0 && RSP < NMF / 4 ? RSP : NMF / 4;
  static_assert((BK == 64 || BK == 128) && KS == BK / 32,
                "64-k tiles (a scale group is two of them) or 128-k tiles (one each)");
  static_assert(BM % (RPB * NW) == 0 && BN % (RPW * NW) == 0 && BN % 64 == 0 && (64 * NW) % BN == 0,
                "copy blocks");
  static_assert(STAGES >= 2 && (STAGES - 1) * L < 64, "stages / vmcnt range");
  static_assert((16 / R256) % CPR == 0 && (NW * RPB / R256) % CPR == 0, "swizzle periods");
  static_assert(BFMT == 1 || BFMT == 2, "int8 per-channel or uint8 group-128");
  // EPI: weight copy block d of every wave is in the gate half iff d < HB
  constexpr int HB = (BN / 2) / (RPW * NW);
  static_assert(!EPI || (SPLIT == 0 && (BN / 2) % (RPW * NW) == 0 && (BN / 2) % 64 == 0),
                "gate/up: whole copy and metadata blocks per half");

  // weight chunk swizzle (see the header): keeps 16 consecutive rows' fragment reads on distinct
  // banks for 64-byte and 128-byte rows alike
  auto wswz = [](int r) { return BK == 64 ? (r >> 2) & 3 : (r >> 1) & 7; };
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * SBYTES + (BFMT == 1 ? MROWS * 4 : 0)];
  static_assert(STAGES * SBYTES + (BFMT == 1 ? MROWS * 4 : 0) <= 160 * 1024, "LDS");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  constexpr int BNO = EPI ? BN / 2 : BN;  // output columns per tile
  const int nm = (M + BM - 1) / BM, nn = N / BNO;
  const int ng = K / 128;                     // scale groups per weight row
  int tmi, tni, sk = 0;
  if constexpr (SPLIT)
    split_tile_of<GROUP, XCD>(blockIdx.x, nm, nn, ksplit, tmi, tni, sk);
  else
    tile_of<GROUP, XCD>(blockIdx.x, nm, nn, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BNO;
  // k-tiles of this workgroup: [kbase, kbase + NT)
  const int NTALL = K / BK;
  const int kper = SPLIT ? (NTALL + ksplit - 1) / ksplit : NTALL;
  const int kbase = sk * kper;
  const int NT = min(kper, NTALL - kbase);

  // ---- copies -------------------------------------------------------------------------------
  // A: as k_gemm_ilv (SWZ2 chunk swizzle).  W: BK-byte rows, 16-byte chunk c of row r stored at
  // chunk c ^ wswz(r); copy b fills rows RPW b .. RPW b + RPW - 1, lane l the physical chunk
  // l % WCH of row RPW b + l / WCH, whose logical chunk is (l % WCH) ^ wswz(that row).
  const int crow = wave * RPB + lane / CPR;
  const int cchunk = lds_chunk<BK, SWZ>(crow, lane % CPR) * 8;
  const _Float16* panelA = A + (long)m0 * lda;
  const uint8_t* panelW = W + (long)n0 * ldw;
  const uint8_t* panelWu = W + (long)(up + n0) * ldw;  // EPI: the up half of the tile
  const int nrecA = min(M - m0, BM) * lda * 2, nrecW = BNO * ldw;
  int voff[A_BLK + B_BLK];
#pragma unroll
  for (int d = 0; d < A_BLK; ++d)
    voff[d] = (min(crow + d * NW * RPB, M - 1 - m0) * lda + cchunk) * 2;
#pragma unroll
  for (int d = 0; d < B_BLK; ++d) {
    const int r = (d * NW + wave) * RPW + lane / WCH;
    const int rb = EPI && d >= HB ? r - BN / 2 : r;  // row inside its panel
    voff[A_BLK + d] = rb * ldw + (((lane % WCH) ^ wswz(r)) * 16);
  }
  // fmt 2: zero-point and scale of row q*64 + l (q = this wave) for the stage's group, one byte /
  // one half per lane at a 4-byte lane stride.  EPI: rows of the up half come from the up rows.
  const int mrow = (wave % (BN / 64)) * 64 + lane;
  const bool mup = EPI && (wave % (BN / 64)) * 64 >= BN / 2;
  const long mbase = mup ? (long)up + n0 : (long)n0;
  const int mrel = mup ? mrow - BN / 2 : mrow;  // row inside its metadata panel
  const uint8_t* panelZ = zero + (BFMT == 2 ? mbase * ng : 0);
  const _Float16* panelS = scale + (BFMT == 2 ? mbase * ng : mbase);
  auto dma = [&](int kt, int d) {
    const int ks = kbase + min(kt, NT - 1);
    uint8_t* st = smem + (kt % STAGES) * SBYTES;
    if (d < A_BLK) {
      buf_lds16(panelA, nrecA, st + (d * NW + wave) * 1024, voff[d], ks * BK * 2);
    } else if (d < A_BLK + B_BLK) {
      buf_lds16(EPI && d - A_BLK >= HB ? panelWu : panelW, nrecW,
                st + ABYTES + ((d - A_BLK) * NW + wave) * 1024, voff[d], ks * BK);
    } else if constexpr (BFMT == 2) {
      const int g = ks * BK / 128;
      if (d == A_BLK + B_BLK)
        buf_lds_n<1>(panelZ, BNO * ng, st + ABYTES + BBYTES + wave * 256, mrel * ng, g);
      else
        buf_lds_n<2>(panelS, BNO * ng * 2, st + ABYTES + BBYTES + MROWS * 4 + wave * 256,
                     mrel * ng * 2, g * 2);
    }
  };

  typename MF::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  const int fr = lane % 16, fk = lane / 16;
  int aOff[KS], bOff[KS];  // byte offsets inside a stage
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int ra = wm * WTM + fr, rb = wn * WTN + fr;
    aOff[ks] = (ra * BK + lds_chunk<BK, SWZ>(ra, ks * 4 + fk) * 8) * 2;
    bOff[ks] = ABYTES + rb * BK + (((ks * 2 + fk / 2) ^ wswz(fr)) * 16) + (fk & 1) * 8;
  }
  const int rowm = (wn * WTN + fr) * 4;       // this lane's metadata slot of block j = 0

  f16x8 fa[2][TM];
  u32x2 braw[2][TN];                          // weight bytes of the current / next substep
  // per block j: fp16 1024 + zero-point (fmt 2; 1152 for the sign-flipped int8 of fmt 1) and the
  // scale -- of the current scale group, and (fmt 2) of the next one, read ahead
  _Float16 bias[TN], sc[TN], nbias[TN], nsc[TN];
  if constexpr (BFMT == 1) {
#pragma unroll
    for (int j = 0; j < TN; ++j) bias[j] = (_Float16)1152.0f;
  }
  auto read_meta = [&](const uint8_t* st, _Float16 (&bi)[TN], _Float16 (&s)[TN], int j) {
    bi[j] = (_Float16)(1024.0f + (float)st[ABYTES + BBYTES + rowm + j * 64]);
    s[j] = *reinterpret_cast<const _Float16*>(st + ABYTES + BBYTES + MROWS * 4 + rowm + j * 64);
  };
  auto deq = [&](const u32x2& w, int j) -> f16x8 {
    const uint32_t x0 = BFMT == 1 ? w[0] ^ 0x80808080u : w[0];
    const uint32_t x1 = BFMT == 1 ? w[1] ^ 0x80808080u : w[1];
    return dequant8(x0, x1, bias[j], sc[j]);
  };

  // One substep on buffer bb: the MFMAs of this substep run block column by block column (j
  // outer), each column's weight fragment dequantised from braw[bb] one chunk ahead of its
  // MFMAs; the next substep's fragments (tile rkt, substep rks) are read into fa / braw [bb^1]
  // in the first RSPAN chunks; META: also the next scale group's metadata (fmt 2); DMA: refill
  // of the stage of tile dkt.
  constexpr int NRD = TM + TN + (BFMT == 2 ? 2 * TN : 0);  // reads of a substep with metadata
  constexpr int CH = NMF / 4;                              // chunks of 4 MFMAs
  constexpr int CPJ = CH / TN;                             // chunks per block column
  static_assert(CH % TN == 0 && CPJ >= 1 && RSPAN <= CH && L <= 4 * CH, "substep chunking");
  auto substep = [&](auto bufc, auto dmac, auto metac, int rkt, int rks, int dkt) {
    constexpr int bb = decltype(bufc)::value;
    constexpr bool DMA = decltype(dmac)::value;
    constexpr bool META = decltype(metac)::value;
    const uint8_t* st = smem + (rkt % STAGES) * SBYTES;
    f16x8 fbt[2];
    fbt[0] = deq(braw[bb][0], 0);
#pragma unroll
    for (int q = 0; q < CH; ++q) {
#pragma unroll
      for (int r = 0; r < NRD; ++r) {
        if (r * RSPAN / NRD != q) continue;
        if (r < TM) {
          fa[bb ^ 1][r] = *reinterpret_cast<const f16x8*>(st + aOff[rks] + r * 16 * BK * 2);
        } else if (r < TM + TN) {
          braw[bb ^ 1][r - TM] = *reinterpret_cast<const u32x2*>(st + bOff[rks] + (r - TM) * 16 * BK);
        } else if constexpr (BFMT == 2 && META) {
          if ((r - TM - TN) % 2 == 0) read_meta(st, nbias, nsc, (r - TM - TN) / 2);
        }
      }
      if constexpr (DMA) {
#pragma unroll
        for (int d = 0; d < L; ++d)
          if (d * CH / L == q) dma(dkt, d);
      }
      const int j = q / CPJ;
      // the next column's fragment, one chunk before its MFMAs
      if (q % CPJ == CPJ - 1 && j + 1 < TN) fbt[(j + 1) & 1] = deq(braw[bb][j + 1], j + 1);
#pragma unroll
      for (int t = q * 4; t < q * 4 + 4; ++t)
        acc[t % TM][t / TM] = MF::run(fbt[(t / TM) & 1], fa[bb][t % TM], acc[t % TM][t / TM]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // k-tile kt (substeps 0 .. KS-1).  The last is the barrier substep: copies of tile kt+1
  // landed everywhere, stage kt % STAGES free; fmt 2: it also reads tile kt+1's metadata (every
  // stage carries its scale group's), which becomes current right after it -- the barrier
  // substep's own fragments are still tile kt's.
  auto plain = [&](auto sc, int kt) {       // substep s < KS-1: MFMAs of s, fragments of s + 1
    constexpr int s = decltype(sc)::value;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0): this substep's fragments are in
    asm volatile("" ::: "memory");
    substep(IC<s & 1>{}, IC<false>{}, IC<false>{}, kt, s + 1, 0);
  };
  auto ktile = [&](auto metac, int kt) {
    constexpr bool META = decltype(metac)::value;
    plain(IC<0>{}, kt);
    if constexpr (KS == 4) {
      plain(IC<1>{}, kt);
      plain(IC<2>{}, kt);
    }
    asm volatile("" ::: "memory");
    s_wait_vm<(STAGES - 2) * L>();            // (also lgkmcnt 0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    substep(IC<(KS - 1) & 1>{}, IC<true>{}, metac, kt + 1, 0, kt + STAGES);
    if constexpr (BFMT == 2 && META) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
      for (int j = 0; j < TN; ++j) { bias[j] = nbias[j]; sc[j] = nsc[j]; }
    }
  };

  // prologue: fmt 1 scales (once), then every stage in flight; tile 0 landed and visible; its
  // metadata and first fragments read
  uint8_t* const sc1 = smem + STAGES * SBYTES;
  if constexpr (BFMT == 1)
    buf_lds_n<2>(panelS, BNO * 2, sc1 + wave * 256, mrel * 2, 0);
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
#pragma unroll
    for (int d = 0; d < L; ++d) dma(s, d);
  asm volatile("" ::: "memory");
  s_wait_vm<(STAGES - 1) * L>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    if constexpr (BFMT == 1) sc[j] = *reinterpret_cast<const _Float16*>(sc1 + rowm + j * 64);
    else read_meta(smem, bias, sc, j);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[0][i] = *reinterpret_cast<const f16x8*>(smem + aOff[0] + i * 16 * BK * 2);
#pragma unroll
  for (int j = 0; j < TN; ++j) braw[0][j] = *reinterpret_cast<const u32x2*>(smem + bOff[0] + j * 16 * BK);
  __builtin_amdgcn_sched_barrier(0);

  for (int kt = 0; kt < NT; ++kt) ktile(IC<BFMT == 2>{}, kt);
  s_wait_vm<0>();

  if constexpr (SPLIT) {
    // fp32 partial tile of split sk: each lane's 4 consecutive n of one m per block, 16 bytes
    float* part = ws + (long)sk * M * N;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * WTM + i * 16 + fr;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *reinterpret_cast<f32x4*>(part + (long)m * N + n0 + wn * WTN + j * 16 + 4 * fk) = acc[i][j];
    }
    return;
  }

  // ---- epilogue: C tile through LDS, as k_gemm_ilv ---------------------------------------------
  // The lane and thread indices are rebuilt here (lane_id) rather than kept from the prologue:
  // with 256 accumulators and the fragment buffers live, a value held across the loop spills.
  constexpr int RB = BN * 2, CPRW = RB / 16, RPP = NW * 64 / CPRW;
  static_assert(BM * BN * 2 <= STAGES * SBYTES && CPRW >= 16 && (CPRW & (CPRW - 1)) == 0, "C tile in LDS");
  const bool c16 = ((reinterpret_cast<uintptr_t>(C) | (uintptr_t)ldc * 2) & 15) == 0;
  __syncthreads();
  const int elane = lane_id();
  const int efr = elane % 16, efk = elane / 16;
  const int etid = wave * 64 + elane;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = wm * WTM + i * 16 + efr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int cb = (wn * WTN + j * 16 + 4 * efk) * 2;
      f16x4 o;
      o[0] = (_Float16)acc[i][j][0];
      o[1] = (_Float16)acc[i][j][1];
      o[2] = (_Float16)acc[i][j][2];
      o[3] = (_Float16)acc[i][j][3];
      *reinterpret_cast<f16x4*>(smem + r * RB + (((cb >> 4) ^ (r & 15)) << 4) + (cb & 15)) = o;
    }
  }
  __syncthreads();
  if constexpr (EPI) {
    // output row r, chunk c (8 columns): gate chunk c, up chunk c + CPRW/2 of image row r
    constexpr int CPO = CPRW / 2, RPO = NW * 64 / CPO;
#pragma unroll 4
    for (int p = 0; p < BM / RPO; ++p) {
      const int r = p * RPO + etid / CPO, c = etid % CPO;
      const f16x8 g = as_f16x8(*reinterpret_cast<const u32x4*>(smem + r * RB + ((c ^ (r & 15)) << 4)));
      const f16x8 u =
          as_f16x8(*reinterpret_cast<const u32x4*>(smem + r * RB + (((c + CPO) ^ (r & 15)) << 4)));
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = silu_mul_f16((float)g[e], (float)u[e]);
      const u32x4 v = __builtin_bit_cast(u32x4, o);
      if (m0 + r < M) {
        _Float16* dst = C + (long)(m0 + r) * ldc + n0 + c * 8;
        if (c16) {
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
        } else {
          __builtin_nontemporal_store(u32x2{v[0], v[1]}, reinterpret_cast<u32x2*>(dst));
          __builtin_nontemporal_store(u32x2{v[2], v[3]}, reinterpret_cast<u32x2*>(dst + 4));
        }
      }
    }
    return;
  }
#pragma unroll 4
  for (int p = 0; p < BM / RPP; ++p) {
    const int r = p * RPP + etid / CPRW, c = etid % CPRW;
    const u32x4 v = *reinterpret_cast<const u32x4*>(smem + r * RB + ((c ^ (r & 15)) << 4));
    if (m0 + r < M) {
      _Float16* dst = C + (long)(m0 + r) * ldc + n0 + c * 8;
      if (c16) {
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
      } else {
        __builtin_nontemporal_store(u32x2{v[0], v[1]}, reinterpret_cast<u32x2*>(dst));
        __builtin_nontemporal_store(u32x2{v[2], v[3]}, reinterpret_cast<u32x2*>(dst + 4));
      }
    }
  }
}
