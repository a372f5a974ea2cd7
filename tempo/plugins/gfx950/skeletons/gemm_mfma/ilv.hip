// gemm_mfma/ilv.hip -- the interleaved prefill GEMM (fp16 x fp16).  Uses the tile machinery of
// gemm_mfma/kernel.hip (lds_chunk, tile_of, s_wait_vm, buf_lds16), which must come first.
// ============================================================================================
// k_gemm_ilv -- fp16 B only, prefill: one wave per SIMD, large wave tiles, and a main loop that
// is software-pipelined by hand ("interleaved").
//
// Each wave owns a (BM/WM) x (BN/WN) tile of C (128 x 128 for the shipped 256 x 256 / 4-wave
// row: 256 fp32 accumulators per lane, all in AGPRs), so every fragment byte read from LDS feeds
// twice the MFMAs it does in a 64 x 64 wave tile: LDS traffic per flop is halved, which is what
// the power-limited matrix cores of this part spend their budget on besides the MFMAs.
//
// Substep = 32 k (one v_mfma_f32_16x16x32_f16 per 16 x 16 block of the wave tile).  A substep
// issues its TM*TN MFMAs on the fragments read during the previous substep, and between them
// (in CH chunks fenced by sched_barrier) the LDS reads of the next substep's fragments -- in the
// first RSP chunks, so they have landed long before they are needed -- and, in the substep that
// holds the tile barrier, the LDS-DMA copies that refill the stage the barrier has just freed.
// One barrier per k-tile; no MFMA ever waits on an LDS read issued in the same substep.
//
// Stage of tile t = t % STAGES.  The barrier of tile t (in its last substep) is passed once
// every wave has finished reading tile t (lgkmcnt 0) and its own copies of tile t+1 have landed
// (vmcnt); after it tile t+1 is readable by all and stage t % STAGES is refilled with tile
// t + STAGES.  Past the last tile the refill re-copies tile NT-1 into a stage nobody reads again
// and the last substep reads fragments it does not use: the loop body stays one straight-line
// region, so the interleave holds from the first tile to the last.  Those copies are younger
// than every copy a later wait counts, so the vmcnt arithmetic is unchanged, and the kernel
// drains them (vmcnt 0) before the epilogue, so no copy lands after the workgroup has left.
//
// Copies are buffer loads with an LDS destination (buffer_load_dwordx4 ... lds): the resource
// descriptor (SGPRs) points at this tile's A or B panel, each copy's per-lane byte offset is a
// loop constant and the k offset goes in the scalar offset, so a copy costs no vector address
// arithmetic (the 64-bit per-copy address adds of the global form took VALU issue slots next to
// the MFMAs).
//
// Epilogue: where the C tile fits the stages (and a C row is a power of two of at least 256
// bytes), it goes through LDS (free by then) -- fp16 values written in the MFMA layout into a
// row-major image whose 16-byte chunks are XOR-swizzled by row, read back as whole rows and
// written out with 16-byte nontemporal stores, eight lanes per 128-byte line.  Stored straight
// from the MFMA layout, each row gets 32-byte pieces per instruction, and those partial-line
// writes took twice as long (8 us against 4 us per 256 x 256 tile).
//
// Requirements (applicable() + the ladder): N % BN == 0, K % 64 == 0 (an even number of
// substeps), 16-byte aligned rows of A and B, C and ldc 8-byte aligned, panel byte offsets below
// 2^31 (BM*lda*2, BN*ldb*2).  M is predicated: A rows past M-1 are re-read from row M-1 and
// never stored.
//
// SPLIT = 1 (split-K): the grid is tiles x ksplit workgroups (split_tile_of); workgroup split sk
// takes the k-tiles [sk*kper, min((sk+1)*kper, K/BK)), kper = ceil((K/BK) / ksplit) -- the host
// picks ksplit so that no split is empty -- and writes its fp32 partial tile straight from the
// accumulators to ws[sk][M][N] (16 bytes per lane and block); k_splitk_reduce then adds the
// splits in order and rounds once.  Narrow-N, long-K shapes get enough workgroups this way.
//
// EPI = 1 (fused gate/up, prefill): C[M][N] = silu(A.B[0..N)^T) * (A.B[N..2N)^T), B holding the
// gate rows then the up rows (2N rows, N the output width).  A workgroup covers BN/2 output
// columns: its B tile is BN/2 gate rows followed by the BN/2 matching up rows (two panels, the
// copy blocks of each half a compile-time set), so the gate and up results of one output sit
// in the same C tile image in LDS, BN/2 columns apart; the epilogue reads both halves back and
// writes fp16_rn(silu(g) * u) of the fp16-rounded g and u (silu_mul_f16).  No split-K.
//
// Build: this kernel is compiled with -mllvm -amdgpu-sched-strategy=iterative-minreg (its own
// translation unit).  The default pre-RA scheduler reorders the 256 accumulator chains of a
// 128 x 128 wave tile such that the register allocator no longer keeps each accumulator in one
// AGPR tuple, and the loop fills with v_accvgpr_read/write/mov copies.
// ============================================================================================
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUP, int XCD, int RSP,
          int SPLIT = 0, int EPI = 0>
__global__ __launch_bounds__(WM * WN * 64, 1) void k_gemm_ilv(
    const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
    int M, int N, int K, int lda, int ldb, int ldc, float* __restrict__ ws, int ksplit, int up) {
  using MF = Mfma<16>;
  constexpr int SWZ = 2;
  constexpr int NW = WM * WN;
  constexpr int CPR = BK / 8;                 // 16-byte chunks per tile row
  constexpr int RPB = 1024 / (BK * 2);        // tile rows per 1 KiB copy block
  constexpr int R256 = BK * 2 >= 256 ? 1 : 256 / (BK * 2);  // rows per SWZ 2 key step
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int KS = BK / 32;                 // substeps per k-tile
  constexpr int A_BLK = BM / RPB / NW, B_BLK = BN / RPB / NW;
  constexpr int L = A_BLK + B_BLK;            // copies per wave per k-tile
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int NMF = TM * TN, NR = TM + TN;  // MFMAs and fragment reads per substep
  constexpr int CH = NR > L ? NR : L;
  constexpr int RSPAN = RSP > 0 && RSP < CH ? RSP : CH;
  static_assert(BM % (RPB * NW) == 0 && BN % (RPB * NW) == 0, "copy blocks per wave");
  static_assert(STAGES >= 2 && (STAGES - 1) * L < 64, "stages / vmcnt range");
  // EPI: the gate half of the B tile is its first HB copy blocks of every wave
  constexpr int HB = (BN / 2) / (NW * RPB);
  static_assert(!EPI || (SPLIT == 0 && (BN / 2) % (NW * RPB) == 0), "gate/up: whole copy blocks");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0 && (KS == 1 || KS == 2), "tile shape");
  // rows 16 apart (fragment blocks) and NW*RPB apart (copy blocks) share the swizzle key, so
  // one per-lane offset serves every block of an operand
  static_assert((16 / R256) % CPR == 0 && (NW * RPB / R256) % CPR == 0, "swizzle periods");

  __shared__ __attribute__((aligned(1024))) _Float16 smem[STAGES * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  constexpr int BNO = EPI ? BN / 2 : BN;  // output columns per tile
  const int nm = (M + BM - 1) / BM, nn = N / BNO;
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

  // Copy d of this wave fills 1 KiB block (ib*NW + wave) of the A (d < A_BLK) or B tile; lane l
  // fetches the 16-byte chunk that belongs at LDS slot l (the swizzle is an involution).  The
  // buffers start at the tile's panels; A rows past M-1 are clamped to row M-1.
  const int crow = wave * RPB + lane / CPR;                       // tile row of block ib = 0
  const int cchunk = lds_chunk<BK, SWZ>(crow, lane % CPR) * 8;    // element offset in the row
  const _Float16* panelA = A + (long)m0 * lda;
  const _Float16* panelB = B + (long)n0 * ldb;
  // EPI: the up half of the B tile starts at row up + n0 (up = the full output width; a launch
  // over some of the output columns has B offset to its first gate row)
  const _Float16* panelU = B + (long)(up + n0) * ldb;
  const int nrecA = min(M - m0, BM) * lda * 2, nrecB = (EPI ? BN / 2 : BN) * ldb * 2;
  int voff[L];
#pragma unroll
  for (int d = 0; d < L; ++d) {
    const bool isA = d < A_BLK;
    const int ib = isA ? d : d - A_BLK;
    const int r = crow + ib * NW * RPB;
    const int rb = EPI && !isA && ib >= HB ? r - BN / 2 : r;  // row inside its B panel
    voff[d] = isA ? (min(r, M - 1 - m0) * lda + cchunk) * 2 : (rb * ldb + cchunk) * 2;
  }
  auto dma = [&](int kt, int ksrc, int d) {
    const bool isA = d < A_BLK;
    const int ib = isA ? d : d - A_BLK;
    _Float16* dst = smem + (kt % STAGES) * STAGE + (isA ? 0 : BM * BK) + (ib * NW + wave) * RPB * BK;
    const _Float16* pan = isA ? panelA : (EPI && ib >= HB ? panelU : panelB);
    buf_lds16(pan, isA ? nrecA : nrecB, dst, voff[d], (kbase + ksrc) * BK * 2);
  };

  typename MF::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  const int fr = lane % 16, fk = lane / 16;
  int aOff[KS], bOff[KS];  // fragment offsets (elements) inside a stage, per substep
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int ra = wm * WTM + fr, rb = wn * WTN + fr;
    aOff[ks] = ra * BK + lds_chunk<BK, SWZ>(ra, ks * 4 + fk) * 8;
    bOff[ks] = BM * BK + rb * BK + lds_chunk<BK, SWZ>(rb, ks * 4 + fk) * 8;
  }

  f16x8 fa[2][TM], fb[2][TN];
  // One substep on fragment buffer bb: read the next substep (tile rkt, substep rks) into bb^1,
  // refill (DMA) the stage of tile dkt with k-tile dsrc, and run the MFMAs on bb.
  auto substep = [&](auto bufc, auto dmac, int rkt, int rks, int dkt, int dsrc) {
    constexpr int bb = decltype(bufc)::value;
    constexpr bool DMA = decltype(dmac)::value;
    const _Float16* s = smem + (rkt % STAGES) * STAGE;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (r * RSPAN / NR != q) continue;
        if (r < TM)
          fa[bb ^ 1][r] = *reinterpret_cast<const f16x8*>(s + aOff[rks] + r * 16 * BK);
        else
          fb[bb ^ 1][r - TM] = *reinterpret_cast<const f16x8*>(s + bOff[rks] + (r - TM) * 16 * BK);
      }
      if constexpr (DMA) {
#pragma unroll
        for (int d = 0; d < L; ++d)
          if (d * CH / L == q) dma(dkt, dsrc, d);
      }
#pragma unroll
      for (int t = q * NMF / CH; t < (q + 1) * NMF / CH; ++t)
        acc[t / TN][t % TN] = MF::run(fb[bb][t % TN], fa[bb][t / TN], acc[t / TN][t % TN]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int NU = NT * KS;  // substeps (even: K % 64 == 0)
  auto step = [&](auto bufc, auto barc, int u) {
    constexpr bool BAR = decltype(barc)::value;
    const int kt = KS == 1 ? u : u >> 1;
    asm volatile("" ::: "memory");
    if constexpr (BAR) {
      // this wave's reads of tile kt are done and its copies of tile kt+1 have landed ...
      s_wait_vm<(STAGES - 2) * L>();
      // ... and everyone's: tile kt+1 is readable, stage kt % STAGES is free
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      substep(bufc, IC<true>{}, kt + 1, 0, kt + STAGES, min(kt + STAGES, NT - 1));
    } else {
      // this substep's fragments were read in the first chunks of the previous one: the wait
      // is free, and placing it here keeps the compiler from waiting after this substep's
      // first reads instead
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      asm volatile("" ::: "memory");
      substep(bufc, IC<false>{}, kt, 1, 0, 0);
    }
  };

  // prologue: every stage in flight, tile 0 landed and visible, its first fragments read
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
#pragma unroll
    for (int d = 0; d < L; ++d) dma(s, min(s, NT - 1), d);
  asm volatile("" ::: "memory");
  s_wait_vm<(STAGES - 1) * L>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[0][i] = *reinterpret_cast<const f16x8*>(smem + aOff[0] + i * 16 * BK);
#pragma unroll
  for (int j = 0; j < TN; ++j) fb[0][j] = *reinterpret_cast<const f16x8*>(smem + bOff[0] + j * 16 * BK);
  __builtin_amdgcn_sched_barrier(0);

  for (int u = 0; u < NU; u += 2) {
    step(IC<0>{}, IC<KS == 1>{}, u);
    step(IC<1>{}, IC<true>{}, u + 1);
  }
  s_wait_vm<0>();  // the refills past the end land before the workgroup's LDS is released

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

  // ---- epilogue ------------------------------------------------------------------------------
  // Rows are written out in 16-byte pieces when C and ldc allow it, else in 8-byte halves.
  const bool c16 = ((reinterpret_cast<uintptr_t>(C) | (uintptr_t)ldc * 2) & 15) == 0;
  auto store16 = [&](_Float16* dst, const u32x4& v) {
    if (c16) {
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
    } else {
      __builtin_nontemporal_store(u32x2{v[0], v[1]}, reinterpret_cast<u32x2*>(dst));
      __builtin_nontemporal_store(u32x2{v[2], v[3]}, reinterpret_cast<u32x2*>(dst + 4));
    }
  };
  constexpr int RB = BN * 2;                  // bytes per C row
  constexpr int CPRW = RB / 16;               // 16-byte chunks per C row
  constexpr bool LDS_EPI = BM * BN <= STAGES * STAGE && CPRW >= 16 && (CPRW & (CPRW - 1)) == 0 &&
                           (NW * 64) % CPRW == 0;
  static_assert(!EPI || LDS_EPI, "gate/up: the epilogue pairs the halves through LDS");
  if constexpr (LDS_EPI) {
    // The C tile through LDS (the stages are free by then): a row-major fp16 image whose 16-byte
    // chunk c of row r sits at chunk c ^ (r % 16), so the 16 rows of an MFMA block write to 16
    // distinct bank groups and a row's chunks read back conflict-free; then whole rows out.
    constexpr int RPP = NW * 64 / CPRW;       // C rows per pass of the whole workgroup
    __syncthreads();                          // every wave is done with the stages
    uint8_t* cs = reinterpret_cast<uint8_t*>(smem);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * WTM + i * 16 + fr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int cb = (wn * WTN + j * 16 + 4 * fk) * 2;  // byte offset of the lane's 4 values
        f16x4 o;
        o[0] = (_Float16)acc[i][j][0];
        o[1] = (_Float16)acc[i][j][1];
        o[2] = (_Float16)acc[i][j][2];
        o[3] = (_Float16)acc[i][j][3];
        *reinterpret_cast<f16x4*>(cs + r * RB + (((cb >> 4) ^ (r & 15)) << 4) + (cb & 15)) = o;
      }
    }
    __syncthreads();
    if constexpr (EPI) {
      // output row r, chunk c (8 columns): gate chunk c, up chunk c + CPRW/2 of image row r
      constexpr int CPO = CPRW / 2, RPO = NW * 64 / CPO;
#pragma unroll 4
      for (int p = 0; p < BM / RPO; ++p) {
        const int r = p * RPO + tid / CPO, c = tid % CPO;
        const f16x8 g = as_f16x8(*reinterpret_cast<const u32x4*>(cs + r * RB + ((c ^ (r & 15)) << 4)));
        const f16x8 u =
            as_f16x8(*reinterpret_cast<const u32x4*>(cs + r * RB + (((c + CPO) ^ (r & 15)) << 4)));
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = silu_mul_f16((float)g[e], (float)u[e]);
        if (m0 + r < M) store16(C + (long)(m0 + r) * ldc + n0 + c * 8, __builtin_bit_cast(u32x4, o));
      }
      return;
    }
#pragma unroll 4
    for (int p = 0; p < BM / RPP; ++p) {
      const int r = p * RPP + tid / CPRW, c = tid % CPRW;
      const u32x4 v = *reinterpret_cast<const u32x4*>(cs + r * RB + ((c ^ (r & 15)) << 4));
      if (m0 + r < M) store16(C + (long)(m0 + r) * ldc + n0 + c * 8, v);
    }
  } else {
    // straight from the MFMA layout: each lane owns 4 consecutive n of one m per block
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * WTM + i * 16 + fr;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * WTN + j * 16 + 4 * fk;
        f16x4 o;
        o[0] = (_Float16)acc[i][j][0];
        o[1] = (_Float16)acc[i][j][1];
        o[2] = (_Float16)acc[i][j][2];
        o[3] = (_Float16)acc[i][j][3];
        *reinterpret_cast<f16x4*>(C + (long)m * ldc + n) = o;
      }
    }
  }
}
