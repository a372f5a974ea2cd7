// gemm_mfma -- tiled C[M,N] = A[M,K] . B[N,K]^T on CDNA4 matrix cores (gfx950).
//
// Semantics follow the reference's naive kernel (kernels/naive/gemm_fp16.cu:60-68): fp16
// operands, fp32 accumulation, one RNE rounding to fp16 per output.  The order of the k
// summation differs (MFMA dot products), which is why parity is a relL2 gate, not bit equality.
//
// Template axes (the plugin's search space, tempo/plugins/gfx950/space.py):
//   BM, BN   macro tile of C per workgroup
//   BK       k extent of one LDS stage (the LDS holds two stages: double buffer)
//   WM, WN   waves along M and N (workgroup = WM*WN*64 lanes); wave tile (BM/WM) x (BN/WN)
//   MS       MFMA shape: 32 -> v_mfma_f32_32x32x16_f16, 16 -> v_mfma_f32_16x16x32_f16
//   SWZ      LDS chunk swizzle: 0 none, 1 chunk ^ (row % CPR), 2 chunk ^ ((row/2) % CPR)
//   GROUP    raster group height in tiles (L2 reuse); 0 = row-major tile order
//   XCD      1 = remap block ids so each of the 8 XCDs owns a contiguous run of tiles
//   BFMT     B operand format: 0 fp16, 1 int8 + per-row fp16 scale, 2 uint8 + per-(row,group)
//            fp16 scale and uint8 zero-point.  Formats 1 and 2 dequantise while staging the
//            B tile into LDS (once per workgroup, not once per wave), bit-exact with the
//            closed forms in cdna4.h.
//
// Layout in registers: the MFMA "A" operand is fed from B rows (n) and the "B" operand from A
// rows (m), so each lane's result values are 4 consecutive n of one m -- the epilogue writes
// 8-byte runs of C instead of 2-byte scatters.
//
// LDS layout: per stage, A tile [BM][BK] and B tile [BN][BK] fp16, k contiguous, 16-byte chunks
// swizzled by row so the 16-byte MFMA feed reads (one row per lane) spread over the banks.
//
// Requirements checked by the launcher (applicable()): N % BN == 0, K % BK == 0, 16-byte
// aligned rows; M is predicated (rows past M are loaded from row M-1 and never stored).

// LDS chunk swizzle: the 16-byte chunk c of tile row `row` is stored at chunk c ^ f(row).
// SWZ 1: f = (row / rows-per-128B) % CPR -- spreads 8 consecutive rows over 32 banks.
// SWZ 2: f = (row / rows-per-256B) % CPR -- spreads 16 consecutive rows over 64 banks.
template <int BK, int SWZ>
__device__ __forceinline__ int lds_chunk(int row, int chunk) {
  constexpr int CPR = BK / 8;  // 16-byte chunks per row
  constexpr int ROW_BYTES = BK * 2;
  if constexpr (SWZ == 1) {
    constexpr int R128 = ROW_BYTES >= 128 ? 1 : 128 / ROW_BYTES;
    return chunk ^ ((row / R128) & (CPR - 1));
  } else if constexpr (SWZ == 2) {
    constexpr int R256 = ROW_BYTES >= 256 ? 1 : 256 / ROW_BYTES;
    return chunk ^ ((row / R256) & (CPR - 1));
  } else {
    return chunk;
  }
}

// Tile order: block id -> (tile_m, tile_n).
template <int GROUP, int XCD>
__device__ __forceinline__ void tile_of(int bid, int nm, int nn, int& tm, int& tn) {
  const int total = nm * nn;
  if constexpr (XCD) {
    // Workgroups are handed to the 8 XCDs round-robin (bid % 8).  Give XCD x the contiguous
    // run [x*total/8, (x+1)*total/8) of the tile order so its concurrent tiles share panels in
    // that XCD's own L2.
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  }
  if constexpr (GROUP > 0) {
    const int per = GROUP * nn;
    const int g = bid / per;
    const int first = g * GROUP;
    const int gs = min(GROUP, nm - first);
    const int r = bid - g * per;
    tm = first + r % gs;
    tn = r / gs;
  } else {
    tm = bid / nn;
    tn = bid - tm * nn;
  }
}

// Split-K tile order: block id -> (tile_m, tile_n, split).  The XCD remap runs over all
// tiles x ksplit workgroups, then the order is split-major: the workgroups an XCD holds at once
// share k ranges, i.e. the same activation panel slices, in that XCD's L2.
template <int GROUP, int XCD>
__device__ __forceinline__ void split_tile_of(int bid, int nm, int nn, int ksplit, int& tm, int& tn,
                                              int& sk) {
  const int tiles = nm * nn;
  if constexpr (XCD) {
    const int total = tiles * ksplit;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  }
  sk = bid / tiles;
  tile_of<GROUP, 0>(bid - sk * tiles, nm, nn, tm, tn);
}

// Split-K reduction: C[m][n] = fp16_rn(ws[0][m][n] + ws[1][m][n] + ... + ws[S-1][m][n]), the
// partial sums added in the fixed order s = 0 .. S-1 in fp32 (deterministic), one rounding to
// fp16.  ws is [S][M][N] fp32 (rows of N), N % 4 == 0; each thread takes 4 consecutive n.  The
// partial loads of UNROLL splits are issued together before their adds, so a thread keeps UNROLL
// loads in flight instead of waiting for each one (the reduction is a pure streaming read).
// (A template so that every translation unit that includes this file may instantiate it.)
template <int UNROLL = 8>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int S, int M,
                                                       int N, _Float16* __restrict__ C, int ldc) {
  const long per = (long)M * N;
  const long i4 = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i4 >= per) return;
  const int m = (int)(i4 / N), n = (int)(i4 - (long)m * N);
  const float* src = ws + i4;
  f32x4 acc = *reinterpret_cast<const f32x4*>(src);
  int s = 1;
  for (; s + UNROLL <= S; s += UNROLL) {
    f32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = *reinterpret_cast<const f32x4*>(src + (s + u) * per);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc += v[u];
  }
  for (; s < S; ++s) acc += *reinterpret_cast<const f32x4*>(src + s * per);
  f16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (_Float16)acc[e];
  *reinterpret_cast<f16x4*>(C + (long)m * ldc + n) = o;
}

template <int BM, int BN, int BK, int WM, int WN, int MS, int SWZ, int GROUP, int XCD, int BFMT>
struct GemmCfg {
  static constexpr int THREADS = WM * WN * 64;
  static constexpr int CPR = BK / 8;
  static constexpr int WTM = BM / WM;  // wave tile rows (m)
  static constexpr int WTN = BN / WN;  // wave tile cols (n)
  static constexpr int TM = WTM / MS;  // MFMA blocks per wave along m
  static constexpr int TN = WTN / MS;
  static constexpr int KS = BK / Mfma<MS>::KSTEP;  // MFMA k-steps per stage
  static constexpr int A_IT = BM * CPR / THREADS;  // 16-byte A chunks per thread per stage
  static constexpr int B_IT = BN * CPR / THREADS;
  static constexpr int LDS_BYTES = 2 * (BM + BN) * BK * 2;
  static_assert(BK % Mfma<MS>::KSTEP == 0, "BK must hold whole MFMA k-steps");
  static_assert(WTM % MS == 0 && WTN % MS == 0, "wave tile must hold whole MFMA blocks");
  static_assert((BM * CPR) % THREADS == 0 && (BN * CPR) % THREADS == 0, "tile/thread split");
  static_assert(CPR == 4 || CPR == 8, "BK of 32 or 64");
};

// Raw B chunk as loaded from global memory: 16 bytes of fp16, or 8 bytes of int8/uint8.
template <int BFMT>
struct BRaw;
template <>
struct BRaw<0> { u32x4 v; };
template <>
struct BRaw<1> { u32x2 v; };
template <>
struct BRaw<2> { u32x2 v; };

template <int BM, int BN, int BK, int WM, int WN, int MS, int SWZ, int GROUP, int XCD, int BFMT>
__global__ __launch_bounds__(WM * WN * 64, 1) void k_gemm(
    const _Float16* __restrict__ A, const void* __restrict__ Bv,
    const _Float16* __restrict__ scale, const uint8_t* __restrict__ zero,
    _Float16* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldc, int group) {
  using Cfg = GemmCfg<BM, BN, BK, WM, WN, MS, SWZ, GROUP, XCD, BFMT>;
  using MF = Mfma<MS>;
  constexpr int T = Cfg::THREADS, CPR = Cfg::CPR;
  constexpr int TM = Cfg::TM, TN = Cfg::TN;

  __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (BM + BN) * BK];
  _Float16* const sA = smem;                 // [2][BM][BK]
  _Float16* const sB = smem + 2 * BM * BK;   // [2][BN][BK]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nm = (M + BM - 1) / BM, nn = N / BN;
  int tmi, tni;
  tile_of<GROUP, XCD>(blockIdx.x, nm, nn, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;

  // ---- global -> register staging -------------------------------------------------------
  const u32x4* gA[Cfg::A_IT];
  int sAoff[Cfg::A_IT];
#pragma unroll
  for (int i = 0; i < Cfg::A_IT; ++i) {
    const int q = tid + i * T, r = q / CPR, c = q % CPR;
    const int gm = min(m0 + r, M - 1);
    gA[i] = reinterpret_cast<const u32x4*>(A + (long)gm * lda + c * 8);
    sAoff[i] = r * BK + lds_chunk<BK, SWZ>(r, c) * 8;
  }
  int sBoff[Cfg::B_IT];
  long gBoff[Cfg::B_IT];  // element offset of the chunk's row start + k
  int bRow[Cfg::B_IT], bC[Cfg::B_IT];
#pragma unroll
  for (int i = 0; i < Cfg::B_IT; ++i) {
    const int q = tid + i * T, r = q / CPR, c = q % CPR;
    bRow[i] = n0 + r;
    bC[i] = c;
    gBoff[i] = (long)(n0 + r) * ldb + c * 8;
    sBoff[i] = r * BK + lds_chunk<BK, SWZ>(r, c) * 8;
  }
  _Float16 rowScale[Cfg::B_IT];
  if constexpr (BFMT == 1) {
#pragma unroll
    for (int i = 0; i < Cfg::B_IT; ++i) rowScale[i] = scale[bRow[i]];
  }

  u32x4 ra[Cfg::A_IT];
  BRaw<BFMT> rb[Cfg::B_IT];

  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < Cfg::A_IT; ++i) ra[i] = gA[i][k0 / 8];
#pragma unroll
    for (int i = 0; i < Cfg::B_IT; ++i) {
      if constexpr (BFMT == 0)
        rb[i].v = *reinterpret_cast<const u32x4*>(
            reinterpret_cast<const _Float16*>(Bv) + gBoff[i] + k0);
      else
        rb[i].v = *reinterpret_cast<const u32x2*>(
            reinterpret_cast<const uint8_t*>(Bv) + gBoff[i] + k0);
    }
  };
  auto store_stage = [&](int buf, int k0) {
    _Float16* a = sA + buf * BM * BK;
    _Float16* b = sB + buf * BN * BK;
#pragma unroll
    for (int i = 0; i < Cfg::A_IT; ++i) *reinterpret_cast<u32x4*>(a + sAoff[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < Cfg::B_IT; ++i) {
      u32x4 v;
      if constexpr (BFMT == 0) {
        v = rb[i].v;
      } else if constexpr (BFMT == 1) {
        v = as_u32x4(dequant8_i8(rb[i].v[0], rb[i].v[1], rowScale[i]));
      } else {
        const int k = k0 + bC[i] * 8;
        const long gi = (long)bRow[i] * (K / group) + k / group;
        v = as_u32x4(dequant8_u8(rb[i].v[0], rb[i].v[1], zero[gi], scale[gi]));
      }
      *reinterpret_cast<u32x4*>(b + sBoff[i]) = v;
    }
  };

  typename MF::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < MF::NACC; ++v) acc[i][j][v] = 0.f;

  // fragment read offsets (row part) inside one stage
  const int fr = lane % MS;
  const int fk = lane / MS;  // k-group of this lane
  int aRow[TM], bRowF[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) aRow[i] = wm * Cfg::WTM + i * MS + fr;
#pragma unroll
  for (int j = 0; j < TN; ++j) bRowF[j] = wn * Cfg::WTN + j * MS + fr;

  const int NT = K / BK;
  load_stage(0);
  store_stage(0, 0);
  __syncthreads();

  for (int kt = 0; kt < NT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < NT) load_stage((kt + 1) * BK);
    const _Float16* a = sA + cur * BM * BK;
    const _Float16* b = sB + cur * BN * BK;
#pragma unroll
    for (int ks = 0; ks < Cfg::KS; ++ks) {
      const int chunk = ks * (64 / MS) + fk;
      f16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const f16x8*>(a + aRow[i] * BK +
                                                lds_chunk<BK, SWZ>(aRow[i], chunk) * 8);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const f16x8*>(b + bRowF[j] * BK +
                                                lds_chunk<BK, SWZ>(bRowF[j], chunk) * 8);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(fb[j], fa[i], acc[i][j]);
    }
    if (kt + 1 < NT) store_stage(cur ^ 1, (kt + 1) * BK);
    __syncthreads();
  }

  // ---- epilogue: each lane owns 4 consecutive n of one m per result group ----------------
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * Cfg::WTM + i * MS + (lane % MS);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int g = 0; g < MF::GROUPS; ++g) {
        const int n = n0 + wn * Cfg::WTN + j * MS + mfma_out_row<MS>(lane, g, 0);
        f16x4 o;
        o[0] = (_Float16)acc[i][j][4 * g + 0];
        o[1] = (_Float16)acc[i][j][4 * g + 1];
        o[2] = (_Float16)acc[i][j][4 * g + 2];
        o[3] = (_Float16)acc[i][j][4 * g + 3];
        *reinterpret_cast<f16x4*>(C + (long)m * ldc + n) = o;
      }
    }
  }
}

// ============================================================================================
// k_gemm_dma -- fp16 B only.  Same tile, swizzle and epilogue as k_gemm, but the global -> LDS
// copy is the gfx950 LDS-DMA load (global_load_lds_dwordx4): data goes straight from L2 into
// LDS without passing through registers, the copy costs one instruction per 1 KiB per wave, and
// STAGES-1 k-tiles are in flight while one is computed.
//
// One DMA instruction fills a contiguous 1 KiB of LDS, lane l writing bytes [16l, 16l+16).  The
// swizzle is therefore applied on the GLOBAL side: lane l fetches the chunk that belongs at LDS
// slot l.  Waits are explicit (s_waitcnt vmcnt(N) for this wave's own copies, then s_barrier
// for everyone's); the compiler does not order LDS reads after LDS-DMA writes by itself.
// ============================================================================================
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt vmcnt(N) lgkmcnt(0).  gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4,
// lgkmcnt bits 11:8, vmcnt[5:4] bits 15:14.
template <int N>
__device__ __forceinline__ void s_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

// 16-byte-per-lane buffer load into LDS: lane l's 16 bytes at byte offset voff + soff of the
// raw buffer [base, base + nrec) land at lds + 16 l.  (A helper function rather than inline in
// the kernel's lambdas: inside a lambda of a kernel template the host pass drops the kernel's
// launch stub.)
__device__ __forceinline__ void buf_lds16(const void* base, int nrec, void* lds, int voff, int soff) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nrec, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}
// The same with 1- or 2-byte lanes (zero-points, scales); such lanes land 4 bytes apart in LDS.
template <int SIZE>
__device__ __forceinline__ void buf_lds_n(const void* base, int nrec, void* lds, int voff, int soff) {
  static_assert(SIZE == 1 || SIZE == 2, "byte or half lanes");
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nrec, 0x00020000);
  if constexpr (SIZE == 1)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 1, voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 2, voff, soff, 0, 0);
}

// XT = 1 pipelines across k-tile boundaries: the wait + barrier for tile kt+1, the DMA issue of
// tile kt+STAGES and the first fragment reads of tile kt+1 all happen BEFORE the last MFMA group
// of tile kt, so the matrix cores have work while the workgroup synchronises.  The prologue then
// fills all STAGES buffers.  XT = 0 keeps the plain loop (wait + barrier at the top of a tile).
// MINB = workgroups the compiler must leave room for on one CU (register budget 512 / waves per
// SIMD); 2 lets two small-tile workgroups share a CU, so one computes while the other waits.
// MS = MFMA shape (32: v_mfma_f32_32x32x16_f16, 16: v_mfma_f32_16x16x32_f16).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int SWZ, int GROUP, int XCD,
          int XT = 0, int MINB = 1, int MS = 32>
__global__ __launch_bounds__(WM * WN * 64, MINB) void k_gemm_dma(
    const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C,
    int M, int N, int K, int lda, int ldb, int ldc) {
  using MF = Mfma<MS>;
  constexpr int NW = WM * WN;
  constexpr int CPR = BK / 8;
  constexpr int RPB = 1024 / (BK * 2);  // tile rows per 1 KiB DMA block
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / MS, TN = WTN / MS;
  constexpr int KS = BK / MF::KSTEP;
  constexpr int A_BLK = BM / RPB / NW;  // DMA instructions per wave per stage
  constexpr int B_BLK = BN / RPB / NW;
  constexpr int L = A_BLK + B_BLK;
  constexpr int STAGE_ELEMS = (BM + BN) * BK;
  static_assert(BM % (RPB * NW) == 0 && BN % (RPB * NW) == 0, "DMA blocks per wave");
  static_assert(STAGES >= 2 && (STAGES - 2 + XT) * L < 64, "stages / vmcnt range");
  static_assert(WTM % MS == 0 && WTN % MS == 0 && BK % MF::KSTEP == 0, "tile shape");

  __shared__ __attribute__((aligned(1024))) _Float16 smem[STAGES * STAGE_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  const int nm = (M + BM - 1) / BM, nn = N / BN;
  int tmi, tni;
  tile_of<GROUP, XCD>(blockIdx.x, nm, nn, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;

  // per-lane global sources: DMA block i of this wave = tile block (i*NW + wave)
  const _Float16* srcA[A_BLK];
  const _Float16* srcB[B_BLK];
  {
    const int rin = lane / CPR, phys = lane % CPR;
#pragma unroll
    for (int i = 0; i < A_BLK; ++i) {
      const int row = (i * NW + wave) * RPB + rin;
      const int c = lds_chunk<BK, SWZ>(row, phys);  // involution: logical chunk of slot `phys`
      srcA[i] = A + (long)min(m0 + row, M - 1) * lda + c * 8;
    }
#pragma unroll
    for (int i = 0; i < B_BLK; ++i) {
      const int row = (i * NW + wave) * RPB + rin;
      const int c = lds_chunk<BK, SWZ>(row, phys);
      srcB[i] = B + (long)(n0 + row) * ldb + c * 8;
    }
  }
  auto issue = [&](int kt) {
    const int st = kt % STAGES;
    _Float16* sa = smem + st * STAGE_ELEMS;
    _Float16* sb = sa + BM * BK;
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_BLK; ++i)
      __builtin_amdgcn_global_load_lds((void*)(srcA[i] + k0),
                                       (lds_void_t*)(sa + (i * NW + wave) * RPB * BK), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < B_BLK; ++i)
      __builtin_amdgcn_global_load_lds((void*)(srcB[i] + k0),
                                       (lds_void_t*)(sb + (i * NW + wave) * RPB * BK), 16, 0, 0);
  };

  typename MF::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < MF::NACC; ++v) acc[i][j][v] = 0.f;

  const int fr = lane % MS, fk = lane / MS;
  int aOff[TM], bOff[TN];  // row offsets (elements) of this lane's fragment rows
#pragma unroll
  for (int i = 0; i < TM; ++i) aOff[i] = (wm * WTM + i * MS + fr);
#pragma unroll
  for (int j = 0; j < TN; ++j) bOff[j] = (wn * WTN + j * MS + fr);

  const int NT = K / BK;
  if constexpr (XT) {
    f16x8 fa[2][TM], fb[2][TN];
    auto read = [&](auto bufc, const _Float16* a, int ks) {
      constexpr int bb = decltype(bufc)::value;
      const _Float16* b = a + BM * BK;
      const int chunk = ks * (64 / MS) + fk;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[bb][i] = *reinterpret_cast<const f16x8*>(a + aOff[i] * BK +
                                                    lds_chunk<BK, SWZ>(aOff[i], chunk) * 8);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[bb][j] = *reinterpret_cast<const f16x8*>(b + bOff[j] * BK +
                                                    lds_chunk<BK, SWZ>(bOff[j], chunk) * 8);
    };
    auto mma = [&](auto bufc) {
      constexpr int bb = decltype(bufc)::value;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(fb[bb][j], fa[bb][i], acc[i][j]);
    };
    static_assert(KS % 2 == 0, "fragment buffers alternate; a tile holds an even k-step count");
    // prologue: every buffer gets a tile; wait for tile 0 (tiles 1..STAGES-1 stay in flight)
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (s < NT) issue(s);
    asm volatile("" ::: "memory");
    if (NT >= STAGES) s_wait_vm<(STAGES - 1) * L>();
    else s_wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read(IC<0>{}, smem, 0);
    __builtin_amdgcn_sched_barrier(0);
    for (int kt = 0; kt < NT; ++kt) {
      const _Float16* a = smem + (kt % STAGES) * STAGE_ELEMS;
#pragma unroll
      for (int ks = 0; ks < KS - 2; ks += 2) {
        read(IC<1>{}, a, ks + 1);
        mma(IC<0>{});
        __builtin_amdgcn_sched_barrier(0);
        read(IC<0>{}, a, ks + 2);
        mma(IC<1>{});
        __builtin_amdgcn_sched_barrier(0);
      }
      read(IC<1>{}, a, KS - 1);
      mma(IC<0>{});
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < NT) {
        // Tile kt+1 has landed for this wave (tiles up to kt+STAGES-1 may still be in flight)
        // and this wave's reads of tile kt are complete (lgkmcnt 0) ...
        asm volatile("" ::: "memory");
        if (kt + STAGES < NT) s_wait_vm<(STAGES - 2) * L>();
        else s_wait_vm<0>();
        // ... and everyone's: tile kt+1 is readable and buffer kt % STAGES is free.
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + STAGES < NT) issue(kt + STAGES);
        read(IC<0>{}, smem + ((kt + 1) % STAGES) * STAGE_ELEMS, 0);
      }
      mma(IC<1>{});
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < NT) issue(s);

  for (int kt = 0; kt < NT; ++kt) {
    // this wave's copies of tile kt have landed (later tiles may still be in flight) ...
    asm volatile("" ::: "memory");  // compiler-only fence: no LDS access crosses the barrier
    if (kt + STAGES - 2 < NT) s_wait_vm<(STAGES - 2) * L>();
    else s_wait_vm<0>();
    // ... and everyone's have; everyone is also done reading the buffer about to be refilled
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + STAGES - 1 < NT) issue(kt + STAGES - 1);

    const _Float16* a = smem + (kt % STAGES) * STAGE_ELEMS;
    const _Float16* b = a + BM * BK;
    f16x8 fa[2][TM], fb[2][TN];
    auto read = [&](auto bufc, int ks) {
      constexpr int bb = decltype(bufc)::value;
      const int chunk = ks * (64 / MS) + fk;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[bb][i] = *reinterpret_cast<const f16x8*>(a + aOff[i] * BK +
                                                    lds_chunk<BK, SWZ>(aOff[i], chunk) * 8);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[bb][j] = *reinterpret_cast<const f16x8*>(b + bOff[j] * BK +
                                                    lds_chunk<BK, SWZ>(bOff[j], chunk) * 8);
    };
    auto mma = [&](auto bufc) {
      constexpr int bb = decltype(bufc)::value;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(fb[bb][j], fa[bb][i], acc[i][j]);
    };
    // Fragment double buffer: the reads of step ks+1 are issued before the 16 MFMAs of step ks
    // and the scheduler is not allowed to sink them (sched_barrier), so LDS latency hides
    // under the matrix-core work instead of stalling every few MFMAs.
    read(IC<0>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS; ks += 2) {
      if (ks + 1 < KS) read(IC<1>{}, ks + 1);
      mma(IC<0>{});
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 2 < KS) read(IC<0>{}, ks + 2);
      if (ks + 1 < KS) mma(IC<1>{});
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  }

  // ---- epilogue: each lane owns 4 consecutive n of one m per result group ----------------
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * MS + (lane % MS);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int g = 0; g < MF::GROUPS; ++g) {
        const int n = n0 + wn * WTN + j * MS + mfma_out_row<MS>(lane, g, 0);
        f16x4 o;
        o[0] = (_Float16)acc[i][j][4 * g + 0];
        o[1] = (_Float16)acc[i][j][4 * g + 1];
        o[2] = (_Float16)acc[i][j][4 * g + 2];
        o[3] = (_Float16)acc[i][j][4 * g + 3];
        *reinterpret_cast<f16x4*>(C + (long)m * ldc + n) = o;
      }
    }
  }
}
