// gemv_stream/phase.hip -- the phase-ordered decode kernel of the W8A16 delivery.  Uses the
// copy vocabulary of gemv_stream/kernel.hip (lds_void_stream_t, s_wait_vm_stream, line_key) and
// the dequantisation of common/cdna4.h.
// ============================================================================================
// k_stream_phase -- the decode kernel with the k loop outside the slab loop (wide N, M <= 32).
//
// One workgroup per CU (256 of them), 8 waves; workgroup b owns the weight rows [b rwg, (b+1) rwg)
// with rwg = N / 256 (a multiple of 4): NS - 1 slabs of 16 rows and a last slab of 4 .. 16.  Wave w
// owns the k chunk [1024 w / 8 ... ) = K / 8 (a multiple of 128: SPC steps of 128 k).  The wave
// walks its chunk phase by phase (a phase = one 128-k step) and, inside a phase, the NS slabs:
// step (s, sl) is 16 rows x 128 bytes of slab sl at k step s, copied HBM -> LDS by two whole-line
// LDS-DMA copies (the line kernel's copy map and chunk swizzle) into a private ring of D slots.
// The point of the order: a phase needs the activations of ONE 128-k step (16 MB registers per
// lane), which travel by LDS-DMA into a per-wave staging slot during the phase before and are
// read into registers at the phase's first step -- so the activations ride the weight stream a
// phase ahead instead of being fetched up front, the ring carries weights only, and the
// activation registers do not grow with K.  Each slab keeps its own accumulators for the whole
// chunk (NS x MB f32x4 per lane).  At the end the 8 chunk partial sums of each slab are added
// through LDS in chunk order (one slab per round, one wave per slab), written as fp16 into an
// LDS image of the workgroup's output columns, and stored row by row.
// Activations: MB = 1 / 2 (M <= 16 / 32): lane l's 16 bytes of row 16 mb + l % 16 (rows past M
// re-read row M-1) per copy, four copies per 16 rows, a phase ahead; MB = 0 (M = 1): every
// phase's 256-byte slice of row 0 (one dword copy each) staged before the first step, read by
// broadcast.  Metadata (fmt 1 row scales; fmt 2 zero-points and scales of the workgroup's rows,
// all groups) are staged in LDS once, by 4-byte LDS-DMA pieces of their contiguous blocks,
// before the first step.  Rows of the last slab past the workgroup's rows (and copies past the
// chunk's end) fetch a dummy line of A, an L2 hit, into slots whose results nobody stores.
// Waits: every step issues its two weight copies, so "step u has landed" is vmcnt((D-1) * 2),
// plus (MB > 0) the phase's activation copies (4 MB) when they were issued after step u's copies
// (the steps 1 .. D-1 of every phase but the last).  The slab loop is unrolled (the waits are
// compile-time per step) and the phase loop is not; with MB > 0 the last phase (no next
// activations) is peeled.  Requirements (launcher): N % 256 == 0, N / 256 % 4 == 0 with
// NS = ceil(N / 256 / 16) (>= D when MB > 0), K % 1024 == 0, 16-byte aligned A and Wq, 4-byte
// aligned scale and zero, and (fmt 2) group 128.
// EPI = 1 (fused gate/up; p.N below is the output width, W holds the gate rows then, from row
// `up`, the up rows): workgroup b owns the output columns [b cwg, (b+1) cwg) with cwg = N / 256
// (a multiple of 4), and its rwg = 2 cwg rows are cwg gate rows followed by the cwg matching up
// rows -- a lane picks its row's source by which half it falls in.  The output image then holds
// the fp16 gate and up results side by side, and the store writes fp16_rn(silu(g) * u).
// KSL = 1 (k slices across workgroups, plain epilogue): the 256 workgroups are ks slices of K
// times 256 / ks row groups (N / (256 / ks) rows each); a workgroup's K / ks k (its `steps`
// 128-k steps) split over the 8 waves as evenly as whole steps allow (the waves run their phases
// independently; only the final reduction syncs them).  fmt 2 metadata: the slice's groups of the
// workgroup's rows, one byte / one half per (row, group), 4 bytes apart (sub-dword LDS-DMA).  The
// slice's fp32 sum of each output goes to part[slice][m][n]; a second kernel adds the slices in
// order (k_splitk_reduce).
// ============================================================================================
struct PhaseArgs {
  const _Float16* A;
  const uint8_t* B;
  const _Float16* scale;
  const uint8_t* zero;
  _Float16* C;
  int M, K, lda, ldb, ldc;
  int rwg;   // weight rows per workgroup (N / 256; EPI: 2 cwg)
  int cwg;   // output columns per workgroup (rwg; EPI: N / 256)
  long up;   // EPI: first row of the up half of W (the output width N)
  int G;     // groups of 128 k per row (K / 128)
  int steps; // 128-k steps of a workgroup's k range (K / 128 / ks)
  int ks;    // KSL: k slices across workgroups
  int N;     // KSL: row pitch of the partial sums
  float* part;  // KSL: fp32 partial sums [ks][M][N]
  int stg_off, out_off, meta_off, meta_s_off;  // LDS byte offsets
};

template <int B, int E, class F>
__device__ __forceinline__ void unroll_for(F&& f) {
  if constexpr (B < E) {
    f(IC<B>{});
    unroll_for<B + 1, E>(f);
  }
}

template <int MB, int NS, int D, int BFMT, int EPI = 0, int KSL = 0>
struct StreamPhase {
  static constexpr int NWV = 8;                  // waves = k chunks per workgroup
  static constexpr int L = 2;                    // weight copies per step
  static constexpr int MBE = MB > 0 ? MB : 1;    // 16-column blocks of the result
  static constexpr int LA = MB > 0 ? 4 * MB : 1; // activation copies per phase
  static constexpr int SLOT = 2048;              // one ring slot: 16 rows x 128 bytes
  static constexpr int CUS = 256;                // workgroups: one per CU of the part
  static_assert((MB == 0 || NS >= D) && D >= 2 && (D - 1) * L + LA < 64,
                "ring depth / vmcnt range");
  static_assert(!(EPI && KSL), "k slices take the plain epilogue");
  // activation staging per wave: one phase's copies (MB > 0), every phase's slice (MB = 0) --
  // S = the workgroup's 128-k steps, at most ceil(S / NWV) per wave
  static constexpr int stg_wave(int S) { return MB > 0 ? LA * 1024 : (S + NWV - 1) / NWV * 256; }
  // vmcnt of "step (s, sl) landed": LAST = the phase issues no next activations
  static constexpr int wait_of(int sl, bool last) {
    return (D - 1) * L + (MB > 0 && !last && sl > 0 && sl < D ? LA : 0);
  }
  // LDS layout (bytes): rings, activation staging (after the loop: the chunk partial sums), the
  // output image, metadata; -1 if it exceeds 160 KiB
  static constexpr int ring_bytes() { return NWV * D * SLOT; }
  static constexpr int stg_bytes(int S) {
    return NWV * stg_wave(S) > 2 * NWV * MBE * 1024 ? NWV * stg_wave(S) : 2 * NWV * MBE * 1024;
  }
  static constexpr int out_bytes() {
    return KSL ? 0 : (MBE * 16 * NS * 16 * 2 + 1023) / 1024 * 1024;
  }
  // metadata per row: whole K, packed (G bytes of z, G halves of s), or the slice's S groups,
  // 4 bytes apart each (KSL)
  static constexpr int meta_z_bytes(int G, int S) {
    return BFMT == 2 ? (NS * 16 * (KSL ? 4 * S : G) + 1023) / 1024 * 1024 : 0;
  }
  static constexpr int meta_s_bytes(int G, int S) {
    return ((BFMT == 2 ? NS * 16 * (KSL ? 4 * S : 2 * G) : NS * 32) + 1023) / 1024 * 1024;
  }
  static constexpr int lds(int G, int S) {
    return ring_bytes() + stg_bytes(S) + out_bytes() + meta_z_bytes(G, S) + meta_s_bytes(G, S);
  }
};

template <int MB, int NS, int D, int BFMT, int EPI = 0, int KSL = 0>
__global__ __launch_bounds__(512, 1) void k_stream_phase(PhaseArgs p) {
  using SP = StreamPhase<MB, NS, D, BFMT, EPI, KSL>;
  constexpr int NWV = SP::NWV, L = SP::L, LA = SP::LA, SLOT = SP::SLOT, MBE = SP::MBE;
  constexpr int NSX = NS * 16;  // output image row length (columns)
  extern __shared__ __attribute__((aligned(1024))) uint8_t dsm[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kg = lane >> 4;
  const int rwg = p.rwg, cwg = p.cwg, S = p.steps;
  const int groups = KSL ? SP::CUS / p.ks : SP::CUS;       // row groups
  const int rg = (int)blockIdx.x % groups, slice = (int)blockIdx.x / groups;
  const long row0 = (long)rg * cwg;  // first row (EPI: of the gate half)
  // this wave's steps of the workgroup's S: as even as whole steps allow
  const int sbase = S / NWV, sextra = S - sbase * NWV;
  const int spc = sbase + (wave < sextra ? 1 : 0);
  const int first = wave * sbase + (wave < sextra ? wave : sextra);
  const int kbeg = (slice * S + first) * 128;
  uint8_t* ring = dsm + wave * D * SLOT;
  uint8_t* stg = dsm + p.stg_off + wave * SP::stg_wave(S);
  f32x4* red = reinterpret_cast<f32x4*>(dsm + p.stg_off);  // after the loop: [2][NWV][MBE][64]
  _Float16* outl = reinterpret_cast<_Float16*>(dsm + p.out_off);
  const uint8_t* meta_z = dsm + p.meta_off;
  const _Float16* meta_s = reinterpret_cast<const _Float16*>(dsm + p.meta_s_off);
  const uint8_t* dummy = reinterpret_cast<const uint8_t*>(p.A) + 16 * lane;  // 1 KiB of A (L2)

  // metadata blocks of the workgroup's rows, 256-byte pieces (a dword per lane) over the waves
  auto copy_block = [&](uint8_t* dst, const uint8_t* src, int bytes) {
    for (int pc = wave; pc * 256 < bytes; pc += NWV) {
      const int off = pc * 256 + 4 * lane;
      if (off < bytes)
        __builtin_amdgcn_global_load_lds((void*)(src + off), (lds_void_stream_t*)(dst + pc * 256),
                                         4, 0, 0);
    }
  };
  // (EPI: the gate block, then the up block behind it, in the rows' workgroup order)
  if constexpr (KSL && BFMT == 2) {
    // the slice's groups of each row: (row r, group j) at 4 (r S + j), byte / half copies
    const int tot = rwg * S;
    for (int pc = wave; pc * 64 < tot; pc += NWV) {
      const int i = pc * 64 + lane;
      if (i < tot) {
        const int r = i / S, j = i - r * S;
        const long gi = (row0 + r) * p.G + slice * S + j;
        __builtin_amdgcn_global_load_lds((void*)(p.zero + gi), (lds_void_stream_t*)(dsm + p.meta_off + pc * 256),
                                         1, 0, 0);
        __builtin_amdgcn_global_load_lds((void*)(p.scale + gi),
                                         (lds_void_stream_t*)(dsm + p.meta_s_off + pc * 256), 2, 0, 0);
      }
    }
  } else {
#pragma unroll
    for (int half = 0; half < 1 + EPI; ++half) {
      const long r = row0 + half * p.up;
      if constexpr (BFMT == 1) {
        copy_block(dsm + p.meta_s_off + half * cwg * 2,
                   reinterpret_cast<const uint8_t*>(p.scale + r), cwg * 2);
      } else {
        copy_block(dsm + p.meta_off + half * cwg * p.G, p.zero + r * p.G, cwg * p.G);
        copy_block(dsm + p.meta_s_off + half * cwg * 2 * p.G,
                   reinterpret_cast<const uint8_t*>(p.scale + r * p.G), cwg * 2 * p.G);
      }
    }
  }
  // activation copies of phase s: copy (mb, h, q) carries lane l's 16 bytes -- row 16 mb + l % 16,
  // k kbeg + 128 s + 64 h + 16 (l / 16) + 8 q -- read back by the same lane; MB = 0: one dword per
  // lane of row 0's 256-byte slice
  const _Float16* arow[MBE];
#pragma unroll
  for (int mb = 0; mb < MBE; ++mb)
    arow[mb] = MB == 0 ? p.A + kbeg + 2 * lane
                       : p.A + (long)min(16 * mb + r16, p.M - 1) * p.lda + kbeg + 16 * kg;
  auto dma_act = [&](int s) {
    if constexpr (MB == 0) {  // phase s's slice into its own staging slot
      __builtin_amdgcn_global_load_lds((void*)(arow[0] + 128 * s), (lds_void_stream_t*)(stg + 256 * s),
                                       4, 0, 0);
    } else {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            __builtin_amdgcn_global_load_lds(
                (void*)(arow[mb] + 128 * s + 64 * h + 8 * q),
                (lds_void_stream_t*)(stg + ((mb * 2 + h) * 2 + q) * 1024), 16, 0, 0);
    }
  };
  // weight copy i of a step fills rows 8i .. 8i+7: lane l row 8i + l/8, physical chunk l%8 =
  // logical chunk (l%8) ^ key(row); a lane whose row of the last slab lies past the workgroup's
  // rows fetches the dummy line instead
  const uint8_t* wsrc[2];
  const uint8_t* wsrc_up[2];  // EPI: rows of the up half (workgroup row v >= cwg)
  int wrow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    wrow[i] = 8 * i + lane / 8;
    const int c = (lane % 8) ^ line_key(wrow[i]);
    wsrc[i] = p.B + (row0 + wrow[i]) * p.ldb + kbeg + c * 16;
    wsrc_up[i] = EPI ? p.B + (p.up + row0 + wrow[i] - cwg) * p.ldb + kbeg + c * 16 : wsrc[i];
  }
  const long slab_stride = 16L * p.ldb;
  // copies of step (s, sl) into ring slot `slot`; past = beyond the chunk's last step.  One copy
  // instruction per half whatever its source (a selected address, no branch: copies in a branch
  // make the compiler wait for every copy in flight where the paths merge)
  auto dma_w = [&](int s, int sl, int slot, bool past) {
    uint8_t* dst = ring + slot * SLOT;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bool real = !past && (sl < NS - 1 || 16 * sl + wrow[i] < rwg);
      const uint8_t* base = EPI && 16 * sl + wrow[i] >= cwg ? wsrc_up[i] : wsrc[i];
      const uint8_t* src = real ? base + sl * slab_stride + s * 128 : dummy;
      __builtin_amdgcn_global_load_lds((void*)src, (lds_void_stream_t*)(dst + i * 1024), 16, 0,
                                       2 /* nt */);
    }
  };

  if constexpr (MB == 0) {
    for (int s = 0; s < spc; ++s) dma_act(s);
  } else {
    dma_act(0);
  }
  unroll_for<0, D>([&](auto uc) {  // the first D steps (MB > 0: NS >= D, all of phase 0)
    constexpr int u = decltype(uc)::value;
    dma_w(u / NS, u % NS, u % D, u / NS >= spc);
  });
  asm volatile("" ::: "memory");
  s_wait_vm_stream<(D - 1) * L>();  // metadata, the first activations and step 0 have landed
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();     // ... in every wave: the metadata pieces are all in
  asm volatile("" ::: "memory");

  const int key = line_key(r16);
  const int g0 = KSL ? first : kbeg / 128;  // the wave's first group in the staged metadata
  f32x4 acc[NS][MBE];
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
#pragma unroll
    for (int mb = 0; mb < MBE; ++mb) acc[sl][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 a[MBE][2][2];

  // one phase: the NS steps of k step s (ring slot of step (s, sl) = (s NS + sl) % D)
  auto phase = [&](int s, auto lastc) {
    constexpr bool LAST = decltype(lastc)::value;
    const int ub = s * NS;
    unroll_for<0, NS>([&](auto slc) {
      constexpr int sl = decltype(slc)::value;
      asm volatile("" ::: "memory");
      s_wait_vm_stream<SP::wait_of(sl, LAST)>();  // step (s, sl) landed (sl = 0: and phase s's
      asm volatile("" ::: "memory");              // activations)
      if constexpr (sl == 0) {
#pragma unroll
        for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q)
              a[mb][h][q] = MB == 0
                  ? *reinterpret_cast<const u32x4*>(stg + 256 * s + (64 * h + 16 * kg + 8 * q) * 2)
                  : *reinterpret_cast<const u32x4*>(stg + ((mb * 2 + h) * 2 + q) * 1024 + 16 * lane);
      }
      const uint8_t* slot = ring + ((ub + sl) % D) * SLOT;
      u32x4 w[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        w[h] = *reinterpret_cast<const u32x4*>(slot + r16 * 128 + (((4 * h + kg) ^ key) * 16));
      uint8_t z = 0;
      _Float16 scl;
      if constexpr (BFMT == 2 && KSL) {
        z = meta_z[4 * ((sl * 16 + r16) * S + g0 + s)];
        scl = meta_s[2 * ((sl * 16 + r16) * S + g0 + s)];
      } else if constexpr (BFMT == 2) {
        z = meta_z[(sl * 16 + r16) * p.G + g0 + s];
        scl = meta_s[(sl * 16 + r16) * p.G + g0 + s];
      } else {
        scl = meta_s[sl * 16 + r16];
      }
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot (and the staging) are read
      asm volatile("" ::: "memory");
      if constexpr (MB > 0 && sl == 0 && !LAST) dma_act(s + 1);
      {
        constexpr int nx = sl + D;  // step D ahead: (s + nx / NS, nx % NS)
        dma_w(s + nx / NS, nx % NS, (ub + nx) % D, s + nx / NS >= spc);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f16x8 w0, w1;
        if constexpr (BFMT == 1) {
          w0 = dequant8_i8(w[h][0], w[h][1], scl);
          w1 = dequant8_i8(w[h][2], w[h][3], scl);
        } else {
          w0 = dequant8_u8(w[h][0], w[h][1], z, scl);
          w1 = dequant8_u8(w[h][2], w[h][3], z, scl);
        }
#pragma unroll
        for (int mb = 0; mb < MBE; ++mb) {
          acc[sl][mb] = Mfma<16>::run(w0, as_f16x8(a[mb][h][0]), acc[sl][mb]);
          acc[sl][mb] = Mfma<16>::run(w1, as_f16x8(a[mb][h][1]), acc[sl][mb]);
        }
      }
    });
  };
  if constexpr (MB == 0) {  // every phase alike: no activation copies in the loop
    for (int s = 0; s < spc; ++s) phase(s, IC<1>{});
  } else {
    for (int s = 0; s < spc - 1; ++s) phase(s, IC<0>{});
    phase(spc - 1, IC<1>{});
  }

  s_wait_vm_stream<0>();  // the copies past the end have landed
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();  // every wave is past its staging reads: the partial sums reuse it
  asm volatile("" ::: "memory");
  // the 8 chunk partial sums of slab sl, added in chunk order by wave sl % 8 (double-buffered)
  unroll_for<0, NS>([&](auto slc) {
    constexpr int sl = decltype(slc)::value;
    constexpr int rb = sl & 1;
#pragma unroll
    for (int mb = 0; mb < MBE; ++mb) red[((rb * NWV + wave) * MBE + mb) * 64 + lane] = acc[sl][mb];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (wave == sl % NWV) {
#pragma unroll
      for (int mb = 0; mb < MBE; ++mb) {
        f32x4 t = red[((rb * NWV + 0) * MBE + mb) * 64 + lane];
#pragma unroll
        for (int c = 1; c < NWV; ++c) {
          const f32x4 v = red[((rb * NWV + c) * MBE + mb) * 64 + lane];
          t[0] += v[0];
          t[1] += v[1];
          t[2] += v[2];
          t[3] += v[3];
        }
        if constexpr (KSL) {  // the slice's fp32 sums, straight to the partials
          const int m = 16 * mb + r16, c = sl * 16 + 4 * kg;
          if (m < p.M && c < rwg)
            *reinterpret_cast<f32x4*>(p.part + ((long)slice * p.M + m) * p.N + row0 + c) = t;
        } else {
          f16x4 o;
          o[0] = (_Float16)t[0];
          o[1] = (_Float16)t[1];
          o[2] = (_Float16)t[2];
          o[3] = (_Float16)t[3];
          *reinterpret_cast<f16x4*>(outl + (16 * mb + r16) * NSX + sl * 16 + 4 * kg) = o;
        }
      }
    }
  });
  if constexpr (KSL) return;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // rows m < M of the workgroup's cwg output columns, 8 bytes per thread and pass (EPI: the
  // gate result of column c and the up result cwg columns further in the image)
  const int cpr = cwg / 4;
  for (int i = threadIdx.x; i < p.M * cpr; i += 64 * NWV) {
    const int m = i / cpr, c = i - m * cpr;
    u32x2 v = *reinterpret_cast<const u32x2*>(outl + m * NSX + 4 * c);
    if constexpr (EPI) {
      const f16x4 g = __builtin_bit_cast(f16x4, v);
      const f16x4 u = *reinterpret_cast<const f16x4*>(outl + m * NSX + cwg + 4 * c);
      f16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = silu_mul_f16((float)g[e], (float)u[e]);
      v = __builtin_bit_cast(u32x2, o);
    }
    *reinterpret_cast<u32x2*>(p.C + (long)m * p.ldc + row0 + 4 * c) = v;
  }
}
