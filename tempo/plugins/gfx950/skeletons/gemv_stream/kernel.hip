// gemv_stream -- the small-M (decode) regime of C[M,N] = A[M,K] . deq(B)[N,K]^T on gfx950.
//
// At M <= 32 the operation is bound by reading B once from HBM (2MNK flops against NK or 2NK
// bytes).  The kernel therefore streams B exactly once with 16-byte loads, dequantises in
// registers (formats 1 and 2, bit-exact closed forms in cdna4.h) and feeds the values straight
// into v_mfma_f32_16x16x32_f16 -- the weight rows are the MFMA "A" operand (16 rows per
// instruction), the activation rows the "B" operand (16 columns, padded past M).  The matrix
// cores are >20x over-provisioned here; what they save is the VALU time a dot-product path
// would spend on 2MNK multiply-adds, leaving the VALU to the dequantisation alone.
//
// Work unit = one wave: R groups of 16 weight rows x one K chunk.  A workgroup holds 4 units.
// With S > 1 chunks per row slab the units write fp32 partials to a workspace and the last
// unit to finish a slab (counted with an atomic per slab) sums the S partials in chunk order
// 0..S-1 -- so the result does not depend on arrival order -- writes fp16 C and re-arms the
// counter to zero for the next call.
//
// Template axes: MB (16-column blocks of M: M <= 16*MB), R (row groups per wave), U (k-steps
// of 64 loaded per pipeline stage), BFMT (0 fp16, 1 int8 + row scale, 2 uint8 + group scale
// and zero-point, group 128).
//
// k order inside one 64-step: lane (row r = l%16, kgroup g = l/16) owns the 16 consecutive
// k-values [16g, 16g+16) of its row; the first MFMA takes elements 0..7, the second 8..15.
// The activation fragment uses the same map, so each product pairs equal k.

struct StreamArgs {
  const _Float16* A;   // [M][lda]
  const void* B;       // [N][ldb] fp16 / int8 / uint8
  const _Float16* scale;
  const uint8_t* zero;
  _Float16* C;         // [M][ldc]
  float* ws;           // [S][M][N] fp32 partials (S > 1 only)
  unsigned* counters;  // [N / (16R)] arrival counters, zero between calls (S > 1 only)
  int M, N, K, lda, ldb, ldc;
  int S;               // k chunks per slab
  int chunk;           // k per chunk (multiple of 64*U, except the last chunk)
  int group;           // k per scale group (fmt 2)
};

template <int BFMT>
struct WRaw;  // per lane, per row group, per 64-step: the 16 k-values of its row
template <>
struct WRaw<0> { u32x4 v[2]; };  // 32 bytes fp16
template <>
struct WRaw<1> { u32x4 v; };     // 16 bytes int8
template <>
struct WRaw<2> { u32x4 v; };     // 16 bytes uint8

template <int MB, int R, int U, int BFMT>
__global__ __launch_bounds__(256) void k_stream(StreamArgs p) {
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int slabs = p.N / (16 * R);
  if (unit >= slabs * p.S) return;  // whole-wave exit: no barrier in this kernel
  const int slab = unit / p.S;
  const int split = unit - slab * p.S;
  const int kbeg = split * p.chunk;
  const int kend = min(p.K, kbeg + p.chunk);

  const int r16 = lane & 15;  // row within a 16-row group / column within a 16-col block
  const int kg = lane >> 4;   // k-group 0..3
  const int nbase = slab * 16 * R;

  // weight row pointers
  const uint8_t* wrow[R];
  _Float16 rscale[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long n = nbase + r * 16 + r16;
    constexpr int EB = BFMT == 0 ? 2 : 1;
    wrow[r] = reinterpret_cast<const uint8_t*>(p.B) + (n * p.ldb + 16 * kg) * EB;
    if constexpr (BFMT == 1) rscale[r] = p.scale[n];
  }
  // activation row pointers (rows past M read row M-1; their results are never stored)
  const _Float16* arow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int m = min(b * 16 + r16, p.M - 1);
    arow[b] = p.A + (long)m * p.lda + 16 * kg;
  }

  f32x4 acc[R][MB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[r][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  WRaw<BFMT> w[2][U][R];
  u32x4 a[2][U][MB][2];

  auto issue = [&](auto bufc, int k0) {
    constexpr int buf = decltype(bufc)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + 64 * u;
      const bool live = k < kend;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (BFMT == 0) {
          const u32x4* q = reinterpret_cast<const u32x4*>(wrow[r] + (long)k * 2);
          if (live) { w[buf][u][r].v[0] = q[0]; w[buf][u][r].v[1] = q[1]; }
        } else {
          const u32x4* q = reinterpret_cast<const u32x4*>(wrow[r] + k);
          if (live) w[buf][u][r].v = q[0];
        }
      }
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const u32x4* q = reinterpret_cast<const u32x4*>(arow[b] + k);
        if (live) { a[buf][u][b][0] = q[0]; a[buf][u][b][1] = q[1]; }
      }
    }
  };

  auto compute = [&](auto bufc, int k0) {
    constexpr int buf = decltype(bufc)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + 64 * u;
      if (k >= kend) break;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        f16x8 w0, w1;
        if constexpr (BFMT == 0) {
          w0 = as_f16x8(w[buf][u][r].v[0]);
          w1 = as_f16x8(w[buf][u][r].v[1]);
        } else if constexpr (BFMT == 1) {
          const u32x4 q = w[buf][u][r].v;
          w0 = dequant8_i8(q[0], q[1], rscale[r]);
          w1 = dequant8_i8(q[2], q[3], rscale[r]);
        } else {
          const u32x4 q = w[buf][u][r].v;
          const long n = nbase + r * 16 + r16;
          const long gi = n * (p.K / p.group) + (k + 16 * kg) / p.group;
          const uint8_t z = p.zero[gi];
          const _Float16 s = p.scale[gi];
          w0 = dequant8_u8(q[0], q[1], z, s);
          w1 = dequant8_u8(q[2], q[3], z, s);
        }
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          acc[r][b] = Mfma<16>::run(w0, as_f16x8(a[buf][u][b][0]), acc[r][b]);
          acc[r][b] = Mfma<16>::run(w1, as_f16x8(a[buf][u][b][1]), acc[r][b]);
        }
      }
    }
  };

  // two-stage register pipeline: loads of stage s+1 are in flight while stage s computes.
  // The loop is unrolled by two so every register-array index is a compile-time constant.
  constexpr int STEP = 64 * U;
  int k0 = kbeg;
  issue(IC<0>{}, k0);
  while (true) {
    if (k0 + STEP < kend) issue(IC<1>{}, k0 + STEP);
    compute(IC<0>{}, k0);
    k0 += STEP;
    if (k0 >= kend) break;
    if (k0 + STEP < kend) issue(IC<0>{}, k0 + STEP);
    compute(IC<1>{}, k0);
    k0 += STEP;
    if (k0 >= kend) break;
  }

  // ---- result: lane holds C[m = b*16 + r16][n = nbase + r*16 + 4*kg + v], v = 0..3 ----------
  if (p.S == 1) {
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = b * 16 + r16;
      if (m >= p.M) continue;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = nbase + r * 16 + 4 * kg;
        f16x4 o;
        o[0] = (_Float16)acc[r][b][0];
        o[1] = (_Float16)acc[r][b][1];
        o[2] = (_Float16)acc[r][b][2];
        o[3] = (_Float16)acc[r][b][3];
        *reinterpret_cast<f16x4*>(p.C + (long)m * p.ldc + n) = o;
      }
    }
    return;
  }

  // split-K: publish this chunk's partial, then the last arrival reduces the slab.
  const long plane = (long)p.M * p.N;
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int m = b * 16 + r16;
    if (m >= p.M) continue;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = nbase + r * 16 + 4 * kg;
      *reinterpret_cast<f32x4*>(p.ws + split * plane + (long)m * p.N + n) = acc[r][b];
    }
  }
  __threadfence();
  unsigned prev = 0;
  if (lane == 0) prev = atomicAdd(p.counters + slab, 1u);
  prev = __shfl(prev, 0);
  if (prev != (unsigned)(p.S - 1)) return;
  __threadfence();
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int m = b * 16 + r16;
    if (m >= p.M) continue;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = nbase + r * 16 + 4 * kg;
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < p.S; ++sp) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p.ws + sp * plane + (long)m * p.N + n);
        s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
      }
      f16x4 o;
      o[0] = (_Float16)s[0];
      o[1] = (_Float16)s[1];
      o[2] = (_Float16)s[2];
      o[3] = (_Float16)s[3];
      *reinterpret_cast<f16x4*>(p.C + (long)m * p.ldc + n) = o;
    }
  }
  if (lane == 0) p.counters[slab] = 0u;  // re-arm for the next call on this workspace
}

// Debug/verification entry: dequantise a [rows x cols] tile of B starting at (n0, k0) with the
// same device functions the GEMM feeds use, writing fp16 [rows][cols].  cols % 8 == 0.
template <int BFMT>
__global__ void k_dequant_tile(StreamArgs p, int n0, int k0, int rows, int cols, _Float16* out) {
  const int per_row = cols / 8;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int r = idx / per_row, c8 = idx - r * per_row;
  const long n = n0 + r;
  const long k = k0 + c8 * 8;
  f16x8 v;
  if constexpr (BFMT == 1) {
    const u32x2 q = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(p.B) +
                                                    n * p.ldb + k);
    v = dequant8_i8(q[0], q[1], p.scale[n]);
  } else {
    const u32x2 q = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(p.B) +
                                                    n * p.ldb + k);
    const long gi = n * (p.K / p.group) + k / p.group;
    v = dequant8_u8(q[0], q[1], p.zero[gi], p.scale[gi]);
  }
  *reinterpret_cast<f16x8*>(out + (long)r * cols + c8 * 8) = v;
}
