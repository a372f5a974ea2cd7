// cdna4.h -- device vocabulary shared by the gfx950 skeletons (CDNA4, wave64, MFMA).
//
// The skeleton sources carry no namespace of their own: the freeze step that writes a shipped
// kernel file (kernels/shipped/<op>/gfx950/kernel.hip) and the plugin's render() wrap them in
// the op's namespace, so two shipped ops linked into one library never share a symbol.
//
// MFMA lane maps used below (wave64):
//   32x32x16 f16: operand lane l carries row (l % 32) and the 8 k-values of k-group (l / 32);
//                 result lane l carries column (l % 32), rows 8*(v/4) + 4*(l/32) + (v%4), v<16.
//   16x16x32 f16: operand lane l carries row (l % 16) and the 8 k-values of k-group (l / 16);
//                 result lane l carries column (l % 16), rows 4*(l/16) + v, v<4.
// The k-group -> k assignment only has to be the same for both operands (a sum over k does not
// care about its order), so the skeletons may permute k freely as long as A and B agree.  The
// row/column maps of the result are what the epilogue depends on; the plugin's tensor section
// declares them and an on-GPU bijection probe checks them.

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// compile-time integer tag (lets a generic lambda take a constant register-buffer index)
template <int V>
struct IC {
  static constexpr int value = V;
};

template <int MS>
struct Mfma;

template <>
struct Mfma<32> {
  typedef f32x16 acc_t;
  static constexpr int KSTEP = 16;  // k per instruction
  static constexpr int NACC = 16;   // result floats per lane
  static constexpr int GROUPS = 4;  // result row groups of 4 consecutive rows
  static constexpr int GROUP_STRIDE = 8;
  __device__ __forceinline__ static acc_t run(const f16x8& a, const f16x8& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<16> {
  typedef f32x4 acc_t;
  static constexpr int KSTEP = 32;
  static constexpr int NACC = 4;
  static constexpr int GROUPS = 1;
  static constexpr int GROUP_STRIDE = 16;
  __device__ __forceinline__ static acc_t run(const f16x8& a, const f16x8& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Result row of value v for lane l (see the map above).
template <int MS>
__device__ __forceinline__ int mfma_out_row(int lane, int g, int e) {
  return g * Mfma<MS>::GROUP_STRIDE + 4 * (lane / MS) + e;
}

// ------------------------------------------------------------------------------------------
// Bit-exact dequantisation in registers.
//
// Weight formats (op-level "fmt"):
//   1  int8, symmetric, one fp16 scale per output channel:   W = fp16_rn(q * s)
//   2  uint8, asymmetric, fp16 scale + uint8 zero-point per (row, 128-group): W = fp16_rn((q-z)*s)
//
// The integer q (or q - z) is built as an fp16 without rounding: the bit pattern 0x64XX is the
// fp16 value 1024 + XX for a byte XX, and subtracting 1024 + z (also exact) leaves q - z exactly
// (|q - z| <= 255 < 2048, where fp16 spacing is 1).  The scale multiply is one IEEE fp16 multiply,
// which is correctly rounded (RNE) -- and since q*s is exact in fp32 (8 x 11 significant bits),
// fp16_rn(fp16 q * fp16 s) == fp16_rn(float(q) * float(s)), the closed form of the formats.
// No q*s - z*s folding: that would round twice.
// ------------------------------------------------------------------------------------------

// Four bytes of w -> four fp16 values 1024 + byte, as two packed halves pairs.
__device__ __forceinline__ void bytes_to_magic(uint32_t w, uint32_t& lo, uint32_t& hi) {
  // v_perm_b32 selector: bytes 0..3 come from the second operand (w), 4..7 from the first.
  lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);  // [b1 | 0x64, b0 | 0x64] -> halves
  hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
}

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// 8 weight bytes (two dwords) -> 8 dequantised fp16 values.  `bias` is 1024 + zero-point
// (uint8 formats) or 1152 (int8 after the sign flip), `s` the fp16 scale, both broadcast.
__device__ __forceinline__ f16x8 dequant8(uint32_t w0, uint32_t w1, _Float16 bias, _Float16 s) {
  uint32_t p0, p1, p2, p3;
  bytes_to_magic(w0, p0, p1);
  bytes_to_magic(w1, p2, p3);
  const f16x2 b2 = {bias, bias};
  const f16x2 s2 = {s, s};
  const f16x2 d0 = (as_h2(p0) - b2) * s2;
  const f16x2 d1 = (as_h2(p1) - b2) * s2;
  const f16x2 d2 = (as_h2(p2) - b2) * s2;
  const f16x2 d3 = (as_h2(p3) - b2) * s2;
  f16x8 r;
  r[0] = d0[0]; r[1] = d0[1]; r[2] = d1[0]; r[3] = d1[1];
  r[4] = d2[0]; r[5] = d2[1]; r[6] = d3[0]; r[7] = d3[1];
  return r;
}

// int8 (two's complement) bytes: flip the sign bit so byte = q + 128, then bias = 1152.
__device__ __forceinline__ f16x8 dequant8_i8(uint32_t w0, uint32_t w1, _Float16 s) {
  return dequant8(w0 ^ 0x80808080u, w1 ^ 0x80808080u, (_Float16)1152.0f, s);
}

__device__ __forceinline__ f16x8 dequant8_u8(uint32_t w0, uint32_t w1, uint8_t z, _Float16 s) {
  return dequant8(w0, w1, (_Float16)(1024.0f + (float)z), s);
}

// The lane index recomputed from the exec-mask bit count (mbcnt), for epilogues: a value derived
// from threadIdx.x and kept across a register-full main loop gets spilled; this one is rebuilt
// where it is needed.
__device__ __forceinline__ int lane_id() {
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ f16x8 as_f16x8(const u32x4& u) { return __builtin_bit_cast(f16x8, u); }
__device__ __forceinline__ u32x4 as_u32x4(const f16x8& h) { return __builtin_bit_cast(u32x4, h); }

// Fused gate/up epilogue: silu(g) * u on the fp16-rounded GEMM results, i.e. exactly what the
// unfused chain (two fp16 GEMM outputs, then silu and a product) sees, in fp32, one rounding to
// fp16 at the end.  silu(x) = x / (1 + e^-x); e^-x by the hardware exponential.
__device__ __forceinline__ _Float16 silu_mul_f16(float g, float u) {
  const float gh = (float)(_Float16)g;
  const float uh = (float)(_Float16)u;
  return (_Float16)(gh / (1.0f + __expf(-gh)) * uh);
}
