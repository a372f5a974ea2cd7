/*
 * tempo_gfx950.h -- C ABI of the MI355X (gfx950) kernels behind the Tempolator plugin
 * `tempo/plugins/gfx950` and the shipped deliveries kernels/shipped/{gemm_fp16,gemm_w8a16}/gfx950.
 *
 * Library: cuda_tempiler_amd/libtempo_gfx950.so (built by cuda_tempiler_amd/build.py).
 *
 * Conventions (all entry points):
 *   - plain pointers and sizes; no framework types.  Device pointers are HIP device memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).  Every launch is
 *     asynchronous on that stream; the caller owns every input and output buffer.
 *   - split-K rows (narrow N, long K: fp32 partial sums of k ranges, reduced by a second kernel
 *     on the same stream) need a workspace of tempo_gemm_*_workspace_bytes() bytes.  The launch
 *     entry points take it from the library's pool: one device buffer per (device, stream),
 *     allocated with hipMalloc the first time a shape needs it and grown (after a synchronise of
 *     that stream) when a larger one does.  So the first split-K call on a stream allocates;
 *     later calls of the same or smaller shapes do not.  Calls on different streams never
 *     share a workspace.  Every other row uses no workspace and allocates nothing.
 *   - the int returned is a hipError_t value: 0 = success; TEMPO_FALLBACK (9, the value of
 *     hipErrorInvalidConfiguration) = "shape not covered, take your own path" -- a legal
 *     answer, not a failure (reference kernels/shipped/gemm_fp16/sm_70/dispatch.inc:12-13,26).
 *     Other values propagate from the HIP runtime.
 *   - fp16 data is IEEE binary16; results round to nearest even.
 */
#ifndef TEMPO_GFX950_H
#define TEMPO_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tempo_stream_t;

#define TEMPO_OK 0
#define TEMPO_FALLBACK 9

/* ------------------------------------------------------------------------------------------
 * gemm_fp16:  C[M][N] = fp16_rn( sum_k A[m][k] * B[n][k] ), fp32 accumulation.
 * Replaces the reference's shipped launcher tempo::gen::GemmParams / applicable() / launch()
 * (kernels/shipped/gemm_fp16/sm_70/launch.cuh:20-26, :59-67, :75; launch.cu:20-22).  Same
 * fields, same meaning (strides in elements, k contiguous).
 * ------------------------------------------------------------------------------------------ */
typedef struct TempoGemmParams {
  const void* A; /* fp16 [M][lda] */
  const void* B; /* fp16 [N][ldb] */
  void* C;       /* fp16 [M][ldc] */
  int M, N, K;
  int lda, ldb, ldc;
} TempoGemmParams;

/* 1 = covered (launch will run a kernel), 0 = not covered (caller takes its own path).
 * Reference: launch.cuh:59-67 applicable() plus the ladder coverage of dispatch.inc. */
int tempo_gemm_fp16_applicable(const TempoGemmParams* p);
/* Reference: launch.cu:20-22 tempo::gen::launch(const GemmParams&, cudaStream_t).  A split-K
 * row takes its fp32 partial sums from the library's pool: one device buffer per (device,
 * stream), allocated on first use and grown with hipMalloc when a larger shape needs it (a
 * grown-out buffer is kept, not freed, until the process ends, so work already queued or a graph
 * captured earlier never sees it freed).  On a stream under graph capture the pool cannot grow:
 * such a call returns hipErrorStreamCaptureUnsupported (900) and launches nothing; use
 * tempo_gemm_fp16_launch_ws there. */
int tempo_gemm_fp16_launch(const TempoGemmParams* p, tempo_stream_t stream);
/* tempo_gemm_fp16_launch with the caller's workspace (ws, ws_bytes device memory; may be NULL /
 * 0 for shapes whose row needs none): never allocates, never synchronises.  A row needing more
 * than ws_bytes (tempo_gemm_fp16_workspace_bytes) returns hipErrorOutOfMemory (2) without
 * launching.  No reference counterpart (its launcher has no workspace, launch.cuh:20-26): this
 * is for callers whose own allocator must own every buffer -- a framework capturing HIP graphs
 * (torch's graph-aware caching allocator), arenas of a serving loop. */
int tempo_gemm_fp16_launch_ws(const TempoGemmParams* p, void* ws, size_t ws_bytes,
                              tempo_stream_t stream);
/* Bytes of workspace the row tempo_gemm_fp16_launch runs for this shape needs (0: none, or not
 * covered).  Host-only.  No reference counterpart: the reference's ladder has no split-K row
 * (kernels/shipped/gemm_fp16/sm_70/dispatch.inc:15-26). */
size_t tempo_gemm_fp16_workspace_bytes(const TempoGemmParams* p);

/* ------------------------------------------------------------------------------------------
 * gemm_w8a16:  C = fp16_rn( A . deq(Wq)^T ), fp32 accumulation, weights dequantised in
 * registers bit-exactly:
 *   fmt 1 (TEMPO_W8_SYM_I8):   Wq int8  [N][ldw], scale fp16 [N]          W = fp16_rn(q * s[n])
 *   fmt 2 (TEMPO_W8_ASYM_U8):  Wq uint8 [N][ldw], scale fp16 [N][K/group], zero uint8 [N][K/group]
 *                              W = fp16_rn((q - z[n][k/group]) * s[n][k/group])
 * Replaces the reference's W8A16 skeleton launch (tempo/plugins/sm70/skeletons/gemm_w8a16/
 * harness.cu:88-94, k_gemm8 in kernel.cuh:226-296), which is symmetric and scale-free; the
 * scaled formats extend it as declared in the north star (GPTQ formula of
 * bench/gemm_baseline.py:229, stored [N][K]).
 * ------------------------------------------------------------------------------------------ */
#define TEMPO_W8_SYM_I8 1
#define TEMPO_W8_ASYM_U8 2

typedef struct TempoW8A16Params {
  const void* A;     /* fp16 [M][lda] */
  const void* Wq;    /* int8 or uint8 [N][ldw] */
  const void* scale; /* fp16, [N] (fmt 1) or [N][K/group] (fmt 2) */
  const void* zero;  /* NULL (fmt 1) or uint8 [N][K/group] (fmt 2) */
  void* C;           /* fp16 [M][ldc] */
  int M, N, K;
  int lda, ldw, ldc;
  int group; /* fmt 2: k per scale group (128; divides K); fmt 1: ignored */
  int fmt;
} TempoW8A16Params;

int tempo_gemm_w8a16_applicable(const TempoW8A16Params* p);
/* Split-K rows take the library's pool, as tempo_gemm_fp16_launch does (same growth, retirement
 * and graph-capture rule). */
int tempo_gemm_w8a16_launch(const TempoW8A16Params* p, tempo_stream_t stream);
/* tempo_gemm_w8a16_launch with the caller's workspace, as tempo_gemm_fp16_launch_ws. */
int tempo_gemm_w8a16_launch_ws(const TempoW8A16Params* p, void* ws, size_t ws_bytes,
                               tempo_stream_t stream);
/* Bytes of workspace the row tempo_gemm_w8a16_launch runs for this shape needs (0: none, or not
 * covered).  Host-only; no reference counterpart (as for tempo_gemm_fp16_workspace_bytes). */
size_t tempo_gemm_w8a16_workspace_bytes(const TempoW8A16Params* p);

/* tempo_gemm_w8a16_launch that allocates nothing, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same rows, kernels and results as tempo_gemm_w8a16_launch (bit for bit); a
 * split-K row takes its workspace from a static device array of TEMPO_NOALLOC_SCRATCH_BYTES per
 * GPU instead of the allocating pool, and a row that would need more returns
 * hipErrorOutOfMemory (2) without launching.  The current ladder never needs more: an
 * interleaved split-K row keeps tiles x splits <= 256, so its workspace is at most
 * 256 x 128 x 256 x 4 bytes = 32 MiB; a line row with k slices needs ks x M x N x 4 bytes with
 * ks <= 8 and M <= 32, and slices only grids short of whole rounds of the part (3.75 MiB at most
 * today, at (32, 5120, 12288)).
 * Every call on one GPU shares that GPU's array (the first call on a device looks its address
 * up): calls that overlap on one GPU -- on different streams, or from different threads without
 * ordering -- race on it.  Nothing in it needs clearing: a split-K launch writes every partial
 * sum it later reads. */
#define TEMPO_NOALLOC_SCRATCH_BYTES (32u << 20)
int tempo_gemm_w8a16_launch_noalloc(const TempoW8A16Params* p, tempo_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Fused gate/up epilogue (the MLP's first projection):
 *   C[m][n] = silu(G[m][n]) * U[m][n],  G = A . B[0..N)^T,  U = A . B[N..2N)^T
 * with N the OUTPUT width: B (fp16) or Wq / scale / zero (W8A16) hold 2N rows, the gate rows
 * then the up rows (the merged gate_up layout; the production shape S1 of
 * bench/shapes/qwen36_27b_int8.json is this GEMM at 2N = 34816).  G and U are rounded to fp16
 * before the epilogue, so the result is the unfused chain's up to the last bit of silu.  The
 * reference names this fusion and its price and does not ship it (docs/NOT_YET.md:141-146,
 * kernels/shipped/gemm_fp16/sm_70/INTEGRATION.md:21).  Every M is covered (decode rows on the
 * streaming kernels, prefill rows on the interleaved kernels) where N % 128 == 0 and K fits a
 * row; other shapes return TEMPO_FALLBACK (run the plain GEMM and the elementwise step).
 * ------------------------------------------------------------------------------------------ */
int tempo_gemm_fp16_gate_up_launch(const TempoGemmParams* p, tempo_stream_t stream);
int tempo_gemm_w8a16_gate_up_launch(const TempoW8A16Params* p, tempo_stream_t stream);

/* Debug/verification: dequantise rows [n0, n0+rows) x cols [k0, k0+cols) of Wq into fp16
 * out[rows][cols] with the same device functions the GEMM feeds use (cols % 8 == 0, k0 % 8 == 0).
 * No reference counterpart: the reference's skeleton has no scale, so its dequantisation is the
 * identity (harness.cu:39-46); this entry is what makes "bit-exact dequant" testable. */
int tempo_dequant_tile(const TempoW8A16Params* p, int n0, int k0, int rows, int cols, void* out,
                       tempo_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * GPTQ int8 repack (one-time, at load): checkpoint layout -> the fmt 2 layout of gemm_w8a16.
 *   in:  qweight int32 [K/4][N] (byte k%4 of qweight[k/4][n] = q[k][n]), qzeros int32
 *        [K/group][N/4] (byte n%4 = z[g][n]), scales fp16 [K/group][N]
 *   out: wq uint8 [N][K], scale_out fp16 [N][K/group], zero_out uint8 [N][K/group]
 * A byte permutation (bit-exact).  Requires K % 128 == 0, N % 64 == 0, group == 128, 16-byte
 * aligned qweight and wq; otherwise TEMPO_FALLBACK.  The checkpoint format is the reference's
 * make_gptq_int8 (bench/gemm_baseline.py:214-232, dequantised by the formula of :229).
 * ------------------------------------------------------------------------------------------ */
int tempo_gptq_repack_u8(const void* qweight, const void* qzeros, const void* scales, int K, int N,
                         int group, void* wq, void* scale_out, void* zero_out,
                         tempo_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * fmha_fwd: O = softmax(scale * Q K^T + causal mask) V, fp32 softmax, fp16 O, fp32 LSE
 * (natural log).  GQA: query head h reads KV head h / (H / Hkv).  Causal mask is bottom-right:
 * row i sees keys j <= i + (Sk - Sq).  Strides in elements; Q/O addressed as
 * b*sb + i*ss + h*sh + d, K/V likewise with the KV head.  LSE may be NULL, else [B][H][Sq].
 * Replaces the forward signature of the reference's profiled FMHA (profiled/fwd_ws/fa2_sm70/
 * csrc/volta_fwd_ws.cuh:276-283; attn_fwd_cutlass.cu:137,193,660-666).  The reference ships no
 * FMHA skeleton (tempo/plugins/sm70/__init__.py:57).
 * ------------------------------------------------------------------------------------------ */
typedef struct TempoFmhaParams {
  const void* Q;
  const void* K;
  const void* V;
  void* O;
  float* LSE;
  int B, H, Hkv, Sq, Sk, D;
  float scale;
  int causal;
  long q_sb, q_ss, q_sh;
  long k_sb, k_ss, k_sh;
  long v_sb, v_ss, v_sh;
  long o_sb, o_ss, o_sh;
} TempoFmhaParams;

int tempo_fmha_fwd_applicable(const TempoFmhaParams* p);
int tempo_fmha_fwd_launch(const TempoFmhaParams* p, tempo_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * The naive input kernel (kernels/naive/gemm_fp16.hip): one thread per output, sequential k.
 * The "vs input" bar; reference kernels/naive/gemm_fp16.cu:60-76.
 * ------------------------------------------------------------------------------------------ */
int tempo_naive_gemm_fp16_launch(const void* A, const void* B, void* C, int M, int N, int K,
                                 tempo_stream_t stream);

/* The naive W8A16 input kernel (kernels/naive/gemm_w8a16.hip): dequantise each weight once to
 * fp16_rn((q - z) * s), then the naive fp16 accumulation above.  Dense operands only (lda = ldw
 * = K, ldc = N).  The reference ships no naive W8A16 input; its dense formula is
 * bench/gemm_baseline.py:229. */
int tempo_naive_gemm_w8a16_launch(const TempoW8A16Params* p, tempo_stream_t stream);

/* The naive attention input kernel (kernels/naive/fmha_fwd.hip): one thread per (batch, head,
 * query row), two fp32 passes over the visible keys; dense BSHD storage (Q, O [B][Sq][H][D];
 * K, V [B][Sk][Hkv][D]), D <= 256, LSE optional (NULL: not written).  The "vs input" bar of
 * tempo_fmha_fwd_launch, with the semantics it replaces (profiled/fwd_ws/fa2_sm70/csrc/
 * attn_fwd_cutlass.cu:137,193; volta_fwd_ws.cuh:432,863,1063). */
int tempo_naive_fmha_fwd_launch(const void* Q, const void* K, const void* V, void* O, float* LSE,
                                int B, int H, int Hkv, int Sq, int Sk, int D, float scale,
                                int causal, tempo_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Plugin support (no reference counterpart in the C ABI; the sm70 plugin does these checks
 * from Python, tempo/plugins/sm70/tensor.py:72-86).
 * ------------------------------------------------------------------------------------------ */
/* MFMA result-layout probe: runs one MFMA of shape ms (32 or 16) with rank-1 operands that encode
 * row and column indices, writing out[2][64][nacc] floats (row+1, then col+1, per lane and
 * result register).  nacc = 16 for ms 32, 4 for ms 16.  `out` is device memory. */
int tempo_probe_mfma_layout(int ms, float* out, tempo_stream_t stream);

/* Name of the shipped ladder row a shape dispatches to ("" when not covered).  ops 3, 4, 5 are the
 * fused gate/up variants of ops 0, 1, 2 (N = output width).  op 0 = gemm_fp16,
 * op 1 = gemm_w8a16 (fmt 1), op 2 = gemm_w8a16 (fmt 2).  Host-only; no GPU needed. */
int tempo_route(int op, int M, int N, int K, char* tag, int tag_len);

/* ABI version of this header (bumped on any struct change). */
int tempo_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TEMPO_GFX950_H */
