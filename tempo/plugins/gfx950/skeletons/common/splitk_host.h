// common/splitk_host.h -- host side of the split-K launches, frozen into each delivery's
// kernel.hip after the kernels (it names k_splitk_reduce): the workspace a split-K row needs,
// where it comes from, and how many splits a row takes.
//
// A split-K row adds fp32 partial sums of its k ranges, [splits][M][N], in a workspace and reduces
// them with k_splitk_reduce on the same stream.  The workspace is either memory the caller hands
// over, or the delivery's pool: one buffer per (device, stream), allocated on first use and grown
// when a larger shape needs it, so calls on different streams stay independent and calls on one
// stream are ordered by it.

// Workspace of a split-K row.  `ptr`/`bytes`: device memory the caller hands over (may be
// null / 0); `pool`: the row may take the delivery's per-(device, stream) pool instead; `need`:
// when set, the row only reports the bytes it needs (0 for rows without a workspace) and
// launches nothing.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool pool = false;
  size_t* need = nullptr;
};

// The pool: one buffer per (device, stream), grown on demand.  A buffer that a larger shape
// outgrows is retired, not freed: work already queued on the stream, a graph captured earlier
// or another thread that took the pointer a moment ago may still use it, so it stays allocated
// until the process ends (at most one retired buffer per growth step, each smaller than its
// successor).  Growing needs hipMalloc, which a stream under graph capture cannot take: there
// the pool returns hipErrorStreamCaptureUnsupported and the caller hands over its workspace
// instead (launch_with, or the C ABI's *_launch_ws entry points).  (The frozen file's preamble
// includes <map>, <mutex>, <utility> and <vector>.)
inline void* pool_buffer(hipStream_t s, size_t bytes, hipError_t* err) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> pool;
  static std::vector<void*> retired;
  int dev = 0;
  if ((*err = hipGetDevice(&dev)) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  std::pair<void*, size_t>& e = pool[std::make_pair(dev, s)];
  if (e.second < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((*err = hipStreamIsCapturing(s, &cs)) != hipSuccess) return nullptr;
    if (cs != hipStreamCaptureStatusNone) {
      *err = hipErrorStreamCaptureUnsupported;
      return nullptr;
    }
    void* q = nullptr;
    if (hipMalloc(&q, bytes) != hipSuccess) {
      *err = hipErrorOutOfMemory;
      return nullptr;
    }
    if (e.first) retired.push_back(e.first);
    e = std::make_pair(q, bytes);
  }
  return e.first;
}

// The workspace of a split-K launch: the caller's if it is large enough, else the pool's when the
// row may take it.  nullptr with *err set otherwise (hipErrorOutOfMemory: the caller's buffer is
// too small and no pool was allowed).
inline float* workspace_for(const Workspace& w, size_t bytes, hipStream_t s, hipError_t* err) {
  *err = hipSuccess;
  if (w.ptr && w.bytes >= bytes) return static_cast<float*>(w.ptr);
  if (w.pool) return static_cast<float*>(pool_buffer(s, bytes, err));
  *err = hipErrorOutOfMemory;
  return nullptr;
}

// Split count of a split-K row: the most splits such that tiles x splits stays within `slots`
// workgroups (one round of the part: a split count that spills into a second round makes every
// split of that round wait for it), each split keeping at least `minkt` k-tiles, and no split
// empty.  1 = no split.
inline int split_count(int tiles, int ktiles, int slots, int minkt) {
  if (slots <= 0 || minkt <= 0 || 2 * tiles > slots) return 1;
  int sp = slots / tiles;
  if (sp > ktiles / minkt) sp = ktiles / minkt;
  if (sp <= 1) return 1;
  const int per = (ktiles + sp - 1) / sp;
  return (ktiles + per - 1) / per;
}

// Launch of the split-K reduction: C = fp16_rn(sum over the splits of ws), in split order.
inline hipError_t launch_reduce(const float* ws, int splits, int M, int N, _Float16* C, int ldc,
                                hipStream_t s) {
  const long work = (long)M * N / 4;
  hipLaunchKernelGGL(k_splitk_reduce<8>, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, s, ws,
                     splits, M, N, C, ldc);
  return hipGetLastError();
}
