// common/splitk_host.h -- host side of the split-K launches, frozen into each delivery's
// kernel.hip after the kernels (it names k_splitk_reduce): the workspace a split-K row needs,
// where it comes from, and how many splits a row takes.
//
// A split-K row adds fp32 partial sums of its k ranges, [splits][M][N], in a workspace and reduces
// them with k_splitk_reduce on the same stream.  The workspace is either memory the caller hands
// over, or the delivery's pool: one buffer per (device, stream), allocated on first use and grown
// when a larger shape needs it, so calls on different streams stay independent and calls on one
// stream are ordered by it.  (The frozen file's preamble includes <map>, <mutex> and <utility>.)

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

// The pool: one buffer per (device, stream), grown on demand.  Work already queued on the stream
// may still read the old buffer, so it is freed only after the stream has drained.
inline void* pool_buffer(hipStream_t s, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> pool;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  std::pair<void*, size_t>& e = pool[std::make_pair(dev, s)];
  if (e.second < bytes) {
    if (e.first) {
      if (hipStreamSynchronize(s) != hipSuccess) return nullptr;
      (void)hipFree(e.first);
    }
    e = std::make_pair(nullptr, (size_t)0);
    void* q = nullptr;
    if (hipMalloc(&q, bytes) != hipSuccess) return nullptr;
    e = std::make_pair(q, bytes);
  }
  return e.first;
}

inline float* workspace_for(const Workspace& w, size_t bytes, hipStream_t s) {
  if (w.ptr && w.bytes >= bytes) return static_cast<float*>(w.ptr);
  if (w.pool) return static_cast<float*>(pool_buffer(s, bytes));
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
