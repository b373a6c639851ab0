// Reductions (mapreduce) for gfx950: full, along dim 1 and along dim 2.
//
// Same two stages as the reference's kernels (reference
// src/mapreduce/1D/mapreduce1d_kernel.jl:5-93 for the full reduction,
// src/mapreduce/2D/vecmat_kernel.jl:1-169 for dims=1 and
// src/mapreduce/2D/matvec_kernel.jl:1-239 for dims=2): partial results per
// workgroup, then a combine. MI355X design:
//  * Stage 1 streams with 16-byte nontemporal loads, several in flight per
//    lane, every vector element folded into its own accumulator (16
//    independent Float32 sums per lane: accurate and dependency-free).
//  * Stage 2 is a second, tiny kernel on the same stream. The reference's
//    single launch lets workgroup 1 spin on per-workgroup flags
//    (mapreduce1d_kernel.jl:66-92); a "last workgroup done" ticket was
//    measured here to serialise thousands of same-address device atomics
//    at the end of the grid (the full reduction ran at 1.8 TB/s with 8192
//    workgroups), and fences cost more than the launch they save. Grids of
//    up to kFoldMax workgroups skip the launch with an atomic-free fold
//    instead: epoch-tagged partial slots written with relaxed device-scope
//    stores and gathered by the last workgroup (fold_partial), which saves
//    a launch's host cost (eager 10^6 Float32: 11.0 -> 8.7 us).
//  * Combine orders depend only on the shape and pointer alignment, so every
//    result is bit-for-bit reproducible run to run.
#include "kf_common.h"

namespace kf {

constexpr int kRedBlock = 256;
constexpr int kRedWaves = kRedBlock / kWave;
constexpr int kRedUnroll = 4;
constexpr int kRedMaxBlocks = 8192;

inline size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Every reduction scratch buffer starts with a reserved area that no other
// partial buffer overlaps: an 8-byte epoch word (then padding to 256 bytes)
// and kFoldMax 16-byte slots for the single-level fold of
// reduce_once_kernel. Partial buffers of all reduction kinds sit after it,
// so stale partials of other calls can never read as current fold slots.
constexpr int kFoldMax = 2048;  // workgroups a single-level fold combines
constexpr bool kUseFold = true;
constexpr size_t kRedReserved = 256 + (size_t)kFoldMax * 16;
inline void* red_work(void* scratch) { return scratch ? (uint8_t*)scratch + kRedReserved : nullptr; }

// Block-wide combine in wave order; result valid in thread 0.
template <class T, class Op> __device__ inline T block_reduce(T x, T* s_wave) {
  const int wave = threadIdx.x / kWave;
  x = wave_reduce<Op>(x);
  if (lane_id() == 0) s_wave[wave] = x;
  __syncthreads();
  T r = s_wave[0];
#pragma unroll
  for (int w = 1; w < kRedWaves; ++w) r = Op::combine(r, s_wave[w]);
  return r;
}

// ---------------------------------------------------------------------------
// Full reduction, stage 1: grid-stride over 16-byte vectors. An unaligned
// head and the ragged tail are folded in by workgroup 0, so any
// element-aligned contiguous view takes the vector path.
// ---------------------------------------------------------------------------
template <class T, class Op, class Map>
__global__ __launch_bounds__(kRedBlock) void reduce_kernel(const T* src, int64_t n, int64_t stride,
                                                           T* out, int vec) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const int64_t gtid = (int64_t)blockIdx.x * kRedBlock + tid;
  const int64_t gsize = (int64_t)gridDim.x * kRedBlock;

  T acc = id;
  if (vec) {
    const int64_t head = kmin<int64_t>(n, (int64_t)(((16 - ((uintptr_t)src & 15)) & 15) / sizeof(T)));
    const int64_t nvec = (n - head) / EPV;
    const int64_t tail0 = head + nvec * EPV;
    const uint4* v = reinterpret_cast<const uint4*>(src + head);
    T a[kRedUnroll][EPV];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[u][e] = id;
    int64_t i = gtid;
    for (; i + (kRedUnroll - 1) * gsize < nvec; i += kRedUnroll * gsize) {
      uint4 r[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) r[u] = ld_stream(v + i + u * gsize);
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) {
        T x[EPV];
        __builtin_memcpy(x, &r[u], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], Map::apply(x[e]));
      }
    }
    for (; i < nvec; i += gsize) {
      const uint4 r = ld_stream(v + i);
      T x[EPV];
      __builtin_memcpy(x, &r, 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[0][e] = Op::combine(a[0][e], Map::apply(x[e]));
    }
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc = Op::combine(acc, a[u][e]);
    if (blockIdx.x == 0) {
      if (tid < head) acc = Op::combine(acc, Map::apply(src[tid]));
      if (tail0 + tid < n) acc = Op::combine(acc, Map::apply(src[tail0 + tid]));
    }
  } else {
    T a[kRedUnroll];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) a[u] = id;
    int64_t i = gtid;
    for (; i + (kRedUnroll - 1) * gsize < n; i += kRedUnroll * gsize) {
      T x[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) x[u] = src[(i + u * gsize) * stride];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) a[u] = Op::combine(a[u], Map::apply(x[u]));
    }
    for (; i < n; i += gsize) a[0] = Op::combine(a[0], Map::apply(src[i * stride]));
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) acc = Op::combine(acc, a[u]);
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if (tid == 0) out[blockIdx.x] = part;  // a partial, or the result when gridDim.x == 1
}

// Full reduction, stage 1 (vector path): one-shot workgroups. Workgroup b
// reads the kOnceVecs 16-byte vectors [b*kOnceVecs, (b+1)*kOnceVecs) once and
// writes one partial; the grid covers the whole array. Many short-lived
// workgroups keep far more loads in flight than a grid-stride loop (measured
// 7.3 vs 6.1 TB/s for Float32 reads on MI355X). Workgroup 0 also folds in
// the unaligned head and the ragged tail. The same kernel (head = tail = 0,
// identity map) reduces the partials of the previous level.
constexpr int kOnceUnroll = 2;
constexpr int kOnceVecs = kRedBlock * kOnceUnroll;

// Single-level fold, replacing combine_all_kernel's launch for grids of
// 2..kFoldMax workgroups. Every workgroup but the last publishes its
// partial into its slot as W 64-bit words, each {tag:32, value bits:32},
// with relaxed device-scope stores. The last workgroup polls all slots
// (8 per thread, all in flight together) until every word carries the
// tag, then combines them in slot order with its own partial last, so
// the result does not depend on timing. It stores the result and the tag
// as the new epoch. The tag is epoch + 1, read with a plain load at kernel
// start: the previous call's last workgroup wrote it before that kernel
// ended, and within a call every reader loads it before publishing,
// which the waiter's completion depends on. Slots of older calls never
// match. Only one workgroup ever waits, so progress needs no co-residency;
// a bounded spin (only a corrupted or concurrently shared buffer can
// exhaust it) keeps a bad buffer from hanging the GPU.
constexpr uint32_t kFoldSpinLimit = 1u << 22;
template <class T, class Op> __device__ inline void fold_partial(T part, T* out, uint64_t* hdr, T* s_wave) {
  constexpr int W = Words<T>::W;
  constexpr int PER = kFoldMax / kRedBlock;
  __shared__ uint32_t s_tag;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const uint32_t t = (uint32_t)hdr[0] + 1u;
    s_tag = t == 0 ? 1u : t;
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  uint64_t* slots = hdr + 256 / sizeof(uint64_t);
  const int last = (int)gridDim.x - 1;
  if ((int)blockIdx.x != last) {
    if (tid == 0) {
      const Words<T> w = to_words(part);
#pragma unroll
      for (int i = 0; i < W; ++i) st_agent(slots + 2 * blockIdx.x + i, ((uint64_t)tag << 32) | w.w[i]);
    }
    return;
  }
  // the last workgroup: slot k * kRedBlock + tid of every k on this thread
  const T id = Op::template identity<T>();
  T v[PER];
  bool done[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = id;
    done[k] = k * kRedBlock + tid >= last;
  }
  for (uint32_t polls = 0; polls < kFoldSpinLimit; ++polls) {
    uint64_t d[PER][W];
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (!done[k]) {
#pragma unroll
        for (int i = 0; i < W; ++i) d[k][i] = ld_agent(slots + 2 * (k * kRedBlock + tid) + i);
      }
    bool all = true;
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (!done[k]) {
        bool ok = true;
        Words<T> w;
#pragma unroll
        for (int i = 0; i < W; ++i) {
          ok &= (uint32_t)(d[k][i] >> 32) == tag;
          w.w[i] = (uint32_t)d[k][i];
        }
        if (ok) {
          v[k] = from_words<T>(w);
          done[k] = true;
        } else {
          all = false;
        }
      }
    if (__syncthreads_and(all)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  T acc = v[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) acc = Op::combine(acc, v[k]);
  __syncthreads();  // s_wave still holds this workgroup's own partial sums
  const T others = block_reduce<T, Op>(acc, s_wave);
  if (tid == 0) {
    out[0] = Op::combine(others, part);
    hdr[0] = tag;
  }
}

template <class T, class Op, class Map, bool FOLD = false>
__global__ __launch_bounds__(kRedBlock) void reduce_once_kernel(const T* src, int64_t n, int64_t head,
                                                                int64_t nvec, T* out, uint64_t* fold_hdr) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const uint4* v = reinterpret_cast<const uint4*>(src + head);
  const int64_t base = (int64_t)blockIdx.x * kOnceVecs + tid;
  uint4 r[kOnceUnroll];
#pragma unroll
  for (int u = 0; u < kOnceUnroll; ++u)
    if (base + u * kRedBlock < nvec) r[u] = ld_stream(v + base + u * kRedBlock);
  T a[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) a[e] = id;
#pragma unroll
  for (int u = 0; u < kOnceUnroll; ++u)
    if (base + u * kRedBlock < nvec) {
      T x[EPV];
      __builtin_memcpy(x, &r[u], 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], Map::apply(x[e]));
    }
  T acc = a[0];
#pragma unroll
  for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, a[e]);
  if (blockIdx.x == 0) {
    const int64_t tail0 = head + nvec * EPV;
    if (tid < head) acc = Op::combine(acc, Map::apply(src[tid]));
    if (tail0 + tid < n) acc = Op::combine(acc, Map::apply(src[tail0 + tid]));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if constexpr (!FOLD) {
    if (tid == 0) out[blockIdx.x] = part;  // a partial, or the result when gridDim.x == 1
  } else {
    fold_partial<T, Op>(part, out, fold_hdr, s_wave);  // out is the result
  }
}

// Full reduction, stage 2: one 1024-thread workgroup combines `count`
// partials; each thread issues all of its (at most kRedMaxBlocks/1024) loads
// before combining, so the stage costs about one memory latency.
constexpr int kCombineBlock = 1024;
template <class T, class Op>
__global__ __launch_bounds__(kCombineBlock) void combine_all_kernel(const T* partials, int count, T* dst) {
  constexpr int PER = kRedMaxBlocks / kCombineBlock;
  constexpr int WAVES = kCombineBlock / kWave;
  __shared__ T s_wave[WAVES];
  const T id = Op::template identity<T>();
  T v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = k * kCombineBlock + threadIdx.x;
    v[k] = j < count ? partials[j] : id;
  }
  T x = v[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) x = Op::combine(x, v[k]);
  x = wave_reduce<Op>(x);
  if (lane_id() == 0) s_wave[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    T r = s_wave[0];
    for (int w = 1; w < WAVES; ++w) r = Op::combine(r, s_wave[w]);
    dst[0] = r;
  }
}

// Stage 2 of the split dims reductions: out[i*ds] = op_s partials[s*m + i],
// for batch z = blockIdx.y: partials at z*S*m, outputs at z*dst_bstride.
template <class T, class Op>
__global__ __launch_bounds__(kRedBlock) void combine_split_kernel(const T* partials, int S, int64_t m, T* dst,
                                                                  int64_t ds, int64_t dst_bstride) {
  const int64_t i = (int64_t)blockIdx.x * kRedBlock + threadIdx.x;
  if (i >= m) return;
  partials += (int64_t)blockIdx.y * S * m;
  dst += (int64_t)blockIdx.y * dst_bstride;
  T x = partials[i];
  for (int s = 1; s < S; ++s) x = Op::combine(x, partials[(int64_t)s * m + i]);
  dst[i * ds] = x;
}

template <class T> int reduce_grid(int64_t n) {
  constexpr int64_t per_block = (int64_t)kRedBlock * kRedUnroll * 2;
  int64_t g = (n + per_block - 1) / per_block;
  const int64_t cap = kmin<int64_t>(kRedMaxBlocks, (int64_t)kf_device_cu_count() * 32);
  if (g > cap) g = cap;
  return (int)kmax<int64_t>(g, 1);
}

// Level sizes of the vector path: partial counts after each one-shot level
// until at most kRedMaxBlocks remain for combine_all_kernel.
struct OnceLevels {
  int nlev;
  int64_t count[8];
};
inline OnceLevels once_levels(int64_t nvec, int epv) {
  OnceLevels L{};
  int64_t c = kmax<int64_t>(1, (nvec + kOnceVecs - 1) / kOnceVecs);
  L.count[L.nlev++] = c;
  while (c > kRedMaxBlocks && L.nlev < 8) {
    const int64_t cv = (c + epv - 1) / epv;  // partials read as 16-byte vectors
    c = (cv + kOnceVecs - 1) / kOnceVecs;
    L.count[L.nlev++] = c;
  }
  return L;
}

// Scratch for a full reduction of n elements of es bytes: two ping-pong
// partial buffers for the vector path, or kRedMaxBlocks partials for the
// strided path, whichever is larger.
inline size_t reduce_scratch(size_t es, int64_t n) {
  const int64_t nvec = n / (int64_t)(16 / es);
  const OnceLevels L = once_levels(nvec, (int)(16 / es));
  size_t a = 0, b = 0;
  for (int i = 0; i < L.nlev; ++i) {
    const size_t bytes = round256((size_t)L.count[i] * es + 16);
    if (i % 2 == 0) a = kmax(a, bytes); else b = kmax(b, bytes);
  }
  return kRedReserved + kmax<size_t>(a + b, round256((size_t)kRedMaxBlocks * es));
}

template <class T, class Op, class Map>
int launch_reduce(const void* src, int64_t n, int64_t stride, void* dst, void* scratch,
                  hipStream_t stream) {
  constexpr int EPV = 16 / (int)sizeof(T);
  uint8_t* work = (uint8_t*)red_work(scratch);
  if (stride != 1) {
    const int grid = reduce_grid<T>(n);
    T* out = grid == 1 ? (T*)dst : (T*)work;
    hipLaunchKernelGGL((reduce_kernel<T, Op, Map>), dim3(grid), dim3(kRedBlock), 0, stream,
                       (const T*)src, n, stride, out, 0);
    if (grid > 1)
      hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                         (const T*)work, grid, (T*)dst);
    return kf_check_launch("reduce_kernel");
  }
  const int64_t head = kmin<int64_t>(n, (int64_t)(((16 - ((uintptr_t)src & 15)) & 15) / sizeof(T)));
  const int64_t nvec = (n - head) / EPV;
  const OnceLevels L = once_levels(nvec, EPV);
  if (kUseFold && L.nlev == 1 && L.count[0] > 1 && L.count[0] <= kFoldMax) {
    // one launch: the last workgroup folds the others' partials (fold_partial)
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map, true>), dim3((unsigned)L.count[0]), dim3(kRedBlock), 0,
                       stream, (const T*)src, n, head, nvec, (T*)dst, (uint64_t*)scratch);
    return kf_check_launch("reduce_once_kernel");
  }
  size_t abytes = 0;
  for (int i = 0; i < L.nlev; i += 2) abytes = kmax(abytes, round256((size_t)L.count[i] * sizeof(T) + 16));
  T* buf[2] = {(T*)work, (T*)(work + abytes)};
  // level 0 reads the input (with map, head and tail); later levels reduce partials
  T* out0 = (L.nlev == 1 && L.count[0] == 1) ? (T*)dst : buf[0];
  hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map>), dim3((unsigned)L.count[0]), dim3(kRedBlock), 0, stream,
                     (const T*)src, n, head, nvec, out0, (uint64_t*)nullptr);
  for (int i = 1; i < L.nlev; ++i) {
    const int64_t m = L.count[i - 1];
    const int64_t mv = m / EPV;
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, MapIdentity>), dim3((unsigned)L.count[i]), dim3(kRedBlock), 0,
                       stream, (const T*)buf[(i - 1) % 2], m, (int64_t)0, mv, buf[i % 2], (uint64_t*)nullptr);
  }
  if (out0 != (T*)dst)
    hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                       (const T*)buf[(L.nlev - 1) % 2], (int)L.count[L.nlev - 1], (T*)dst);
  return kf_check_launch("reduce_once_kernel");
}

// ---------------------------------------------------------------------------
// Two-array full reduction: dst = op_i f2(x[i], y[i]) with f2 = x*y (dot
// product) or (x-y)^2 (squared distance). Level 0 reads both arrays
// (one-shot when both are 16-byte aligned and contiguous, grid-stride
// otherwise); later levels reuse the partial reduction above.
// ---------------------------------------------------------------------------
struct Map2Mul {
  static constexpr bool kHasX = true;
  template <class T> __device__ static T apply(T a, T b) { return a * b; }
  __device__ static int32_t apply(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
  __device__ static int64_t apply(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
  __device__ static uint8_t apply(uint8_t a, uint8_t b) { return (uint8_t)(a * b); }
};
struct Map2SqDiff {
  static constexpr bool kHasX = true;
  template <class T> __device__ static T apply(T a, T b) { const T d = a - b; return d * d; }
  __device__ static int32_t apply(int32_t a, int32_t b) {
    const uint32_t d = (uint32_t)a - (uint32_t)b;
    return (int32_t)(d * d);
  }
  __device__ static int64_t apply(int64_t a, int64_t b) {
    const uint64_t d = (uint64_t)a - (uint64_t)b;
    return (int64_t)(d * d);
  }
  __device__ static uint8_t apply(uint8_t a, uint8_t b) { const uint8_t d = (uint8_t)(a - b); return (uint8_t)(d * d); }
};

// x * y * y (weighted sum of squares) and exp(x - y), the reference's
// mapreduce1d tests' other two-array maps (mapreduce1d_test.jl:117-131).
struct Map2WSq {
  template <class T> __device__ static T apply(T a, T b) { return Map2Mul::apply(Map2Mul::apply(a, b), b); }
};
struct Map2ExpDiff {
  __device__ static float apply(float a, float b) { return expf(a - b); }
  __device__ static double apply(double a, double b) { return exp(a - b); }
};

// x * y * z, the three-array map (wrapping for integers).
struct Map3Mul {
  template <class T> __device__ static T apply(T a, T b, T c) { return Map2Mul::apply(Map2Mul::apply(a, b), c); }
};

// K operand arrays of one multi-array reduction (K = 2 or 3), passed by value.
template <class T, int K> struct Operands {
  const T* p[K];
  int64_t s[K];
};
template <class M, class T, int K> __device__ inline T apply_k(const T (&v)[K]) {
  if constexpr (K == 2)
    return M::apply(v[0], v[1]);
  else
    return M::apply(v[0], v[1], v[2]);
}

// Multi-array reduction, vector path: the one-shot workgroups of
// reduce_once_kernel, each loading the same 16-byte vectors of all K arrays.
template <class T, class Op, class M, int K, bool FOLD = false>
__global__ __launch_bounds__(kRedBlock) void reducek_once_kernel(Operands<T, K> a, int64_t n, T* out,
                                                                 uint64_t* fold_hdr) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const int64_t nvec = n / EPV;
  const int64_t base = (int64_t)blockIdx.x * kOnceVecs + tid;
  uint4 r[kOnceUnroll][K];
#pragma unroll
  for (int u = 0; u < kOnceUnroll; ++u)
    if (base + u * kRedBlock < nvec) {
#pragma unroll
      for (int k = 0; k < K; ++k) r[u][k] = ld_stream(reinterpret_cast<const uint4*>(a.p[k]) + base + u * kRedBlock);
    }
  T acc_e[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc_e[e] = id;
#pragma unroll
  for (int u = 0; u < kOnceUnroll; ++u)
    if (base + u * kRedBlock < nvec) {
      T x[K][EPV];
#pragma unroll
      for (int k = 0; k < K; ++k) __builtin_memcpy(x[k], &r[u][k], 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        T v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] = x[k][e];
        acc_e[e] = Op::combine(acc_e[e], apply_k<M, T, K>(v));
      }
    }
  T acc = acc_e[0];
#pragma unroll
  for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, acc_e[e]);
  if (blockIdx.x == 0 && nvec * EPV + tid < n) {
    T v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = a.p[k][nvec * EPV + tid];
    acc = Op::combine(acc, apply_k<M, T, K>(v));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if constexpr (!FOLD) {
    if (tid == 0) out[blockIdx.x] = part;
  } else {
    fold_partial<T, Op>(part, out, fold_hdr, s_wave);  // out is the result
  }
}

// Multi-array reduction, strided operands: grid-stride loop.
template <class T, class Op, class M, int K>
__global__ __launch_bounds__(kRedBlock) void reducek_kernel(Operands<T, K> a, int64_t n, T* out) {
  __shared__ T s_wave[kRedWaves];
  T acc = Op::template identity<T>();
  const int64_t gsize = (int64_t)gridDim.x * kRedBlock;
  for (int64_t i = (int64_t)blockIdx.x * kRedBlock + threadIdx.x; i < n; i += gsize) {
    T v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = a.p[k][i * a.s[k]];
    acc = Op::combine(acc, apply_k<M, T, K>(v));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if (threadIdx.x == 0) out[blockIdx.x] = part;
}

template <class T, class Op, class M, int K>
int launch_reducek(const Operands<T, K>& a, int64_t n, void* dst, void* scratch_base, hipStream_t stream) {
  constexpr int EPV = 16 / (int)sizeof(T);
  void* scratch = red_work(scratch_base);
  bool vec = true;
  for (int k = 0; k < K; ++k) vec = vec && a.s[k] == 1 && (uintptr_t)a.p[k] % 16 == 0;
  if (!vec) {
    const int grid = reduce_grid<T>(n);
    T* out = grid == 1 ? (T*)dst : (T*)scratch;
    hipLaunchKernelGGL((reducek_kernel<T, Op, M, K>), dim3(grid), dim3(kRedBlock), 0, stream, a, n, out);
    if (grid > 1)
      hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                         (const T*)scratch, grid, (T*)dst);
    return kf_check_launch("reducek_kernel");
  }
  const OnceLevels L = once_levels(n / EPV, EPV);
  if (kUseFold && L.nlev == 1 && L.count[0] > 1 && L.count[0] <= kFoldMax) {
    hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K, true>), dim3((unsigned)L.count[0]), dim3(kRedBlock), 0,
                       stream, a, n, (T*)dst, (uint64_t*)scratch_base);
    return kf_check_launch("reducek_once_kernel");
  }
  size_t abytes = 0;
  for (int i = 0; i < L.nlev; i += 2) abytes = kmax(abytes, round256((size_t)L.count[i] * sizeof(T) + 16));
  T* buf[2] = {(T*)scratch, (T*)((uint8_t*)scratch + abytes)};
  T* out0 = (L.nlev == 1 && L.count[0] == 1) ? (T*)dst : buf[0];
  hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K>), dim3((unsigned)L.count[0]), dim3(kRedBlock), 0, stream,
                     a, n, out0, (uint64_t*)nullptr);
  for (int i = 1; i < L.nlev; ++i) {
    const int64_t m = L.count[i - 1];
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, MapIdentity>), dim3((unsigned)L.count[i]), dim3(kRedBlock), 0,
                       stream, (const T*)buf[(i - 1) % 2], m, (int64_t)0, m / EPV, buf[i % 2], (uint64_t*)nullptr);
  }
  if (out0 != (T*)dst)
    hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                       (const T*)buf[(L.nlev - 1) % 2], (int)L.count[L.nlev - 1], (T*)dst);
  return kf_check_launch("reducek_once_kernel");
}

template <class T, class Op, class M2>
int launch_reduce2(const void* x, int64_t xs, const void* y, int64_t ys, int64_t n, void* dst, void* scratch,
                   hipStream_t stream) {
  return launch_reducek<T, Op, M2, 2>(Operands<T, 2>{{(const T*)x, (const T*)y}, {xs, ys}}, n, dst, scratch,
                                      stream);
}

// ---------------------------------------------------------------------------
// dim = 1: one wave per column (a column of a column-major matrix is
// contiguous), optionally split into S row segments when there are too few
// columns to fill the GPU.
// ---------------------------------------------------------------------------
// Element function of the dims kernels: f(a) for a plain reduction, or
// f(a, x) with a vector operand x (matvec: x[j] per column; vecmat: x[i]
// per row).
template <class Map> struct Unary {
  static constexpr bool kHasX = false;
  template <class T> __device__ static T apply(T a, T) { return Map::apply(a); }
};

constexpr int kDimBlock = 256;
constexpr int kDimWaves = kDimBlock / kWave;
constexpr int kDimUnroll = 4;
constexpr int kScalarUnroll = 8;  // element (unaligned) paths: loads in flight per thread
constexpr int kDimMaxSplit = 64;          // dim 1 splits combined by combine_split_kernel
constexpr int kDimMaxSplitNarrow = 4096;  // dim 1 splits combined by reduce_rows_narrow_kernel
constexpr int kRowVecsDefault = 2;    // dim 2, unaligned path: elements per thread per column / 1
constexpr int kColUnrollDefault = 8;  // dim 2, unaligned path: columns per pass
constexpr int kDim2Blocks = 256;      // dim 2: target workgroups (one per CU)
// dim 2, aligned path: the widest strip (16-byte vectors per thread per
// column) that still gives kDim2Blocks workgroups; columns in flight per
// thread for each strip width.
constexpr int kDim2MaxRowVecs = 8;
constexpr int kColUnrollRv1 = 16;
constexpr int kColUnrollRv2 = 8;
constexpr int kColUnrollRv4 = 4;
constexpr int kColUnrollRv8 = 4;
constexpr int col_unroll_for(int rv) {
  return rv == 1 ? kColUnrollRv1 : rv == 2 ? kColUnrollRv2 : rv == 4 ? kColUnrollRv4 : kColUnrollRv8;
}

template <class T, class Op, class F>
__global__ __launch_bounds__(kDimBlock) void reduce_cols_kernel(
    const T* A, int64_t rows, int64_t cols, int64_t col_stride, T* out, int64_t out_stride,
    int64_t seg_rows, int vec, const T* xv, int64_t xs) {
  constexpr int EPV = 16 / (int)sizeof(T);
  const T id = Op::template identity<T>();
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int s = blockIdx.y;
  // grid-stride over blocks of kDimWaves columns (the grid is capped)
  for (int64_t col = (int64_t)blockIdx.x * kDimWaves + wave; col < cols; col += (int64_t)gridDim.x * kDimWaves) {
  T acc = id;
  const T* c = A + col * col_stride;
  const int64_t r0 = (int64_t)s * seg_rows;
  const int64_t r1 = kmin<int64_t>(rows, r0 + seg_rows);
  if (vec) {
    // seg_rows is a multiple of EPV and columns are 16-byte aligned.
    const int64_t nv = r1 > r0 ? (r1 - r0) / EPV : 0;
    const uint4* v = reinterpret_cast<const uint4*>(c + r0);
    const uint4* vx = reinterpret_cast<const uint4*>(xv + r0);  // used only with an operand (16-B aligned, xs = 1)
    T a[kDimUnroll][EPV];
#pragma unroll
    for (int u = 0; u < kDimUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[u][e] = id;
    int64_t i = lane;
    for (; i + (kDimUnroll - 1) * kWave < nv; i += kDimUnroll * kWave) {
      uint4 r[kDimUnroll], rx[kDimUnroll];
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u) {
        r[u] = ld_stream(v + i + u * kWave);
        if constexpr (F::kHasX) rx[u] = vx[i + u * kWave];
      }
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u) {
        T x[EPV], w[EPV];
        __builtin_memcpy(x, &r[u], 16);
        if constexpr (F::kHasX) __builtin_memcpy(w, &rx[u], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], F::apply(x[e], F::kHasX ? w[e] : x[e]));
      }
    }
    for (; i < nv; i += kWave) {
      const uint4 r = ld_stream(v + i);
      T x[EPV], w[EPV];
      __builtin_memcpy(x, &r, 16);
      if constexpr (F::kHasX) {
        const uint4 q = vx[i];
        __builtin_memcpy(w, &q, 16);
      }
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[0][e] = Op::combine(a[0][e], F::apply(x[e], F::kHasX ? w[e] : x[e]));
    }
#pragma unroll
    for (int u = 0; u < kDimUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc = Op::combine(acc, a[u][e]);
    const int64_t t = r0 + nv * EPV + lane;
    if (t < r1) acc = Op::combine(acc, F::apply(c[t], F::kHasX ? xv[t] : c[t]));
  } else {
    // element path: kScalarUnroll loads in flight per lane
    int64_t r = r0 + lane;
    for (; r + (kScalarUnroll - 1) * kWave < r1; r += kScalarUnroll * kWave) {
      T x[kScalarUnroll], w[kScalarUnroll];
#pragma unroll
      for (int u = 0; u < kScalarUnroll; ++u) {
        x[u] = c[r + u * kWave];
        w[u] = F::kHasX ? xv[(r + u * kWave) * xs] : x[u];
      }
#pragma unroll
      for (int u = 0; u < kScalarUnroll; ++u) acc = Op::combine(acc, F::apply(x[u], w[u]));
    }
    for (; r < r1; r += kWave) acc = Op::combine(acc, F::apply(c[r], F::kHasX ? xv[r * xs] : c[r]));
  }
  acc = wave_reduce<Op>(acc);
  // S == 1: out is dst; otherwise out is partials[s*cols + col]
  if (lane == 0) out[gridDim.y == 1 ? col * out_stride : (int64_t)s * cols + col] = acc;
  }
}

// Combine of x over aligned groups of L lanes (L a power of two <= 64),
// lower lanes on the left; the result is valid in each group's first lane.
template <class T> __device__ inline T shfl_xor_t(T v, int m) {
  Words<T> w = to_words(v), r;
#pragma unroll
  for (int i = 0; i < Words<T>::W; ++i) r.w[i] = (uint32_t)__shfl_xor((int)w.w[i], m, kWave);
  return from_words<T>(r);
}
template <class Op, int L, class T> __device__ inline T group_reduce(T x) {
  const int lane = lane_id();
#pragma unroll
  for (int m = 1; m < L; m <<= 1) {
    const T y = shfl_xor_t(x, m);
    x = (lane & m) ? Op::combine(y, x) : Op::combine(x, y);
  }
  return x;
}

// dim = 1, short columns: L lanes per column (kDimBlock / L columns per
// workgroup pass), each lane combining units j, j+L, ... of its column
// (16-byte vectors when VEC: rows % EPV == 0 and aligned columns; elements
// otherwise), then a combine over the L lanes. Grid-stride over column
// blocks, so any column count fits one capped grid.
constexpr int kSegElemsPerLane = 4;  // target element units per lane (16-byte units: 1)
constexpr int kSegMaxLanesVec = 8, kSegMaxLanesElem = 16;
constexpr int kSegMaxUnitsVec = 128, kSegMaxUnitsElem = 256;  // longer columns take one wave each
constexpr int kSegMaxBlocks = 8192;
template <class T, class Op, class F, bool VEC, int L>
__global__ __launch_bounds__(kDimBlock) void reduce_cols_seg_kernel(const T* A, int64_t rows, int64_t cols,
                                                                    int64_t col_stride, T* out, int64_t out_stride,
                                                                    const T* xv, int64_t xs) {
  constexpr int EPV = VEC ? 16 / (int)sizeof(T) : 1;
  constexpr int CPB = kDimBlock / L;
  constexpr int U = 4;
  const T id = Op::template identity<T>();
  const int j = threadIdx.x % L;
  const int64_t nu = rows / EPV;  // VEC: rows % EPV == 0
  for (int64_t cb = (int64_t)blockIdx.x * CPB; cb < cols; cb += (int64_t)gridDim.x * CPB) {
    const int64_t col = cb + threadIdx.x / L;
    T acc = id;
    if (col < cols) {
      const T* c = A + col * col_stride;
      T a[EPV];
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = id;
      int64_t i = j;
      for (; i + (U - 1) * L < nu; i += U * L) {
        if constexpr (VEC) {
          uint4 r[U], rx[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            r[u] = ld_stream(reinterpret_cast<const uint4*>(c) + i + u * L);
            if constexpr (F::kHasX) rx[u] = reinterpret_cast<const uint4*>(xv)[i + u * L];
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            T x[EPV], w[EPV];
            __builtin_memcpy(x, &r[u], 16);
            if constexpr (F::kHasX) __builtin_memcpy(w, &rx[u], 16);
#pragma unroll
            for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], F::apply(x[e], F::kHasX ? w[e] : x[e]));
          }
        } else {
          T x[U], w[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            x[u] = c[i + u * L];
            if constexpr (sizeof(T) == 1) {
              // one byte per register: keeps adjacent byte loads from being
              // fused into a sub-dword vector the backend cannot split
              uint32_t b = x[u];
              __asm__ volatile("" : "+v"(b));
              x[u] = (T)b;
            }
            w[u] = F::kHasX ? xv[(i + u * L) * xs] : x[u];
          }
#pragma unroll
          for (int u = 0; u < U; ++u) a[0] = Op::combine(a[0], F::apply(x[u], w[u]));
        }
      }
      for (; i < nu; i += L) {
        if constexpr (VEC) {
          const uint4 r = ld_stream(reinterpret_cast<const uint4*>(c) + i);
          T x[EPV], w[EPV];
          __builtin_memcpy(x, &r, 16);
          if constexpr (F::kHasX) {
            const uint4 q = reinterpret_cast<const uint4*>(xv)[i];
            __builtin_memcpy(w, &q, 16);
          }
#pragma unroll
          for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], F::apply(x[e], F::kHasX ? w[e] : x[e]));
        } else {
          a[0] = Op::combine(a[0], F::apply(c[i], F::kHasX ? xv[i * xs] : c[i]));
        }
      }
      acc = a[0];
#pragma unroll
      for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, a[e]);
    }
    acc = group_reduce<Op, L>(acc);
    if (j == 0 && col < cols) out[col * out_stride] = acc;
  }
}

// ---------------------------------------------------------------------------
// dim = 2: a workgroup owns a strip of 256*kRowVecs*EPV rows (4-32 KiB of
// each column; thread t holds vectors t, t+256, ... of the strip) and a range
// of columns, which it walks kColUnroll at a time, so every load is part of a
// contiguous run of the strip's width. Strips are split over S column ranges
// whose partials stage 2 combines.
// ---------------------------------------------------------------------------
template <class T, class Op, class F, bool VEC, int kRowVecs = kRowVecsDefault, int kColUnroll = kColUnrollDefault>
__global__ __launch_bounds__(kDimBlock) void reduce_rows_kernel(
    const T* A, int64_t rows, int64_t cols, int64_t col_stride, T* out, int64_t out_stride, int64_t seg_cols,
    int64_t a_bstride, int64_t out_bstride, const T* xv, int64_t xs) {
  constexpr int EPV = VEC ? 16 / (int)sizeof(T) : 1;
  // batch z = blockIdx.z: one (rows x cols) matrix per batch entry
  A += (int64_t)blockIdx.z * a_bstride;
  out += gridDim.y == 1 ? (int64_t)blockIdx.z * out_bstride : (int64_t)blockIdx.z * gridDim.y * rows;
  constexpr int RS = kDimBlock * kRowVecs * EPV;
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const int s = blockIdx.y;
  const int64_t strip = (int64_t)blockIdx.x * RS;
  const int64_t c0 = (int64_t)s * seg_cols;
  const int64_t c1 = kmin<int64_t>(cols, c0 + seg_cols);

  T a[kRowVecs][EPV];
#pragma unroll
  for (int u = 0; u < kRowVecs; ++u)
#pragma unroll
    for (int e = 0; e < EPV; ++e) a[u][e] = id;
  const bool full = strip + RS <= rows;
  if (VEC && full) {
    const T* p = A + strip;
    int64_t c = c0;
    for (; c + kColUnroll <= c1; c += kColUnroll) {
      uint4 r[kColUnroll][kRowVecs];
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q)
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u)
          r[q][u] = ld_stream(reinterpret_cast<const uint4*>(p + (c + q) * col_stride) + u * kDimBlock + tid);
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q) {
        const T w = F::kHasX ? xv[(c + q) * xs] : id;
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u) {
          T x[EPV];
          __builtin_memcpy(x, &r[q][u], sizeof(x));
#pragma unroll
          for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], F::apply(x[e], w));
        }
      }
    }
    for (; c < c1; ++c) {
      const T w = F::kHasX ? xv[c * xs] : id;
#pragma unroll
      for (int u = 0; u < kRowVecs; ++u) {
        const uint4 r = ld_stream(reinterpret_cast<const uint4*>(p + c * col_stride) + u * kDimBlock + tid);
        T x[EPV];
        __builtin_memcpy(x, &r, sizeof(x));
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], F::apply(x[e], w));
      }
    }
  } else {
    // element path (unaligned, or the ragged last strip): kColUnroll
    // columns of loads in flight; rows past the end read row 0's element and
    // drop it
    int64_t c = c0;
    if constexpr (!VEC)  // the aligned kernel takes this branch only for its one ragged strip
    for (; c + kColUnroll <= c1; c += kColUnroll) {
      T x[kColUnroll][kRowVecs][EPV];
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q)
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u)
#pragma unroll
          for (int e = 0; e < EPV; ++e) {
            const int64_t r = strip + (int64_t)(u * kDimBlock + tid) * EPV + e;
            x[q][u][e] = A[(r < rows ? r : 0) + (c + q) * col_stride];
          }
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q) {
        const T w = F::kHasX ? xv[(c + q) * xs] : id;
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u)
#pragma unroll
          for (int e = 0; e < EPV; ++e)
            if (strip + (int64_t)(u * kDimBlock + tid) * EPV + e < rows)
              a[u][e] = Op::combine(a[u][e], F::apply(x[q][u][e], w));
      }
    }
    for (; c < c1; ++c)
#pragma unroll
      for (int u = 0; u < kRowVecs; ++u)
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          const int64_t r = strip + (int64_t)(u * kDimBlock + tid) * EPV + e;
          if (r < rows) a[u][e] = Op::combine(a[u][e], F::apply(A[r + c * col_stride], F::kHasX ? xv[c * xs] : id));
        }
  }
#pragma unroll
  for (int u = 0; u < kRowVecs; ++u)
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const int64_t r = strip + (int64_t)(u * kDimBlock + tid) * EPV + e;
      if (r < rows) out[gridDim.y == 1 ? r * out_stride : (int64_t)s * rows + r] = a[u][e];
    }
}


// dim = 2, narrow matrices (at most kDimBlock row units: 16-byte vectors
// when VEC, i.e. rows % EPV == 0 and aligned columns, else elements): the
// workgroup is split into P = kDimBlock / units column phases; thread
// (unit, phase) walks columns phase, phase + P, ... of its column range, kNarrowUnroll
// loads in flight, and the phases are combined in order through LDS. Also
// the second stage of split reductions: the S partial columns are a
// rows x S matrix reduced along dim 2 the same way.
constexpr int kNarrowUnroll = 8;
constexpr int kNarrowBlocks = 512;  // target workgroups over batch x column ranges
template <class T, class Op, class F, bool VEC>
__global__ __launch_bounds__(kDimBlock) void reduce_rows_narrow_kernel(
    const T* A, int64_t rows, int64_t cols, int64_t col_stride, T* out, int64_t out_stride, int64_t seg_cols,
    int64_t a_bstride, int64_t out_bstride, const T* xv, int64_t xs) {
  constexpr int EPV = VEC ? 16 / (int)sizeof(T) : 1;
  constexpr int U = kNarrowUnroll;
  __shared__ T s_acc[kDimBlock * EPV];
  A += (int64_t)blockIdx.z * a_bstride;
  out += gridDim.y == 1 ? (int64_t)blockIdx.z * out_bstride : (int64_t)blockIdx.z * gridDim.y * rows;
  const T id = Op::template identity<T>();
  const int nunits = (int)(rows / EPV);  // <= kDimBlock (host-checked)
  const int P = kDimBlock / nunits;
  const int t = threadIdx.x;
  const int unit = t % nunits, ph = t / nunits;
  const int64_t c0 = (int64_t)blockIdx.y * seg_cols;
  const int64_t c1 = kmin<int64_t>(cols, c0 + seg_cols);
  T a[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) a[e] = id;
  if (ph < P) {
    const T* p = A + (int64_t)unit * EPV;
    int64_t c = c0 + ph;
    for (; c + (int64_t)(U - 1) * P < c1; c += (int64_t)U * P) {
      if constexpr (VEC) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = ld_stream(reinterpret_cast<const uint4*>(p + (c + (int64_t)u * P) * col_stride));
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const T w = F::kHasX ? xv[(c + (int64_t)u * P) * xs] : id;
          T x[EPV];
          __builtin_memcpy(x, &r[u], 16);
#pragma unroll
          for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], F::apply(x[e], w));
        }
      } else {
        T x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = p[(c + (int64_t)u * P) * col_stride];
#pragma unroll
        for (int u = 0; u < U; ++u) a[0] = Op::combine(a[0], F::apply(x[u], F::kHasX ? xv[(c + (int64_t)u * P) * xs] : id));
      }
    }
    for (; c < c1; c += P) {
      const T w = F::kHasX ? xv[c * xs] : id;
      if constexpr (VEC) {
        const uint4 r = ld_stream(reinterpret_cast<const uint4*>(p + c * col_stride));
        T x[EPV];
        __builtin_memcpy(x, &r, 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], F::apply(x[e], w));
      } else {
        a[0] = Op::combine(a[0], F::apply(p[c * col_stride], w));
      }
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) s_acc[t * EPV + e] = a[e];
  }
  __syncthreads();
  if (t < nunits) {
    // phases in column order: phase q holds columns q, q + P, ...; every op
    // here is commutative, and phase order keeps the combine deterministic
#pragma unroll
    for (int e = 0; e < EPV; ++e) a[e] = s_acc[t * EPV + e];
    for (int q = 1; q < P; ++q)
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], s_acc[(q * nunits + t) * EPV + e]);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const int64_t r = (int64_t)t * EPV + e;
      out[gridDim.y == 1 ? r * out_stride : (int64_t)blockIdx.y * rows + r] = a[e];
    }
  }
}

struct DimPlan {
  int64_t groups;  // column groups (dim 1) or row strips (dim 2)
  int split;       // S workgroups cooperating on one group
  int row_vecs;    // dim 2: strip width in vectors (elements on the unaligned path) per thread
  int seg_lanes;   // dim 1: lanes per column of reduce_cols_seg_kernel (0: one wave per column)
  bool narrow;     // dim 2: reduce_rows_narrow_kernel
  bool unit_vec;   // seg / narrow kernels: 16-byte units (rows % EPV == 0, aligned columns)
  size_t partial_bytes;
};

// Launch plan; a pure function of (element size, shape, dim, alignment) so
// the scratch query and the launch agree.
constexpr int64_t kMaxBatchPerLaunch = 65535;  // grid.z limit

// Row units of an m-row operand for the seg / narrow kernels: 16-byte
// vectors when m is a multiple of the vector width (and the columns are
// aligned), else elements.
inline int64_t row_units(size_t es, int64_t m, bool aligned) {
  const int64_t ev = (int64_t)(16 / es);
  return aligned && m % ev == 0 ? m / ev : m;
}
constexpr int64_t kColsMaxBlocks = 65536;  // wave-per-column grid cap (grid-stride beyond)

inline DimPlan plan_dim(size_t es, int64_t rows, int64_t cols, int dim, bool vec, int64_t batch = 1) {
  const int64_t nb = kmin<int64_t>(kmax<int64_t>(batch, 1), kMaxBatchPerLaunch);
  DimPlan p{};
  const int epv = vec ? (int)(16 / es) : 1;
  if (dim == 1) {
    // Short columns: L lanes per column, one 16-byte unit or about
    // kSegElemsPerLane elements each, at most 8 (16) lanes. Float32, 1 GiB:
    // 16 rows 5.7 TB/s at 4 lanes against 3.5 at 1; 64 rows 6.2 at 8 lanes
    // against 5.7 at 16; unaligned 16 rows 5.4 at 4 lanes against 2.5 at
    // 16; unaligned 128 rows 5.8 at 16 lanes against 5.1 at 8; unaligned
    // 256 rows 6.1 here against 3.3 with a wave per column, while aligned
    // 1024 rows stay faster with a wave per column (6.8 against 6.4).
    const int64_t nu = row_units(es, rows, vec);
    const bool uv = vec && nu != rows;
    const int64_t per = uv ? 1 : kSegElemsPerLane;
    const int max_lanes = uv ? kSegMaxLanesVec : kSegMaxLanesElem;
    int L = 1;
    while (L < max_lanes && (int64_t)L * per < nu) L <<= 1;
    if (nu <= (uv ? kSegMaxUnitsVec : kSegMaxUnitsElem)) {
      p.seg_lanes = L;
      p.unit_vec = uv;
      p.groups = kmin<int64_t>((cols + kDimBlock / L - 1) / (kDimBlock / L), kSegMaxBlocks);
      p.split = 1;
    } else {
      p.groups = kmin<int64_t>((cols + kDimWaves - 1) / kDimWaves, kColsMaxBlocks);
      int64_t S = 1;
      if (cols < 16384) {
        // The split partials are a cols x S matrix; when it is narrow its
        // combine is reduce_rows_narrow_kernel and S may be large (few long
        // columns), else the serial combine_split_kernel keeps S small.
        const bool narrow2 = row_units(es, cols, true) <= kDimBlock;
        S = (16384 + cols - 1) / cols;
        const int64_t by_rows = rows / ((int64_t)kWave * 4 * kDimUnroll * 4);  // >= 4 unrolled passes each
        S = kmin<int64_t>(S, kmax<int64_t>(by_rows, 1));
        S = kmin<int64_t>(S, narrow2 ? kDimMaxSplitNarrow : kDimMaxSplit);
      }
      p.split = (int)S;
    }
  } else if (row_units(es, rows, vec) <= kDimBlock) {
    // Narrow: one strip covers every row; column ranges fill the GPU.
    const int64_t nu = row_units(es, rows, vec);
    p.narrow = true;
    p.unit_vec = vec && nu != rows;
    p.groups = 1;
    const int64_t P = kDimBlock / nu;
    int64_t S = (kNarrowBlocks + nb - 1) / nb;
    S = kmin<int64_t>(S, kmax<int64_t>(cols / (2 * kNarrowUnroll * P), 1));
    p.split = (int)kmin<int64_t>(S, 65535);
  } else {
    // Aligned path: the widest strip that still leaves one workgroup per
    // CU, so each workgroup streams the longest contiguous runs; with too
    // few rows even for 1-vector strips, columns are split instead.
    // Float32: 4M x 64 6.8 TB/s at 8 vectors (512 workgroups) against 5.7
    // at 2; 1M x 256 7.1 at 4 against 5.6 at 2; 65536 x 4096 6.8 at 1 (S = 4)
    // against 6.6 at 2 (S = 8) and 6.1 at 4 (S = 16).
    int rv = kRowVecsDefault;
    if (vec) {
      rv = 1;
      for (int c = kDim2MaxRowVecs; c > 1; c /= 2) {
        const int64_t rsc = (int64_t)kDimBlock * c * epv;
        if ((rows + rsc - 1) / rsc * nb >= kDim2Blocks) {
          rv = c;
          break;
        }
      }
    }
    p.row_vecs = rv;
    const int cu = vec ? col_unroll_for(rv) : kColUnrollDefault;
    const int64_t rs = (int64_t)kDimBlock * rv * epv;
    p.groups = (rows + rs - 1) / rs;
    int64_t S = 1;
    if (p.groups * nb < kDim2Blocks) {
      S = (kDim2Blocks + p.groups * nb - 1) / (p.groups * nb);
      S = kmin<int64_t>(S, kmax<int64_t>(cols / (2 * cu), 1));
      S = kmin<int64_t>(S, 256);
    }
    p.split = (int)S;
  }
  if (p.split > 1) p.partial_bytes = round256((size_t)p.split * (size_t)(dim == 1 ? cols : rows) * es * (size_t)nb);
  return p;
}

inline bool dim_vec_ok(const void* A, int64_t cs, size_t es) {
  return ((uintptr_t)A % 16 == 0) && ((cs * (int64_t)es) % 16 == 0);
}

template <class T, class Op, class F>
void launch_narrow(bool unit_vec, dim3 grid, const T* A, int64_t rows, int64_t cols, int64_t cs, T* out, int64_t ods,
                   int64_t seg, int64_t a_bstride, int64_t out_bstride, const T* x, int64_t xs, hipStream_t stream) {
  if (unit_vec)
    hipLaunchKernelGGL((reduce_rows_narrow_kernel<T, Op, F, true>), grid, dim3(kDimBlock), 0, stream, A, rows, cols,
                       cs, out, ods, seg, a_bstride, out_bstride, x, xs);
  else
    hipLaunchKernelGGL((reduce_rows_narrow_kernel<T, Op, F, false>), grid, dim3(kDimBlock), 0, stream, A, rows, cols,
                       cs, out, ods, seg, a_bstride, out_bstride, x, xs);
}

// Second stage of a split dims reduction: nz batches of an m x S partial
// matrix (column s at s*m, batch z at z*S*m; the scratch is 256-byte
// aligned) reduced along dim 2 into dst[i*ds + z*dst_bstride].
template <class T, class Op>
void launch_combine(const T* part, int S, int64_t m, T* dst, int64_t ds, int64_t dst_bstride, unsigned nz,
                    hipStream_t stream) {
  const int64_t nu = row_units(sizeof(T), m, true);
  if (nu <= kDimBlock)
    launch_narrow<T, Op, Unary<MapIdentity>>(nu != m, dim3(1, 1, nz), part, m, S, m, dst, ds, S, (int64_t)S * m,
                                             dst_bstride, nullptr, 0, stream);
  else
    hipLaunchKernelGGL((combine_split_kernel<T, Op>), dim3((unsigned)((m + kRedBlock - 1) / kRedBlock), nz),
                       dim3(kRedBlock), 0, stream, part, S, m, dst, ds, dst_bstride);
}

template <class T, class Op, class F>
int launch_reduce_dim(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst,
                      int64_t ds, void* scratch, hipStream_t stream, int64_t batch = 1, int64_t a_bstride = 0,
                      const void* x = nullptr, int64_t xs = 0) {
  bool vec = dim_vec_ok(A, cs, sizeof(T)) && (batch == 1 || (a_bstride * (int64_t)sizeof(T)) % 16 == 0);
  // vecmat (dim 1 with an operand) reads x along the rows: same vector path only if x is too
  if (F::kHasX && dim == 1) vec = vec && xs == 1 && (uintptr_t)x % 16 == 0;
  const DimPlan p = plan_dim(sizeof(T), rows, cols, dim, vec, batch);
  if (dim == 1) {
    if (p.seg_lanes) {
      const dim3 grid((unsigned)p.groups);
#define KF_SEG(V, L)                                                                                          \
  hipLaunchKernelGGL((reduce_cols_seg_kernel<T, Op, F, V, L>), grid, dim3(kDimBlock), 0, stream, (const T*)A, rows, \
                     cols, cs, (T*)dst, ds, (const T*)x, xs)
#define KF_SEG_L(V)                    \
  switch (p.seg_lanes) {               \
    case 1: KF_SEG(V, 1); break;       \
    case 2: KF_SEG(V, 2); break;       \
    case 4: KF_SEG(V, 4); break;       \
    case 8: KF_SEG(V, 8); break;       \
    default: KF_SEG(V, 16); break;     \
  }
      if (p.unit_vec) {
        KF_SEG_L(true)
      } else {
        KF_SEG_L(false)
      }
#undef KF_SEG_L
#undef KF_SEG
      return kf_check_launch("reduce_cols_seg_kernel");
    }
    T* out = p.split > 1 ? (T*)scratch : (T*)dst;
    constexpr int EPV = 16 / (int)sizeof(T);
    int64_t seg = (rows + p.split - 1) / p.split;
    seg = (seg + EPV - 1) / EPV * EPV;
    hipLaunchKernelGGL((reduce_cols_kernel<T, Op, F>), dim3((unsigned)p.groups, p.split), dim3(kDimBlock), 0,
                       stream, (const T*)A, rows, cols, cs, out, ds, seg, (int)vec, (const T*)x, xs);
    if (p.split > 1) launch_combine<T, Op>((const T*)scratch, p.split, cols, (T*)dst, ds, 0, 1, stream);
    return kf_check_launch("reduce_cols_kernel");
  }
  // dim 2, batched: dst[(i + z*rows)*ds] = op_j f(A[i + j*cs + z*a_bstride])
  const int64_t seg = (cols + p.split - 1) / p.split;
  const int64_t dst_bstride = rows * ds;
  for (int64_t z0 = 0; z0 < batch; z0 += kMaxBatchPerLaunch) {
    const unsigned nz = (unsigned)kmin<int64_t>(kMaxBatchPerLaunch, batch - z0);
    const T* Az = (const T*)A + z0 * a_bstride;
    T* dz = (T*)dst + z0 * dst_bstride;
    T* out = p.split > 1 ? (T*)scratch : dz;
    const dim3 grid((unsigned)p.groups, p.split, nz);
    if (p.narrow) {
      launch_narrow<T, Op, F>(p.unit_vec, grid, Az, rows, cols, cs, out, ds, seg, a_bstride, dst_bstride, (const T*)x,
                              xs, stream);
      if (p.split > 1) launch_combine<T, Op>((const T*)scratch, p.split, rows, dz, ds, dst_bstride, nz, stream);
      continue;
    }
#define KF_ROWS_VEC(RV)                                                                                  \
  hipLaunchKernelGGL((reduce_rows_kernel<T, Op, F, true, RV, col_unroll_for(RV)>), grid, dim3(kDimBlock), 0, stream, \
                     Az, rows, cols, cs, out, ds, seg, a_bstride, dst_bstride, (const T*)x, xs)
    if (vec) {
      switch (p.row_vecs) {
        case 1: KF_ROWS_VEC(1); break;
        case 2: KF_ROWS_VEC(2); break;
        case 4: KF_ROWS_VEC(4); break;
        default: KF_ROWS_VEC(8); break;
      }
    } else
      hipLaunchKernelGGL((reduce_rows_kernel<T, Op, F, false>), grid, dim3(kDimBlock), 0, stream, Az, rows, cols,
                         cs, out, ds, seg, a_bstride, dst_bstride, (const T*)x, xs);
    if (p.split > 1) launch_combine<T, Op>((const T*)scratch, p.split, rows, dz, ds, dst_bstride, nz, stream);
  }
#undef KF_ROWS_VEC
  return kf_check_launch("reduce_rows_kernel");
}

// ---------------------------------------------------------------------------
// Dispatch over (dtype, op, map).
// ---------------------------------------------------------------------------
template <class T, template <class, class, class> class L, class... A>
int dispatch_op_map(kf_op op, kf_map f, A... args) {
  if (f == KF_MAP_ABS2) {
    switch (op) {
      case KF_OP_ADD: return L<T, OpAdd, MapAbs2>::run(args...);
      case KF_OP_MAX: return L<T, OpMax, MapAbs2>::run(args...);
      case KF_OP_MUL: return L<T, OpMul, MapAbs2>::run(args...);
      default: return L<T, OpMin, MapAbs2>::run(args...);
    }
  }
  switch (op) {
    case KF_OP_ADD: return L<T, OpAdd, MapIdentity>::run(args...);
    case KF_OP_MAX: return L<T, OpMax, MapIdentity>::run(args...);
    case KF_OP_MUL: return L<T, OpMul, MapIdentity>::run(args...);
    default: return L<T, OpMin, MapIdentity>::run(args...);
  }
}

template <template <class, class, class> class L, class... A>
int dispatch_all(kf_dtype dt, kf_op op, kf_map f, A... args) {
  switch (dt) {
    case KF_F32: return dispatch_op_map<float, L>(op, f, args...);
    case KF_F64: return dispatch_op_map<double, L>(op, f, args...);
    case KF_I32: return dispatch_op_map<int32_t, L>(op, f, args...);
    case KF_I64: return dispatch_op_map<int64_t, L>(op, f, args...);
    case KF_U8: return dispatch_op_map<uint8_t, L>(op, f, args...);
    default: return kf_set_error(KF_EINVAL, "bad dtype %d", (int)dt);
  }
}

template <class T, class Op, class Map> struct ReduceL {
  static int run(const void* src, int64_t n, int64_t stride, void* dst, void* scratch, hipStream_t s) {
    return launch_reduce<T, Op, Map>(src, n, stride, dst, scratch, s);
  }
};
template <class T, class Op, class Map2> struct Reduce2L {
  static int run(const void* x, int64_t xs, const void* y, int64_t ys, int64_t n, void* dst, void* scratch,
                 hipStream_t s) {
    return launch_reduce2<T, Op, Map2>(x, xs, y, ys, n, dst, scratch, s);
  }
};
template <class T, class Op, class Map> struct ReduceDimL {
  static int run(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst, int64_t ds,
                 void* scratch, hipStream_t s, int64_t batch, int64_t a_bstride) {
    return launch_reduce_dim<T, Op, Unary<Map>>(A, rows, cols, cs, dim, dst, ds, red_work(scratch), s, batch,
                                                a_bstride);
  }
};

// ---------------------------------------------------------------------------
// Post-map and scratch fill.
// ---------------------------------------------------------------------------
struct PostSqrt {
  __device__ static float apply(float x) { return __builtin_sqrtf(x); }
  __device__ static double apply(double x) { return __builtin_sqrt(x); }
};
template <class T, class G>
__global__ __launch_bounds__(256) void post_map_kernel(T* x, int64_t n, int64_t stride) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gsize)
    x[i * stride] = G::apply(x[i * stride]);
}

__global__ void fill_zero_kernel(uint8_t* p, int64_t n) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gsize) p[i] = 0;
}

}  // namespace kf

using namespace kf;

extern "C" size_t kf_reduce_scratch_bytes(kf_dtype dt, int64_t n) {
  (void)n;
  size_t es = kf_dtype_size(dt);
  if (es == 0) es = 8;
  return reduce_scratch(es, kmax<int64_t>(n, 1));
}

extern "C" int kf_reduce(kf_op op, kf_map f, kf_dtype dt, const void* src, int64_t n, int64_t stride,
                         void* dst, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!src || !dst) return kf_set_error(KF_EINVAL, "kf_reduce: null src or dst");
  if (stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce: stride must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)src % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce: src/dst not aligned to the element type");
  const size_t need = kf_reduce_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce: scratch must be 256-byte aligned");
  return dispatch_all<ReduceL>(dt, op, f, src, n, stride, dst, scratch, (hipStream_t)stream);
}

extern "C" size_t kf_reduce2_scratch_bytes(kf_dtype dt, int64_t n) { return kf_reduce_scratch_bytes(dt, n); }

template <class T, class M2, class... A> int dispatch_reduce2_op(kf_op op, A... args) {
  switch (op) {
    case KF_OP_ADD: return Reduce2L<T, OpAdd, M2>::run(args...);
    case KF_OP_MAX: return Reduce2L<T, OpMax, M2>::run(args...);
    case KF_OP_MUL: return Reduce2L<T, OpMul, M2>::run(args...);
    default: return Reduce2L<T, OpMin, M2>::run(args...);
  }
}

template <class T, class... A> int dispatch_reduce2(kf_op op, kf_map2 f, A... args) {
  switch (f) {
    case KF_MAP2_SQDIFF: return dispatch_reduce2_op<T, Map2SqDiff>(op, args...);
    case KF_MAP2_WSQ: return dispatch_reduce2_op<T, Map2WSq>(op, args...);
    case KF_MAP2_EXPDIFF:
      if constexpr (__is_same(T, float) || __is_same(T, double)) return dispatch_reduce2_op<T, Map2ExpDiff>(op, args...);
      return kf_set_error(KF_EINVAL, "kf_reduce2: exp(x - y) needs a floating-point type");
    default: return dispatch_reduce2_op<T, Map2Mul>(op, args...);
  }
}

extern "C" int kf_reduce2(kf_op op, kf_map2 f, kf_dtype dt, const void* x, int64_t x_stride, const void* y,
                          int64_t y_stride, int64_t n, void* dst, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, KF_MAP_IDENTITY, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (f != KF_MAP2_MUL && f != KF_MAP2_SQDIFF && f != KF_MAP2_WSQ && f != KF_MAP2_EXPDIFF)
    return kf_set_error(KF_EINVAL, "kf_reduce2: unknown map %d", (int)f);
  if (f == KF_MAP2_EXPDIFF && dt != KF_F32 && dt != KF_F64)
    return kf_set_error(KF_EINVAL, "kf_reduce2: exp(x - y) needs a floating-point type");
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce2: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!x || !y || !dst) return kf_set_error(KF_EINVAL, "kf_reduce2: null pointer");
  if (x_stride < 1 || y_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce2: strides must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)x % es || (uintptr_t)y % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce2: pointers not aligned to the element type");
  const size_t need = kf_reduce2_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce2: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce2: scratch must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  switch (dt) {
    case KF_F32: return dispatch_reduce2<float>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_F64: return dispatch_reduce2<double>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_I32: return dispatch_reduce2<int32_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_I64: return dispatch_reduce2<int64_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_U8: return dispatch_reduce2<uint8_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    default: return kf_set_error(KF_EINVAL, "kf_reduce2: bad dtype %d", (int)dt);
  }
}

extern "C" size_t kf_reduce3_scratch_bytes(kf_dtype dt, int64_t n) { return kf_reduce_scratch_bytes(dt, n); }

template <class T>
int dispatch_reduce3(kf_op op, const Operands<T, 3>& a, int64_t n, void* dst, void* scratch, hipStream_t s) {
  switch (op) {
    case KF_OP_ADD: return launch_reducek<T, OpAdd, Map3Mul, 3>(a, n, dst, scratch, s);
    case KF_OP_MAX: return launch_reducek<T, OpMax, Map3Mul, 3>(a, n, dst, scratch, s);
    case KF_OP_MUL: return launch_reducek<T, OpMul, Map3Mul, 3>(a, n, dst, scratch, s);
    default: return launch_reducek<T, OpMin, Map3Mul, 3>(a, n, dst, scratch, s);
  }
}

extern "C" int kf_reduce3(kf_op op, kf_map3 f, kf_dtype dt, const void* x, int64_t x_stride, const void* y,
                          int64_t y_stride, const void* z, int64_t z_stride, int64_t n, void* dst, void* scratch,
                          size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, KF_MAP_IDENTITY, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (f != KF_MAP3_MUL) return kf_set_error(KF_EINVAL, "kf_reduce3: unknown map %d", (int)f);
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce3: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!x || !y || !z || !dst) return kf_set_error(KF_EINVAL, "kf_reduce3: null pointer");
  if (x_stride < 1 || y_stride < 1 || z_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce3: strides must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)x % es || (uintptr_t)y % es || (uintptr_t)z % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce3: pointers not aligned to the element type");
  const size_t need = kf_reduce3_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce3: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce3: scratch must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
#define KF_R3(T) \
  dispatch_reduce3<T>(op, Operands<T, 3>{{(const T*)x, (const T*)y, (const T*)z}, {x_stride, y_stride, z_stride}}, \
                      n, dst, scratch, s)
  switch (dt) {
    case KF_F32: return KF_R3(float);
    case KF_F64: return KF_R3(double);
    case KF_I32: return KF_R3(int32_t);
    case KF_I64: return KF_R3(int64_t);
    case KF_U8: return KF_R3(uint8_t);
    default: return kf_set_error(KF_EINVAL, "kf_reduce3: bad dtype %d", (int)dt);
  }
#undef KF_R3
}

extern "C" size_t kf_reduce_dim_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int dim) {
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || rows <= 0 || cols <= 0 || (dim != 1 && dim != 2)) return 256;
  // the plan depends on alignment: reserve for the larger of the two
  const DimPlan pv = plan_dim(es, rows, cols, dim, true), ps = plan_dim(es, rows, cols, dim, false);
  return kRedReserved + kmax<size_t>(256, kmax<size_t>(pv.partial_bytes, ps.partial_bytes));
}

extern "C" int kf_reduce_dim(kf_op op, kf_map f, kf_dtype dt, const void* A, int64_t rows, int64_t cols,
                             int64_t col_stride, int dim, void* dst, int64_t dst_stride, void* scratch,
                             size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (dim != 1 && dim != 2) return kf_set_error(KF_EINVAL, "kf_reduce_dim: dim must be 1 or 2 (got %d)", dim);
  if (rows < 0 || cols < 0) return kf_set_error(KF_EINVAL, "kf_reduce_dim: negative shape");
  if (rows == 0 || cols == 0) {
    if ((dim == 1 ? cols : rows) != 0)
      return kf_set_error(KF_EINVAL, "kf_reduce_dim: reducing an empty dimension has no identity-free result");
    return KF_OK;
  }
  if (!A || !dst) return kf_set_error(KF_EINVAL, "kf_reduce_dim: null A or dst");
  if (col_stride < rows) return kf_set_error(KF_EINVAL, "kf_reduce_dim: col_stride < rows");
  if (dst_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce_dim: dst_stride must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)A % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim: A/dst not aligned to the element type");
  const size_t need = kf_reduce_dim_scratch_bytes(dt, rows, cols, dim);
  const DimPlan p = plan_dim(es, rows, cols, dim, dim_vec_ok(A, col_stride, es));
  if (p.split > 1) {
    if (!scratch || scratch_bytes < need)
      return kf_set_error(KF_ENOSCRATCH, "kf_reduce_dim: scratch of %zu bytes needed, %zu given", need,
                          scratch ? scratch_bytes : (size_t)0);
    if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce_dim: scratch must be 256-byte aligned");
  }
  if (p.groups > 0x7fffffffLL) return kf_set_error(KF_EINVAL, "kf_reduce_dim: shape exceeds the grid limit");
  return dispatch_all<ReduceDimL>(dt, op, f, A, rows, cols, col_stride, dim, dst, dst_stride, scratch,
                                  (hipStream_t)stream, (int64_t)1, (int64_t)0);
}

extern "C" size_t kf_reduce_dim_batched_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int64_t batch) {
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || rows <= 0 || cols <= 0 || batch <= 0) return 256;
  const DimPlan pv = plan_dim(es, rows, cols, 2, true, batch), ps = plan_dim(es, rows, cols, 2, false, batch);
  return kRedReserved + kmax<size_t>(256, kmax<size_t>(pv.partial_bytes, ps.partial_bytes));
}

extern "C" int kf_reduce_dim_batched(kf_op op, kf_map f, kf_dtype dt, const void* A, int64_t rows, int64_t cols,
                                     int64_t col_stride, int64_t batch, int64_t batch_stride, void* dst,
                                     int64_t dst_stride, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (rows < 0 || cols < 0 || batch < 0) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: negative shape");
  if (rows == 0 || batch == 0) return KF_OK;
  if (cols == 0)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: reducing an empty dimension has no identity-free result");
  if (!A || !dst) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: null A or dst");
  if (col_stride < rows) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: col_stride < rows");
  if (batch > 1 && batch_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: batch_stride < 1");
  if (dst_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: dst_stride must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)A % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: A/dst not aligned to the element type");
  const bool vec = dim_vec_ok(A, col_stride, es) && (batch == 1 || (batch_stride * (int64_t)es) % 16 == 0);
  const DimPlan p = plan_dim(es, rows, cols, 2, vec, batch);
  if (p.split > 1) {
    const size_t need = kf_reduce_dim_batched_scratch_bytes(dt, rows, cols, batch);
    if (!scratch || scratch_bytes < need)
      return kf_set_error(KF_ENOSCRATCH, "kf_reduce_dim_batched: scratch of %zu bytes needed, %zu given", need,
                          scratch ? scratch_bytes : (size_t)0);
    if ((uintptr_t)scratch % 256)
      return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: scratch must be 256-byte aligned");
  }
  if (p.groups > 0x7fffffffLL) return kf_set_error(KF_EINVAL, "kf_reduce_dim_batched: shape exceeds the grid limit");
  return dispatch_all<ReduceDimL>(dt, op, f, A, rows, cols, col_stride, 2, dst, dst_stride, scratch,
                                  (hipStream_t)stream, batch, batch_stride);
}

template <class T, class... A> int dispatch_dim_x(kf_op op, kf_map2 f, A... args) {
  if (f == KF_MAP2_SQDIFF) {
    switch (op) {
      case KF_OP_ADD: return launch_reduce_dim<T, OpAdd, Map2SqDiff>(args...);
      case KF_OP_MAX: return launch_reduce_dim<T, OpMax, Map2SqDiff>(args...);
      case KF_OP_MUL: return launch_reduce_dim<T, OpMul, Map2SqDiff>(args...);
      default: return launch_reduce_dim<T, OpMin, Map2SqDiff>(args...);
    }
  }
  switch (op) {
    case KF_OP_ADD: return launch_reduce_dim<T, OpAdd, Map2Mul>(args...);
    case KF_OP_MAX: return launch_reduce_dim<T, OpMax, Map2Mul>(args...);
    case KF_OP_MUL: return launch_reduce_dim<T, OpMul, Map2Mul>(args...);
    default: return launch_reduce_dim<T, OpMin, Map2Mul>(args...);
  }
}

extern "C" int kf_reduce_dim_x(kf_op op, kf_map2 f, kf_dtype dt, const void* A, int64_t rows, int64_t cols,
                               int64_t col_stride, int dim, const void* x, int64_t x_stride, void* dst,
                               int64_t dst_stride, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, KF_MAP_IDENTITY, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if (f != KF_MAP2_MUL && f != KF_MAP2_SQDIFF)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: map %d is not one of x*y, (x-y)^2", (int)f);
  if (dim != 1 && dim != 2) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: dim must be 1 or 2 (got %d)", dim);
  if (rows < 0 || cols < 0) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: negative shape");
  if ((dim == 1 ? cols : rows) == 0) return KF_OK;
  if ((dim == 1 ? rows : cols) == 0)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: reducing an empty dimension has no identity-free result");
  if (!A || !dst || !x) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: null pointer");
  if (col_stride < rows) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: col_stride < rows");
  if (dst_stride < 1 || x_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: strides must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)A % es || (uintptr_t)dst % es || (uintptr_t)x % es)
    return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: pointers not aligned to the element type");
  const DimPlan p = plan_dim(es, rows, cols, dim, dim_vec_ok(A, col_stride, es));
  if (p.split > 1) {
    const size_t need = kf_reduce_dim_scratch_bytes(dt, rows, cols, dim);
    if (!scratch || scratch_bytes < need)
      return kf_set_error(KF_ENOSCRATCH, "kf_reduce_dim_x: scratch of %zu bytes needed, %zu given", need,
                          scratch ? scratch_bytes : (size_t)0);
    if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: scratch must be 256-byte aligned");
  }
  if (p.groups > 0x7fffffffLL) return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: shape exceeds the grid limit");
  hipStream_t s = (hipStream_t)stream;
  const int64_t one = 1, zero = 0;
  switch (dt) {
    case KF_F32: return dispatch_dim_x<float>(op, f, A, rows, cols, col_stride, dim, dst, dst_stride, red_work(scratch), s, one, zero, x, x_stride);
    case KF_F64: return dispatch_dim_x<double>(op, f, A, rows, cols, col_stride, dim, dst, dst_stride, red_work(scratch), s, one, zero, x, x_stride);
    case KF_I32: return dispatch_dim_x<int32_t>(op, f, A, rows, cols, col_stride, dim, dst, dst_stride, red_work(scratch), s, one, zero, x, x_stride);
    case KF_I64: return dispatch_dim_x<int64_t>(op, f, A, rows, cols, col_stride, dim, dst, dst_stride, red_work(scratch), s, one, zero, x, x_stride);
    case KF_U8: return dispatch_dim_x<uint8_t>(op, f, A, rows, cols, col_stride, dim, dst, dst_stride, red_work(scratch), s, one, zero, x, x_stride);
    default: return kf_set_error(KF_EINVAL, "kf_reduce_dim_x: bad dtype %d", (int)dt);
  }
}

template <class T, class G> int launch_post(void* x, int64_t n, int64_t stride, hipStream_t s) {
  const int grid = (int)kmin<int64_t>(8192, kmax<int64_t>(1, (n + 255) / 256));
  hipLaunchKernelGGL((post_map_kernel<T, G>), dim3(grid), dim3(256), 0, s, (T*)x, n, stride);
  return kf_check_launch("post_map_kernel");
}

extern "C" int kf_post_map(kf_post g, kf_dtype dt, void* x, int64_t n, int64_t stride, void* stream) {
  if (g == KF_POST_IDENTITY || n == 0) return KF_OK;
  if (n < 0 || stride < 1) return kf_set_error(KF_EINVAL, "kf_post_map: bad n or stride");
  if (!x) return kf_set_error(KF_EINVAL, "kf_post_map: null pointer");
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || dt == KF_F32X2) return kf_set_error(KF_EINVAL, "kf_post_map: unsupported dtype %d", (int)dt);
  if ((uintptr_t)x % es) return kf_set_error(KF_EINVAL, "kf_post_map: pointer not aligned to the element type");
  hipStream_t s = (hipStream_t)stream;
  if (g == KF_POST_SQRT) {
    if (dt == KF_F32) return launch_post<float, PostSqrt>(x, n, stride, s);
    if (dt == KF_F64) return launch_post<double, PostSqrt>(x, n, stride, s);
    return kf_set_error(KF_EINVAL, "kf_post_map: sqrt needs a floating-point type");
  }
  if (g == KF_POST_ABS2) {
    switch (dt) {
      case KF_F32: return launch_post<float, MapAbs2>(x, n, stride, s);
      case KF_F64: return launch_post<double, MapAbs2>(x, n, stride, s);
      case KF_I32: return launch_post<int32_t, MapAbs2>(x, n, stride, s);
      case KF_I64: return launch_post<int64_t, MapAbs2>(x, n, stride, s);
      default: return launch_post<uint8_t, MapAbs2>(x, n, stride, s);
    }
  }
  return kf_set_error(KF_EINVAL, "kf_post_map: unknown post-map %d", (int)g);
}

extern "C" int kf_scratch_reset(void* scratch, size_t bytes, void* stream) {
  if (bytes == 0) return KF_OK;
  if (!scratch) return kf_set_error(KF_EINVAL, "kf_scratch_reset: null scratch");
  const int grid = (int)kmin<int64_t>(1024, kmax<int64_t>(1, ((int64_t)bytes + 255) / 256));
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (uint8_t*)scratch,
                     (int64_t)bytes);
  return kf_check_launch("fill_zero_kernel");
}
