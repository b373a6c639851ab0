// Full reduction (mapreduce with dims = nothing) for gfx950.
//
// Same two stages as the reference's mapreduce1d_kernel!
// (reference src/mapreduce/1D/mapreduce1d_kernel.jl:5-93): a grid-stride
// pass producing one partial per workgroup, then a single workgroup
// combining the partials. MI355X design:
//  * 16-byte streaming loads, 4 in flight per lane, each vector element
//    folded into its own accumulator (16 independent float sums per lane),
//    which keeps Float32 sums accurate and the loop free of dependencies.
//  * The grid is sized to 8 workgroups per CU (2048 on 256 CUs, capped at
//    kRedMaxBlocks). An unaligned head and the ragged tail are folded in by
//    workgroup 0, so any 4-byte-aligned view takes the vector path.
//  * Stage 2 is "last workgroup done": every workgroup publishes its partial
//    and takes a ticket with an acq_rel device-scope atomic; the workgroup
//    that draws the last ticket combines all partials in index order and
//    clears the counter for the next call. Nothing spins (the reference's
//    block 1 spins on per-block flags, mapreduce1d_kernel.jl:66-92), and
//    the combine order depends only on n and alignment, so results are
//    bit-for-bit reproducible.
#include "kf_common.h"

namespace kf {

constexpr int kRedBlock = 256;
constexpr int kRedWaves = kRedBlock / kWave;
constexpr int kRedUnroll = 4;
constexpr int kRedMaxBlocks = 4096;
constexpr size_t kRedHeaderBytes = 256;

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

// Stage 2 shared by the full and the per-column/row reductions: publish a
// partial, draw a ticket, and let the last of `count` workgroups return true.
__device__ inline bool last_block_done(uint32_t* counter, uint32_t count, bool* s_flag) {
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == count - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  const bool last = *s_flag;
  if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return last;
}

template <class T, class Op, class Map>
__global__ __launch_bounds__(kRedBlock) void reduce_kernel(const T* src, int64_t n, int64_t stride,
                                                           T* dst, uint8_t* scratch, int vec) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  __shared__ bool s_last;
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
  if (gridDim.x == 1) {
    if (tid == 0) dst[0] = part;
    return;
  }
  uint32_t* counter = reinterpret_cast<uint32_t*>(scratch);
  T* partials = reinterpret_cast<T*>(scratch + kRedHeaderBytes);
  if (tid == 0) partials[blockIdx.x] = part;
  if (!last_block_done(counter, gridDim.x, &s_last)) return;
  __syncthreads();  // s_wave is reused below
  T x = id;
  for (uint32_t j = tid; j < gridDim.x; j += kRedBlock) x = Op::combine(x, partials[j]);
  const T total = block_reduce<T, Op>(x, s_wave);
  if (tid == 0) dst[0] = total;
}

template <class T> int reduce_grid(int64_t n) {
  constexpr int64_t per_block = (int64_t)kRedBlock * kRedUnroll * (16 / sizeof(T)) * 4;
  int64_t g = (n + per_block - 1) / per_block;
  const int64_t cap = kmin<int64_t>(kRedMaxBlocks, (int64_t)kf_device_cu_count() * 8);
  if (g > cap) g = cap;
  return (int)kmax<int64_t>(g, 1);
}

template <class T, class Op, class Map>
int launch_reduce(const void* src, int64_t n, int64_t stride, void* dst, void* scratch,
                  hipStream_t stream) {
  const int grid = reduce_grid<T>(n);
  const int vec = stride == 1;
  hipLaunchKernelGGL((reduce_kernel<T, Op, Map>), dim3(grid), dim3(kRedBlock), 0, stream,
                     (const T*)src, n, stride, (T*)dst, (uint8_t*)scratch, vec);
  return kf_check_launch("reduce_kernel");
}

// ---------------------------------------------------------------------------
// dim = 1: one wave per column (a column of a column-major matrix is
// contiguous), optionally split into S row segments when there are too few
// columns to fill the GPU. Follows vecmat_kernel! (reference
// src/mapreduce/2D/vecmat_kernel.jl:1-169) in what it computes; the wave-per-
// column layout with 16-byte loads replaces its tuned Nthreads/Nitem table.
// ---------------------------------------------------------------------------
constexpr int kDimBlock = 256;
constexpr int kDimWaves = kDimBlock / kWave;
constexpr int kDimUnroll = 4;
constexpr int kDimMaxSplit = 64;

struct DimPlan {
  int64_t groups;  // column groups (dim 1) or row strips (dim 2)
  int split;       // S workgroups cooperating on one group
  size_t counter_bytes, partial_bytes;
};

template <class T, class Op, class Map>
__global__ __launch_bounds__(kDimBlock) void reduce_cols_kernel(
    const T* A, int64_t rows, int64_t cols, int64_t col_stride, T* dst, int64_t dst_stride,
    uint8_t* scratch, size_t counter_bytes, int64_t seg_rows, int vec) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ bool s_last;
  const T id = Op::template identity<T>();
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int64_t col = (int64_t)blockIdx.x * kDimWaves + wave;
  const int S = gridDim.y;
  const int s = blockIdx.y;
  T acc = id;
  if (col < cols) {
    const T* c = A + col * col_stride;
    const int64_t r0 = (int64_t)s * seg_rows;
    const int64_t r1 = kmin<int64_t>(rows, r0 + seg_rows);
    if (vec) {
      // seg_rows is a multiple of EPV and columns are 16-byte aligned.
      const int64_t nv = (r1 - r0) / EPV;
      const uint4* v = reinterpret_cast<const uint4*>(c + r0);
      T a[kDimUnroll][EPV];
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u)
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = id;
      int64_t i = lane;
      for (; i + (kDimUnroll - 1) * kWave < nv; i += kDimUnroll * kWave) {
        uint4 r[kDimUnroll];
#pragma unroll
        for (int u = 0; u < kDimUnroll; ++u) r[u] = ld_stream(v + i + u * kWave);
#pragma unroll
        for (int u = 0; u < kDimUnroll; ++u) {
          T x[EPV];
          __builtin_memcpy(x, &r[u], 16);
#pragma unroll
          for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], Map::apply(x[e]));
        }
      }
      for (; i < nv; i += kWave) {
        const uint4 r = ld_stream(v + i);
        T x[EPV];
        __builtin_memcpy(x, &r, 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[0][e] = Op::combine(a[0][e], Map::apply(x[e]));
      }
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc = Op::combine(acc, a[u][e]);
      const int64_t t = r0 + nv * EPV + lane;
      if (t < r1) acc = Op::combine(acc, Map::apply(c[t]));
    } else {
      for (int64_t r = r0 + lane; r < r1; r += kWave) acc = Op::combine(acc, Map::apply(c[r]));
    }
  }
  acc = wave_reduce<Op>(acc);
  if (S == 1) {
    if (col < cols && lane == 0) dst[col * dst_stride] = acc;
    return;
  }
  uint32_t* counters = reinterpret_cast<uint32_t*>(scratch);
  T* partials = reinterpret_cast<T*>(scratch + counter_bytes);
  if (col < cols && lane == 0) {
    partials[(int64_t)s * cols + col] = acc;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  }
  __syncthreads();
  if (!last_block_done(counters + blockIdx.x, (uint32_t)S, &s_last)) return;
  if (col < cols) {
    T x = lane < S ? partials[(int64_t)lane * cols + col] : id;
    x = wave_reduce<Op>(x);
    if (lane == 0) dst[col * dst_stride] = x;
  }
}

// ---------------------------------------------------------------------------
// dim = 2: a workgroup owns a strip of 64*EPV rows (each lane EPV adjacent
// rows, one 16-byte load per column) and a range of columns; its 4 waves
// take interleaved columns and are combined through LDS in wave order.
// Strips with too few workgroups are split over S column ranges whose
// partials the last-done workgroup combines. Computes what matvec_kernel!
// computes (reference src/mapreduce/2D/matvec_kernel.jl:1-239).
// ---------------------------------------------------------------------------
template <class T, class Op, class Map, bool VEC>
__global__ __launch_bounds__(kDimBlock) void reduce_rows_kernel(
    const T* A, int64_t rows, int64_t cols, int64_t col_stride, T* dst, int64_t dst_stride,
    uint8_t* scratch, size_t counter_bytes, int64_t seg_cols) {
  constexpr int EPV = VEC ? 16 / (int)sizeof(T) : 1;
  constexpr int RS = kWave * EPV;
  __shared__ T s_part[kDimWaves][RS];
  __shared__ bool s_last;
  const T id = Op::template identity<T>();
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int S = gridDim.y;
  const int s = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * RS + (int64_t)lane * EPV;
  const int64_t c0 = (int64_t)s * seg_cols;
  const int64_t c1 = kmin<int64_t>(cols, c0 + seg_cols);

  T a[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) a[e] = id;
  if (VEC && row0 + EPV <= rows) {
    const T* p = A + row0;
    int64_t c = c0 + wave;
    for (; c + (kDimUnroll - 1) * kDimWaves < c1; c += kDimUnroll * kDimWaves) {
      uint4 r[kDimUnroll];
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u)
        r[u] = ld_stream(reinterpret_cast<const uint4*>(p + (c + u * kDimWaves) * col_stride));
#pragma unroll
      for (int u = 0; u < kDimUnroll; ++u) {
        T x[EPV];
        __builtin_memcpy(x, &r[u], sizeof(x));
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], Map::apply(x[e]));
      }
    }
    for (; c < c1; c += kDimWaves) {
      const uint4 r = ld_stream(reinterpret_cast<const uint4*>(p + c * col_stride));
      T x[EPV];
      __builtin_memcpy(x, &r, sizeof(x));
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], Map::apply(x[e]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const int64_t r = row0 + e;
      if (r < rows) {
        T x = id;
        for (int64_t c = c0 + wave; c < c1; c += kDimWaves) x = Op::combine(x, Map::apply(A[r + c * col_stride]));
        a[e] = x;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) s_part[wave][lane * EPV + e] = a[e];
  __syncthreads();
  // Each thread now owns one row of the strip (RS <= kDimBlock for EPV <= 4;
  // wider types loop).
  uint32_t* counters = reinterpret_cast<uint32_t*>(scratch);
  T* partials = reinterpret_cast<T*>(scratch + counter_bytes);
  for (int lr = threadIdx.x; lr < RS; lr += kDimBlock) {
    T x = s_part[0][lr];
#pragma unroll
    for (int w = 1; w < kDimWaves; ++w) x = Op::combine(x, s_part[w][lr]);
    const int64_t r = (int64_t)blockIdx.x * RS + lr;
    if (r < rows) {
      if (S == 1) dst[r * dst_stride] = x;
      else partials[(int64_t)s * rows + r] = x;
    }
  }
  if (S == 1) return;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (!last_block_done(counters + blockIdx.x, (uint32_t)S, &s_last)) return;
  for (int lr = threadIdx.x; lr < RS; lr += kDimBlock) {
    const int64_t r = (int64_t)blockIdx.x * RS + lr;
    if (r < rows) {
      T x = partials[r];
      for (int j = 1; j < S; ++j) x = Op::combine(x, partials[(int64_t)j * rows + r]);
      dst[r * dst_stride] = x;
    }
  }
}

inline size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Launch plan. Targets ~16K waves for dim 1 and ~2K workgroups for dim 2;
// must be a pure function of (dtype size, rows, cols, dim) so the scratch
// size query and the launch agree.
inline DimPlan plan_dim(size_t es, int64_t rows, int64_t cols, int dim) {
  DimPlan p{};
  const int epv = (int)(16 / es);
  if (dim == 1) {
    p.groups = (cols + kDimWaves - 1) / kDimWaves;
    int64_t S = 1;
    if (cols < 16384) {
      S = (16384 + cols - 1) / cols;
      const int64_t by_rows = rows / ((int64_t)kWave * epv * kDimUnroll * 4);  // >= 4 unrolled passes each
      S = kmin<int64_t>(S, kmax<int64_t>(by_rows, 1));
      S = kmin<int64_t>(S, kDimMaxSplit);
    }
    p.split = (int)S;
  } else {
    const int64_t rs = (int64_t)kWave * epv;
    p.groups = (rows + rs - 1) / rs;
    int64_t S = 1;
    if (p.groups < 2048) {
      S = (2048 + p.groups - 1) / p.groups;
      const int64_t by_cols = cols / ((int64_t)kDimWaves * 16);  // >= 16 columns per wave
      S = kmin<int64_t>(S, kmax<int64_t>(by_cols, 1));
      S = kmin<int64_t>(S, kDimMaxSplit);
    }
    p.split = (int)S;
  }
  if (p.split > 1) {
    // dim 2 counts counters per 64-row strip: enough for the vector variant
    // (64*EPV rows) and for the unaligned scalar variant (64 rows).
    const int64_t ncounters = dim == 1 ? p.groups : (rows + kWave - 1) / kWave;
    p.counter_bytes = round256((size_t)ncounters * sizeof(uint32_t));
    p.partial_bytes = round256((size_t)p.split * (size_t)(dim == 1 ? cols : rows) * es);
  }
  return p;
}

template <class T, class Op, class Map>
int launch_reduce_dim(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst,
                      int64_t ds, void* scratch, hipStream_t stream) {
  const DimPlan p = plan_dim(sizeof(T), rows, cols, dim);
  const bool aligned = ((uintptr_t)A % 16 == 0) && ((cs * (int64_t)sizeof(T)) % 16 == 0);
  if (dim == 1) {
    constexpr int EPV = 16 / (int)sizeof(T);
    int64_t seg = (rows + p.split - 1) / p.split;
    seg = (seg + EPV - 1) / EPV * EPV;
    hipLaunchKernelGGL((reduce_cols_kernel<T, Op, Map>), dim3((unsigned)p.groups, p.split), dim3(kDimBlock), 0,
                       stream, (const T*)A, rows, cols, cs, (T*)dst, ds, (uint8_t*)scratch, p.counter_bytes,
                       seg, (int)aligned);
    return kf_check_launch("reduce_cols_kernel");
  }
  const int64_t seg = (cols + p.split - 1) / p.split;
  if (aligned) {
    hipLaunchKernelGGL((reduce_rows_kernel<T, Op, Map, true>), dim3((unsigned)p.groups, p.split), dim3(kDimBlock),
                       0, stream, (const T*)A, rows, cols, cs, (T*)dst, ds, (uint8_t*)scratch, p.counter_bytes, seg);
  } else {
    // The scalar variant has 64-row strips: re-plan its grid for that width.
    const int64_t groups = (rows + kWave - 1) / kWave;
    hipLaunchKernelGGL((reduce_rows_kernel<T, Op, Map, false>), dim3((unsigned)groups, p.split), dim3(kDimBlock),
                       0, stream, (const T*)A, rows, cols, cs, (T*)dst, ds, (uint8_t*)scratch, p.counter_bytes, seg);
  }
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
      default: return L<T, OpMin, MapAbs2>::run(args...);
    }
  }
  switch (op) {
    case KF_OP_ADD: return L<T, OpAdd, MapIdentity>::run(args...);
    case KF_OP_MAX: return L<T, OpMax, MapIdentity>::run(args...);
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
template <class T, class Op, class Map> struct ReduceDimL {
  static int run(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst, int64_t ds,
                 void* scratch, hipStream_t s) {
    return launch_reduce_dim<T, Op, Map>(A, rows, cols, cs, dim, dst, ds, scratch, s);
  }
};

// ---------------------------------------------------------------------------
// Copy ceiling and scratch fill.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void copy_kernel(uint4* dst, const uint4* src, int64_t nvec) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * gsize < nvec; i += 4 * gsize) {
    uint4 r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) r[u] = ld_stream(src + i + u * gsize);
#pragma unroll
    for (int u = 0; u < 4; ++u) st_stream(dst + i + u * gsize, r[u]);
  }
  for (; i < nvec; i += gsize) st_stream(dst + i, ld_stream(src + i));
}

__global__ void copy_bytes_kernel(uint8_t* dst, const uint8_t* src, int64_t n) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gsize) dst[i] = src[i];
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
  return kRedHeaderBytes + (size_t)kRedMaxBlocks * es;
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

extern "C" size_t kf_reduce_dim_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int dim) {
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || rows <= 0 || cols <= 0 || (dim != 1 && dim != 2)) return 256;
  const DimPlan p = plan_dim(es, rows, cols, dim);
  return kmax<size_t>(256, p.counter_bytes + p.partial_bytes);
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
  const DimPlan p = plan_dim(es, rows, cols, dim);
  if (p.split > 1) {
    if (!scratch || scratch_bytes < need)
      return kf_set_error(KF_ENOSCRATCH, "kf_reduce_dim: scratch of %zu bytes needed, %zu given", need,
                          scratch ? scratch_bytes : (size_t)0);
    if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce_dim: scratch must be 256-byte aligned");
  }
  if (p.groups > 0x7fffffffLL) return kf_set_error(KF_EINVAL, "kf_reduce_dim: shape exceeds the grid limit");
  return dispatch_all<ReduceDimL>(dt, op, f, A, rows, cols, col_stride, dim, dst, dst_stride, scratch,
                                  (hipStream_t)stream);
}

extern "C" int kf_copy(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return KF_OK;
  if (!dst || !src) return kf_set_error(KF_EINVAL, "kf_copy: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int cap = kf_device_cu_count() * 8;
  if ((uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0) {
    const int64_t nvec = (int64_t)(bytes / 16);
    if (nvec > 0) {
      const int grid = (int)kmin<int64_t>(cap, kmax<int64_t>(1, (nvec + 1023) / 1024));
      hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(256), 0, s, (uint4*)dst, (const uint4*)src, nvec);
    }
    const int64_t rem = (int64_t)(bytes % 16);
    if (rem)
      hipLaunchKernelGGL(copy_bytes_kernel, dim3(1), dim3(64), 0, s, (uint8_t*)dst + nvec * 16,
                         (const uint8_t*)src + nvec * 16, rem);
  } else {
    const int grid = (int)kmin<int64_t>(cap, kmax<int64_t>(1, ((int64_t)bytes + 255) / 256));
    hipLaunchKernelGGL(copy_bytes_kernel, dim3(grid), dim3(256), 0, s, (uint8_t*)dst, (const uint8_t*)src,
                       (int64_t)bytes);
  }
  return kf_check_launch("copy_kernel");
}

extern "C" int kf_scratch_reset(void* scratch, size_t bytes, void* stream) {
  if (bytes == 0) return KF_OK;
  if (!scratch) return kf_set_error(KF_EINVAL, "kf_scratch_reset: null scratch");
  const int grid = (int)kmin<int64_t>(1024, kmax<int64_t>(1, ((int64_t)bytes + 255) / 256));
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (uint8_t*)scratch,
                     (int64_t)bytes);
  return kf_check_launch("fill_zero_kernel");
}
