// Reduction-along-dims kernels and their launch plan, shared by
// kf_reduce_dims.hip (mapreduce with dims) and kf_matvec.hip (matvec /
// vecmat with a vector operand) so the two instantiation sets compile in
// parallel. Reference src/mapreduce/2D/vecmat_kernel.jl:1-169 (dims=1),
// src/mapreduce/2D/matvec_kernel.jl:1-239 (dims=2): partial results per
// workgroup, then a combine when columns or rows are split.
#pragma once
#include <atomic>
#include "kf_reduce.h"

namespace kf {


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

// Stage 2 for many splits of few rows: the S partial columns are cut into
// kCombWaves consecutive ranges, one per wave; lane l of every wave owns row
// blockIdx.x * 64 + l, so each load of a wave reads 64 consecutive partials,
// with kCombUnroll loads in flight; the ranges are then combined in order.
// (One workgroup of the narrow kernel folding 512 partial columns of 1000
// rows took longer than the streaming pass it finished.)
constexpr int kCombWaves = 16;
constexpr int kCombUnroll = 8;
template <class T, class Op>
__global__ __launch_bounds__(kCombWaves * kWave) void combine_cols_kernel(const T* partials, int S, int64_t m,
                                                                          T* dst, int64_t ds, int64_t dst_bstride) {
  __shared__ T s_part[kCombWaves][kWave];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t i = (int64_t)blockIdx.x * kWave + lane;
  partials += (int64_t)blockIdx.y * S * m;
  const int per = (S + kCombWaves - 1) / kCombWaves;
  const int s0 = wave * per, s1 = kmin(S, s0 + per);
  T acc = Op::template identity<T>();
  if (i < m) {
    int s = s0;
    for (; s + kCombUnroll <= s1; s += kCombUnroll) {
      T x[kCombUnroll];
#pragma unroll
      for (int u = 0; u < kCombUnroll; ++u) x[u] = partials[(int64_t)(s + u) * m + i];
#pragma unroll
      for (int u = 0; u < kCombUnroll; ++u) acc = Op::combine(acc, x[u]);
    }
    for (; s < s1; ++s) acc = Op::combine(acc, partials[(int64_t)s * m + i]);
  }
  s_part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && i < m) {
    T x = s_part[0][lane];
#pragma unroll
    for (int w = 1; w < kCombWaves; ++w) x = Op::combine(x, s_part[w][lane]);
    dst[(int64_t)blockIdx.y * dst_bstride + i * ds] = x;
  }
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

// UInt8 sums through v_dot4_u32_u8: for op + with f = identity, abs2 or x*y
// (the reference's UInt8 benchmarks), four bytes fold into a 32-bit
// accumulator per instruction; the low byte of the 32-bit sum is the UInt8
// (mod 256) result, exactly as a byte-by-byte wrapping sum.
template <class T, class Op, class F> struct Dot4 {
  static constexpr int kind = -1;  // not applicable
};
template <> struct Dot4<uint8_t, OpAdd, Unary<MapIdentity>> {
  static constexpr int kind = 0;  // sum of bytes: dot with 0x01010101
};
template <> struct Dot4<uint8_t, OpAdd, Unary<MapAbs2>> {
  static constexpr int kind = 1;  // sum of squares: dot with itself
};
template <> struct Dot4<uint8_t, OpAdd, Map2Mul> {
  static constexpr int kind = 2;  // dot product with the operand
};

// The same UInt8 sums by rows (dims=2, every byte of a vector its own row):
// the even and odd bytes of each 32-bit word accumulate apart in packed
// 16-bit lanes (v_pk_mad_u16: two rows per instruction); the low byte of
// each 16-bit lane is the UInt8 (mod 256) result.
typedef unsigned short kf_us2 __attribute__((ext_vector_type(2)));
template <int K> __device__ inline void pk16_word(uint32_t& ae, uint32_t& ao, uint32_t a, uint32_t w16) {
  const kf_us2 e = __builtin_bit_cast(kf_us2, a & 0x00ff00ffu);
  const kf_us2 o = __builtin_bit_cast(kf_us2, (a >> 8) & 0x00ff00ffu);
  kf_us2 E = __builtin_bit_cast(kf_us2, ae), O = __builtin_bit_cast(kf_us2, ao);
  if constexpr (K == 0) {
    E += e;
    O += o;
  } else if constexpr (K == 1) {
    E += e * e;
    O += o * o;
  } else {
    const kf_us2 w = __builtin_bit_cast(kf_us2, w16);
    E += e * w;
    O += o * w;
  }
  ae = __builtin_bit_cast(uint32_t, E);
  ao = __builtin_bit_cast(uint32_t, O);
}
template <int K> __device__ inline void pk16_vec(uint32_t (&ae)[4], uint32_t (&ao)[4], uint4 a, uint32_t w16) {
  pk16_word<K>(ae[0], ao[0], a.x, w16);
  pk16_word<K>(ae[1], ao[1], a.y, w16);
  pk16_word<K>(ae[2], ao[2], a.z, w16);
  pk16_word<K>(ae[3], ao[3], a.w, w16);
}
// the four result bytes of one word: rows 0 and 2 from the even lanes, 1 and 3 from the odd
__device__ inline uint32_t pk16_bytes(uint32_t ae, uint32_t ao) { return (ae & 0x00ff00ffu) | ((ao & 0x00ff00ffu) << 8); }

constexpr int kDimBlock = 256;
constexpr int kDimWaves = kDimBlock / kWave;
constexpr int kDimUnroll = 4;
constexpr int kScalarUnroll = 8;  // element (unaligned) paths: loads in flight per thread
constexpr int kDimMaxSplit = 64;          // dim 1 splits combined by combine_split_kernel
constexpr int kDimMaxSplitNarrow = 4096;  // dim 1 splits combined by reduce_rows_narrow_kernel
constexpr int kRowVecsDefault = 2;    // dim 2, unaligned path: elements per thread per column / 1
constexpr int kColUnrollDefault = 8;  // dim 2, unaligned path: columns per pass
constexpr int kDim2Blocks = 256;      // dim 2: strip widths keep one workgroup per CU
constexpr int kDim2SplitBlocks = 1024;  // dim 2, fewer than kDim2FewStrips strips: split target
constexpr int kDim2FewStrips = 64;
// dim 2, aligned path: the widest strip (16-byte vectors per thread per
// column) that still gives kDim2Blocks workgroups; columns in flight per
// thread for each strip width.
constexpr int kDim2MaxRowVecs = 8;
constexpr int kDim2MaxRowVecsU8 = 2;
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
    if constexpr (Dot4<T, Op, F>::kind >= 0) {
      constexpr int K = Dot4<T, Op, F>::kind;
      uint32_t d[kDimUnroll] = {};
      int64_t i = lane;
      for (; i + (kDimUnroll - 1) * kWave < nv; i += kDimUnroll * kWave) {
        uint4 r[kDimUnroll], rx[kDimUnroll];
#pragma unroll
        for (int u = 0; u < kDimUnroll; ++u) {
          r[u] = ld_stream(v + i + u * kWave);
          if constexpr (F::kHasX) rx[u] = vx[i + u * kWave];
        }
#pragma unroll
        for (int u = 0; u < kDimUnroll; ++u) d[u] = dot4_vec<K>(d[u], r[u], F::kHasX ? rx[u] : r[u]);
      }
      for (; i < nv; i += kWave) {
        const uint4 r = ld_stream(v + i);
        d[0] = dot4_vec<K>(d[0], r, F::kHasX ? vx[i] : r);
      }
      static_assert(kDimUnroll == 4, "the four dot4 accumulators");
      acc = Op::combine(acc, (T)(d[0] + d[1] + d[2] + d[3]));
    } else {
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
    }
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

// vecmat over few long columns (2..kMultiMaxCols of them, 16-byte aligned):
// workgroup s takes rows [s*seg, s*seg + seg) of every column at once, so
// each 16-byte vector of the operand x is loaded once for all columns. A
// wave per column loads it once per column group, from a different XCD's
// L2 for each group: vecmat of a 10^8 x 10 matrix took 930 us (Float32),
// 1864 us (Float64) and 235 us (UInt8) that way, against 610, 1217 and 164
// us for the same columns without x; here 717, 1314 and 185 us. Without x
// the wave per column stays ahead (Float32 610 against 805 us here). One
// accumulator per column and lane; waves combine through LDS into
// partials[s*cols + c] (or dst when one workgroup covers the rows).
constexpr int kMultiMaxCols = 16;
constexpr int kMultiBlocks = 2048;
// below this the wave per column stays ahead (10^6 x 10 vecmat Float32 11.9
// against 12.9 us, Float64 21.4 / 23.2, UInt8 7.0 / 8.5; 10^7 x 10 UInt8
// 26.7 against 24.6)
constexpr int64_t kMultiMinBytes = 80LL << 20;
template <class T, class Op, class F>
__global__ __launch_bounds__(kDimBlock) void reduce_cols_multi_kernel(
    const T* A, int64_t rows, int cols, int64_t col_stride, T* out, int64_t out_stride, int64_t seg, const T* xv) {
  constexpr int EPV = 16 / (int)sizeof(T);
  constexpr int C = kMultiMaxCols;
  constexpr int K = Dot4<T, Op, F>::kind;
  using Acc = std::conditional_t<(K >= 0), uint32_t, T>;
  __shared__ T s_part[kDimWaves][C];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int64_t r0 = (int64_t)blockIdx.x * seg;
  const int64_t r1 = kmin<int64_t>(rows, r0 + seg);
  const int64_t nv = r1 > r0 ? (r1 - r0) / EPV : 0;  // seg is a multiple of EPV
  Acc acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = K >= 0 ? Acc(0) : Acc(id);
  for (int64_t i = tid; i < nv; i += kDimBlock) {
    uint4 rx;
    if constexpr (F::kHasX) rx = reinterpret_cast<const uint4*>(xv + r0)[i];
    uint4 r[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (c < cols) r[c] = ld_stream(reinterpret_cast<const uint4*>(A + c * col_stride + r0) + i);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c >= cols) continue;
      if constexpr (K >= 0) {
        acc[c] = dot4_vec<K>(acc[c], r[c], F::kHasX ? rx : r[c]);
      } else {
        T a[EPV], w[EPV];
        __builtin_memcpy(a, &r[c], 16);
        if constexpr (F::kHasX) __builtin_memcpy(w, &rx, 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[c] = Op::combine(acc[c], F::apply(a[e], F::kHasX ? w[e] : a[e]));
      }
    }
  }
  // the rows after the last whole vector (fewer than EPV, last workgroup)
  const int64_t t = r0 + nv * EPV + tid;
  T res[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    T v = (T)acc[c];
    if (c < cols && t < r1) {
      const T a = A[c * col_stride + t];
      v = Op::combine(v, F::apply(a, F::kHasX ? xv[t] : a));
    }
    res[c] = wave_reduce<Op>(v);
  }
  if (lane == 0) {
#pragma unroll
    for (int c = 0; c < C; ++c) s_part[wave][c] = res[c];
  }
  __syncthreads();
  if (tid < cols) {
    T v = s_part[0][tid];
#pragma unroll
    for (int w = 1; w < kDimWaves; ++w) v = Op::combine(v, s_part[w][tid]);
    out[gridDim.x == 1 ? tid * out_stride : (int64_t)blockIdx.x * cols + tid] = v;
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
// dim = 1, short columns of a contiguous matrix (column stride = rows, 16-byte
// aligned): workgroups stage blocks of whole columns, at most kFlatBlockBytes
// each, through LDS with 16-byte loads (every load of a block in flight),
// then reduce each column from LDS with L lanes per column (lane j combines
// rows j, j + L, ...; then a shuffle tree). Blocks hold a multiple of 16
// bytes except the matrix's last, whose ragged end is loaded per element.
// Persistent workgroups walk the blocks. With a vector operand x (vecmat),
// x sits in LDS for the whole launch. Replaces L lanes per column reading
// global memory (reduce_cols_seg_kernel), whose short per-lane loops left
// few loads in flight and, for rows not a multiple of the vector width, ran
// on element loads.
// ---------------------------------------------------------------------------
// Workgroups of KERNEL the whole GPU holds at once (occupancy x CUs), for
// persistent grids; queried once per kernel.
template <auto KERNEL> int64_t resident_blocks(int block) {
  static std::atomic<int> per_cu{0};
  int b = per_cu.load(std::memory_order_relaxed);
  if (b == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, KERNEL, block, 0) != hipSuccess || b <= 0) b = 1;
    per_cu.store(b, std::memory_order_relaxed);
  }
  return (int64_t)b * kf_device_cu_count();
}

constexpr int kFlatVecs = 4;                                   // 16-byte vectors per thread per block
constexpr int kFlatBlockBytes = kDimBlock * kFlatVecs * 16;   // 16 KiB
constexpr int kFlatMaxColBytes = 2048;                         // longest column this path takes
// dims=1 takes columns of up to 4 KiB of 4- and 8-byte types (a wave per
// 4000-byte Float32 column left 10^3 x 10^6 vecmat at 767 us)
constexpr int kFlatMaxColBytesWide = 4096;
// one block of columns per workgroup (grid-stride beyond this cap): the
// dispatcher then balances the blocks, where a persistent grid of 4096
// workgroups left its last ones running alone (10 x 10^8 dims=1 Float32 934
// -> 843 us, Float64 1924 -> 1812 us, 100 x 10^7 Float32 720 -> 664 us; 8K
// to 64K workgroups in between)
constexpr int kFlatMaxBlocks = 1 << 24;
// UInt8 blocks are grid-strided over 16K workgroups, 4K from 256 rows:
// 1000 x 10^6 vecmat 241 us at one block each, 188 at 16K, 181 at 4K;
// 1000 x 10^5 25.3 / 22.7 at 16K / 4K; 100 x 10^7 183 / 164 / 175
constexpr int kFlatMaxBlocksU8 = 16384, kFlatMaxBlocksU8Long = 4096;
constexpr int kFlatRowsPerLane = 16;
constexpr int kFlatWordsPerLane = 8;  // UInt8 dot4 columns
template <class T, class Op, class F, int L>
__global__ __launch_bounds__(kDimBlock) void reduce_cols_flat_kernel(const T* A, int64_t rows, int64_t cols,
                                                                     int64_t cpb, T* out, int64_t out_stride,
                                                                     const T* xv, int64_t xs) {
  __shared__ uint4 s_blk[kDimBlock * kFlatVecs];
  // UInt8 dot4 columns off the word boundary (rows % 4 != 0) also keep x
  // pre-shifted for each byte offset sh of a column: word k of copy sh holds
  // x[4k - sh .. 4k - sh + 3] (zero outside x)
  constexpr bool kShiftX = F::kHasX && Dot4<T, Op, F>::kind >= 0;
  constexpr int kXWords = kFlatMaxColBytes / 4 + 1;
  __shared__ __align__(16) T s_x[F::kHasX ? (sizeof(T) >= 4 ? kFlatMaxColBytesWide : kFlatMaxColBytes) / sizeof(T) : 4];
  __shared__ uint32_t s_xsh[kShiftX ? 4 : 1][kShiftX ? kXWords : 1];
  const T* sb = reinterpret_cast<const T*>(s_blk);
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  if constexpr (F::kHasX)
    for (int64_t i = tid; i < rows; i += kDimBlock) s_x[i] = xv[i * xs];
  if constexpr (kShiftX) {
    if (rows % 4 != 0) {
      const int nw = (int)(rows + 3) / 4 + 1;
      for (int k = tid; k < 4 * nw; k += kDimBlock) {
        const int sh = k / nw, kw = k % nw;
        uint32_t v = 0;
        for (int b = 0; b < 4; ++b) {
          const int64_t r = 4 * (int64_t)kw - sh + b;
          if (r >= 0 && r < rows) v |= (uint32_t)(uint8_t)xv[r * xs] << (8 * b);
        }
        s_xsh[sh][kw] = v;
      }
    }
  }
  constexpr int G = kDimBlock / L;
  const int g = tid / L, j = tid % L;
  const int64_t nblk = (cols + cpb - 1) / cpb;
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t c0 = b * cpb;
    const int64_t nc = kmin<int64_t>(cpb, cols - c0);
    const int64_t nel = nc * rows;
    const int64_t nvec = nel * (int64_t)sizeof(T) / 16;  // whole vectors of the block
    const uint4* src = reinterpret_cast<const uint4*>(A + c0 * rows);
    uint4 r[kFlatVecs];
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) r[u] = ld_stream(src + u * kDimBlock + tid);
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) s_blk[u * kDimBlock + tid] = r[u];
    // the ragged end of the matrix's last block, per element
    const int64_t e0 = nvec * 16 / (int64_t)sizeof(T);
    if (e0 + tid < nel) const_cast<T*>(sb)[e0 + tid] = A[c0 * rows + e0 + tid];
    __syncthreads();
    for (int64_t c = g; c < nc; c += G) {
      const T* col = sb + c * rows;
      T acc = id;
      if constexpr (Dot4<T, Op, F>::kind >= 0) {
        constexpr int K = Dot4<T, Op, F>::kind;
        const uint32_t* xw = reinterpret_cast<const uint32_t*>(s_x);
        uint32_t d = 0;
        if (rows % 4 == 0) {  // dword-aligned columns: four rows per dot4
          const uint32_t* cw = reinterpret_cast<const uint32_t*>(col);
          for (int64_t q = j; q < rows / 4; q += L) d = dot4_word<K>(d, cw[q], F::kHasX ? xw[q] : cw[q]);
        } else {
          // the aligned words over the column's bytes [b0, b0 + rows), bytes
          // outside it masked off; x realigned to the column's byte offset
          const int64_t b0 = c * rows;
          const int sh = (int)(b0 & 3);
          const uint32_t* bw = reinterpret_cast<const uint32_t*>(s_blk);
          const int64_t w0 = b0 >> 2, w1 = (b0 + rows - 1) >> 2;
          for (int64_t w = w0 + j; w <= w1; w += L) {
            const int64_t lo = kmax<int64_t>(b0, 4 * w) - 4 * w, hi = kmin<int64_t>(b0 + rows, 4 * w + 4) - 4 * w;
            const uint32_t m = (0xffffffffu << (8 * lo)) & (0xffffffffu >> (8 * (4 - hi)));
            const uint32_t a = bw[w] & m;
            // rows 4w - b0 .. 4w - b0 + 3 of x: word w - w0 of the copy for sh
            uint32_t xa = 0;
            if constexpr (kShiftX) xa = s_xsh[sh][w - w0];
            d = dot4_word<K>(d, a, F::kHasX ? xa : a);
          }
        }
        acc = (T)d;
      } else if constexpr (L == 1) {
        // each lane starts at its own row (c mod rows) and wraps around, so a
        // wave's reads spread over the LDS banks instead of hitting them at
        // the column stride (16 x 10^7 Float32 / Int32 dims=1 147 -> 107 us;
        // other row counts unchanged)
        int64_t i = c % rows;
        for (int64_t t = 0; t < rows; ++t) {
          acc = Op::combine(acc, F::apply(col[i], F::kHasX ? s_x[i] : col[i]));
          if (++i == rows) i = 0;
        }
      } else {
        // lane j of the column's group takes rows j, j + L, ...; when the
        // column stride is a multiple of 64 bytes (every column starting in
        // the same few LDS banks) it starts at a column-dependent one of
        // them and wraps around (32 x 3*10^7 Float32 at 2 lanes: 917 -> 626
        // us; at other strides the rotation only scattered the x reads: 100
        // x 10^7 Float32 vecmat 643 -> 732)
        if ((rows * (int64_t)sizeof(T)) % 64 == 0) {
          const int cnt = (int)((rows - j + L - 1) / L);
          int64_t i = cnt > 0 ? j + (int64_t)L * ((int)c % cnt) : j;
          for (int t = 0; t < cnt; ++t) {
            acc = Op::combine(acc, F::apply(col[i], F::kHasX ? s_x[i] : col[i]));
            i += L;
            if (i >= rows) i = j;
          }
        } else {
          for (int64_t i = j; i < rows; i += L) acc = Op::combine(acc, F::apply(col[i], F::kHasX ? s_x[i] : col[i]));
        }
      }
      acc = group_reduce<Op, L>(acc);
      if (j == 0) out[(c0 + c) * out_stride] = acc;
    }
    __syncthreads();  // the next block overwrites the LDS
  }
}

// A block's slice x[c0 .. c0 + nc) of a UInt8 operand into LDS: 32-bit
// loads when x is contiguous and the slice word-aligned (one byte per lane
// and load doubled the memory instructions of a 10-row matvec).
__device__ inline void stage_x_u8(uint8_t* s_x, const uint8_t* xv, int64_t xs, int64_t c0, int64_t nc) {
  const int tid = threadIdx.x;
  if (xs == 1 && ((uintptr_t)(xv + c0) & 3) == 0) {
    const int64_t nw = nc / 4;
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(xv + c0);
    for (int64_t w = tid; w < nw; w += kDimBlock) reinterpret_cast<uint32_t*>(s_x)[w] = xw[w];
    for (int64_t c = 4 * nw + tid; c < nc; c += kDimBlock) s_x[c] = xv[c0 + c];
  } else {
    for (int64_t c = tid; c < nc; c += kDimBlock) s_x[c] = xv[(c0 + c) * xs];
  }
}

// UInt8 + by rows on dword-aligned columns (rows % 4 == 0) of the flat
// path: thread t owns 32-bit word t % W of every column (rows 4w..4w+3, W =
// rows / 4; words t, t + 256 when W > 256) and column phase t / W, and keeps
// packed 16-bit accumulators (pk16_word); phases are added in order, then
// turned into bytes.
template <int K, bool X>
__device__ inline void flat_rows_u8_words(const uint8_t* A, int64_t rows, int64_t cols, int64_t cpb, uint8_t* out,
                                          int64_t out_stride, const uint8_t* xv, int64_t xs, uint4* s_blk,
                                          uint8_t* s_x) {
  constexpr int RW = 2;  // words per thread: rows <= kFlatMaxColBytes = 2048
  const int tid = threadIdx.x;
  const int W = (int)(rows / 4);
  const int P = W <= kDimBlock ? kDimBlock / W : 1;
  const int ph = W <= kDimBlock ? tid / W : 0;
  const int w0 = W <= kDimBlock ? tid % W : tid;
  const bool active = ph < P;
  const uint32_t* sw = reinterpret_cast<const uint32_t*>(s_blk);
  uint8_t* sb = reinterpret_cast<uint8_t*>(s_blk);
  uint32_t ae[RW] = {}, ao[RW] = {};
  const int64_t nblk = (cols + cpb - 1) / cpb;
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t c0 = b * cpb;
    const int64_t nc = kmin<int64_t>(cpb, cols - c0);
    const int64_t nel = nc * rows;
    const int64_t nvec = nel / 16;
    const uint4* src = reinterpret_cast<const uint4*>(A + c0 * rows);
    uint4 v[kFlatVecs];
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) v[u] = ld_stream(src + u * kDimBlock + tid);
    if constexpr (X) stage_x_u8(s_x, xv, xs, c0, nc);
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) s_blk[u * kDimBlock + tid] = v[u];
    const int64_t e0 = nvec * 16;
    if (e0 + tid < nel) sb[e0 + tid] = A[c0 * rows + e0 + tid];
    __syncthreads();
    if (active) {
      for (int64_t c = ph; c < nc; c += P) {
        const uint32_t w16 = X ? 0x00010001u * (uint32_t)s_x[c] : 0u;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const int wi = w0 + r * kDimBlock;
          if (wi < W) pk16_word<K>(ae[r], ao[r], sw[c * W + wi], w16);
        }
      }
    }
    __syncthreads();
  }
  // phases of word w: add the packed lanes in phase order, then to bytes
  uint32_t* sp = reinterpret_cast<uint32_t*>(s_blk);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    sp[(r * kDimBlock + tid) * 2] = ae[r];
    sp[(r * kDimBlock + tid) * 2 + 1] = ao[r];
  }
  __syncthreads();
  uint8_t* o = gridDim.x == 1 ? out : out + (int64_t)blockIdx.x * rows;
  const int64_t os = gridDim.x == 1 ? out_stride : 1;
  for (int wi = tid; wi < W; wi += kDimBlock) {
    kf_us2 E = {0, 0}, O = {0, 0};
    // word wi lives at thread q*W + wi of phase q (W <= 256), or at thread wi - r*256 of slot r
    for (int q = 0; q < P; ++q) {
      const int slot = W <= kDimBlock ? q * W + wi : wi;  // r * kDimBlock + thread
      E += __builtin_bit_cast(kf_us2, sp[slot * 2]);
      O += __builtin_bit_cast(kf_us2, sp[slot * 2 + 1]);
    }
    const uint32_t bytes = pk16_bytes(__builtin_bit_cast(uint32_t, E), __builtin_bit_cast(uint32_t, O));
#pragma unroll
    for (int k = 0; k < 4; ++k) o[(int64_t)(4 * wi + k) * os] = (uint8_t)(bytes >> (8 * k));
  }
}

// UInt8 + by rows on columns off the word boundary (rows % 4 != 0) of the
// flat path: the block's bytes repeat their row pattern every P =
// lcm(rows, 4) / 4 words, so thread t owns word phase k = t % P (words k,
// k + P, ... of every block; the rows of its 4 byte lanes are fixed) and
// keeps packed 16-bit sums per byte lane (pk16); with x each byte takes its
// own column's value. At the end the threads add their byte-lane sums into
// per-row LDS totals. Needs P <= kDimBlock.
constexpr int64_t flat_period_words(int64_t rows) { return (rows % 2 == 0 ? rows / 2 : rows); }
// From 5 to 128 rows and matrices of 96 MiB (256 MiB with x); elsewhere
// the narrow kernel's element loads keep up (2 x 10^8 sum 43 against 45
// us, 254 x 10^6 49 against 53; matvec 10 x 10^7 38 against 42). Measured
// (us, narrow kernel -> this): 10 x 10^8 sum 223 -> 170, sum of squares 227
// -> 163, matvec 380 -> 328; 7 x 10^8 sum 156 -> 120; 101 x 9*10^6 sum 235
// -> 163, matvec 405 -> 320.
constexpr int kPeriodMaxRows = 128;
template <bool X> constexpr bool flat_period_ok(int64_t rows, int64_t cols) {
  return rows % 4 != 0 && rows >= 5 && rows <= kPeriodMaxRows && rows * cols >= (X ? 256LL << 20 : 96LL << 20);
}
template <int K, bool X>
__device__ inline void flat_rows_u8_period(const uint8_t* A, int64_t rows, int64_t cols, int64_t cpb, uint8_t* out,
                                           int64_t out_stride, const uint8_t* xv, int64_t xs, uint4* s_blk,
                                           uint8_t* s_x) {
  // (a static LDS array here counts against every reduce_rows_flat_kernel
  // instance, the words path included: 8 KiB of it had cost the 100- and
  // 1000-row UInt8 matvecs a workgroup per CU)
  __shared__ uint32_t s_row[kPeriodMaxRows];
  const int tid = threadIdx.x;
  const int P = (int)flat_period_words(rows);
  const int G = kDimBlock / P;           // threads per phase
  const int k = tid % P, g = tid / P;
  const bool active = g < G;
  const int cpp = (int)(4 * (int64_t)P / rows);  // columns per period
  const uint32_t* sw = reinterpret_cast<const uint32_t*>(s_blk);
  uint8_t* sb = reinterpret_cast<uint8_t*>(s_blk);
  int cb0[4];  // column of byte lane b in word k of a block
  bool nx[4];  // byte lane b in the word's second column
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    cb0[b] = (int)((4 * (int64_t)k + b) / rows);
    nx[b] = cb0[b] != cb0[0];
  }
  uint32_t ae = 0, ao = 0;
  for (int64_t i = tid; i < rows; i += kDimBlock) s_row[i] = 0;
  __syncthreads();
  const int64_t nblk = (cols + cpb - 1) / cpb;
  for (int64_t bk = blockIdx.x; bk < nblk; bk += gridDim.x) {
    const int64_t c0 = bk * cpb;
    const int64_t nc = kmin<int64_t>(cpb, cols - c0);
    const int64_t nel = nc * rows;
    const int64_t nvec = nel / 16;
    const uint4* src = reinterpret_cast<const uint4*>(A + c0 * rows);
    uint4 v[kFlatVecs];
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) v[u] = ld_stream(src + u * kDimBlock + tid);
    if constexpr (X) stage_x_u8(s_x, xv, xs, c0, nc);
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) s_blk[u * kDimBlock + tid] = v[u];
    const int64_t e0 = nvec * 16;
    if (e0 + tid < nel) sb[e0 + tid] = A[c0 * rows + e0 + tid];
    __syncthreads();
    if (active) {
      const int64_t nw = (nel + 3) / 4;
      int64_t s = g;  // period index of word k + P*s
      for (int64_t w = k + (int64_t)P * g; w < nw; w += (int64_t)P * G, s += G) {
        uint32_t a = sw[w];
        if (4 * w + 4 > nel) a &= 0xffffffffu >> (8 * (4 * w + 4 - nel));  // bytes past the block's end
        uint32_t w16e = 0, w16o = 0;
        if constexpr (X) {
          // an aligned word of rows >= 2 spans at most two columns, c and c + 1
          const int64_t c = cb0[0] + s * cpp;
          const uint32_t x0 = s_x[c], x1 = s_x[kmin<int64_t>(c + 1, nc - 1)];
          w16e = x0 | ((nx[2] ? x1 : x0) << 16);
          w16o = (nx[1] ? x1 : x0) | ((nx[3] ? x1 : x0) << 16);
        }
        const kf_us2 e = __builtin_bit_cast(kf_us2, a & 0x00ff00ffu);
        const kf_us2 o = __builtin_bit_cast(kf_us2, (a >> 8) & 0x00ff00ffu);
        kf_us2 E = __builtin_bit_cast(kf_us2, ae), O = __builtin_bit_cast(kf_us2, ao);
        if constexpr (K == 0) {
          E += e;
          O += o;
        } else if constexpr (K == 1) {
          E += e * e;
          O += o * o;
        } else {
          E += e * __builtin_bit_cast(kf_us2, w16e);
          O += o * __builtin_bit_cast(kf_us2, w16o);
        }
        ae = __builtin_bit_cast(uint32_t, E);
        ao = __builtin_bit_cast(uint32_t, O);
      }
    }
    __syncthreads();
  }
  if (active) {
    atomicAdd(&s_row[(4 * k + 0) % rows], ae & 0xffffu);
    atomicAdd(&s_row[(4 * k + 1) % rows], ao & 0xffffu);
    atomicAdd(&s_row[(4 * k + 2) % rows], ae >> 16);
    atomicAdd(&s_row[(4 * k + 3) % rows], ao >> 16);
  }
  __syncthreads();
  uint8_t* o = gridDim.x == 1 ? out : out + (int64_t)blockIdx.x * rows;
  const int64_t os = gridDim.x == 1 ? out_stride : 1;
  for (int64_t i = tid; i < rows; i += kDimBlock) o[i * os] = (uint8_t)s_row[i];
}

// dim = 2 counterpart for short contiguous columns: the same blocks of whole
// columns through LDS; thread t owns row t % rows (rows t, t + 256, ... when
// rows > 256) and column phase t / rows of every block, accumulating over
// all blocks it visits; at the end the phases of each row are combined in
// order and each workgroup writes one partial per row (or the result when
// it is alone). With a vector operand x (matvec), each block's slice of x
// is staged in LDS beside it.
template <class T, class Op, class F, int R>
__global__ __launch_bounds__(kDimBlock) void reduce_rows_flat_kernel(const T* A, int64_t rows, int64_t cols,
                                                                     int64_t cpb, T* out, int64_t out_stride,
                                                                     const T* xv, int64_t xs) {
  __shared__ uint4 s_blk[kDimBlock * kFlatVecs];
  __shared__ __align__(16) T s_x[F::kHasX ? kFlatBlockBytes / 2 / sizeof(T) : 1];
  T* sb = reinterpret_cast<T*>(s_blk);
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  if constexpr (Dot4<T, Op, F>::kind >= 0) {
    if (rows % 4 == 0) {
      flat_rows_u8_words<Dot4<T, Op, F>::kind, F::kHasX>(A, rows, cols, cpb, out, out_stride, xv, xs, s_blk, s_x);
      return;
    }
    if (flat_period_ok<F::kHasX>(rows, cols)) {
      flat_rows_u8_period<Dot4<T, Op, F>::kind, F::kHasX>(A, rows, cols, cpb, out, out_stride, xv, xs, s_blk, s_x);
      return;
    }
  }
  const int P = rows <= kDimBlock ? kDimBlock / (int)rows : 1;  // column phases
  const int ph = rows <= kDimBlock ? tid / (int)rows : 0;
  const int i0 = rows <= kDimBlock ? tid % (int)rows : tid;
  const bool active = ph < P;
  T acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = id;
  const int64_t nblk = (cols + cpb - 1) / cpb;
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t c0 = b * cpb;
    const int64_t nc = kmin<int64_t>(cpb, cols - c0);
    const int64_t nel = nc * rows;
    const int64_t nvec = nel * (int64_t)sizeof(T) / 16;
    const uint4* src = reinterpret_cast<const uint4*>(A + c0 * rows);
    uint4 v[kFlatVecs];
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) v[u] = ld_stream(src + u * kDimBlock + tid);
    if constexpr (F::kHasX)
      for (int64_t c = tid; c < nc; c += kDimBlock) s_x[c] = xv[(c0 + c) * xs];
#pragma unroll
    for (int u = 0; u < kFlatVecs; ++u)
      if (u * kDimBlock + tid < nvec) s_blk[u * kDimBlock + tid] = v[u];
    const int64_t e0 = nvec * 16 / (int64_t)sizeof(T);
    if (e0 + tid < nel) sb[e0 + tid] = A[c0 * rows + e0 + tid];
    __syncthreads();
    if (active) {
      for (int64_t c = ph; c < nc; c += P) {
        const T w = F::kHasX ? s_x[c] : id;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int64_t i = i0 + (int64_t)r * kDimBlock;
          if (i < rows) acc[r] = Op::combine(acc[r], F::apply(sb[c * rows + i], w));
        }
      }
    }
    __syncthreads();  // the next block (or the phase combine) overwrites the LDS
  }
  // rows <= 256: combine the phases of row tid in phase order; else every
  // thread holds whole rows
#pragma unroll
  for (int r = 0; r < R; ++r) sb[r * kDimBlock + tid] = acc[r];
  __syncthreads();
  T* o = gridDim.x == 1 ? out : out + (int64_t)blockIdx.x * rows;
  const int64_t os = gridDim.x == 1 ? out_stride : 1;
  if (rows <= kDimBlock) {
    if (tid < rows) {
      T a = sb[tid];
      for (int q = 1; q < P; ++q) a = Op::combine(a, sb[q * rows + tid]);
      o[tid * os] = a;
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = tid + (int64_t)r * kDimBlock;
      if (i < rows) o[i * os] = sb[r * kDimBlock + tid];
    }
  }
}

// Columns per block for reduce_cols_flat_kernel: as many as fit in
// kFlatBlockBytes, a multiple of the count that keeps block starts 16-byte
// aligned; 0 if not even that many fit.
inline int64_t flat_cols_per_block(size_t es, int64_t rows) {
  const int64_t cb = rows * (int64_t)es;
  int64_t g = 16;
  while (cb % g) g >>= 1;
  const int64_t ca = 16 / g;
  return kFlatBlockBytes / cb / ca * ca;
}

// The flat path applies to a single 16-byte aligned contiguous matrix with
// columns of at most kFlatMaxColBytes.
inline bool use_flat_cols(const void* A, int64_t rows, int64_t cs, size_t es, int64_t batch) {
  return batch == 1 && cs == rows && (uintptr_t)A % 16 == 0 && rows * (int64_t)es <= kFlatMaxColBytes &&
         flat_cols_per_block(es, rows) > 0;
}

// Columns of 2-4 KiB go flat only when a block's columns take one pass of
// the workgroup's lanes (columns x lanes per column <= 256): HIP graphs, us,
// wave per column -> flat: Float32 10^3 x 10^6 768 -> 697, 1023 rows 783 ->
// 698; Float64 500 x 10^6 781 -> 646, 511 rows 1200 -> 664, 300 rows 424 ->
// 404; but Float32 600 / 700 rows (two passes) 427 -> 466 / 460 -> 534.
inline bool use_flat_cols_dim1(const void* A, int64_t rows, int64_t cs, size_t es, int64_t batch) {
  if (use_flat_cols(A, rows, cs, es, batch)) return true;
  if (es < 4 || batch != 1 || cs != rows || (uintptr_t)A % 16 != 0 || rows * (int64_t)es > kFlatMaxColBytesWide)
    return false;
  int64_t L = 1;  // lanes per column, as launch_flat_cols picks them
  while (L < kWave && L * kFlatRowsPerLane < rows) L <<= 1;
  const int64_t cpb = flat_cols_per_block(es, rows);
  return cpb > 0 && cpb * L <= kDimBlock;
}

constexpr int kFlatRowsMinSplit = 64;  // column splits of the plan that send dims=2 to the flat path
constexpr int kFlatRowsMaxBlocks = 2048;
constexpr int kFlatRowsMinBlocks = 256;
constexpr int64_t kFlatRowsWgBytes = 64 << 10;
// Workgroups of the dims=2 flat path (one partial rows-vector each): one per
// kFlatRowsWgBytes of the matrix within [kFlatRowsMinBlocks,
// kFlatRowsMaxBlocks], at most one per block of columns; the launch takes
// the larger of this and the plan's column splits (1000 x 10^6 UInt8: 625
// us at the plan's 512 workgroups, 205 at 2048; 10 x 10^6 Float32: 14.3 us
// at the plan's 1220, 18.5 at 610 and 16.3 at 2048).
inline int64_t flat_rows_grid(size_t es, int64_t rows, int64_t cols) {
  const int64_t cpb = flat_cols_per_block(es, rows);
  const int64_t want = kmin<int64_t>(kFlatRowsMaxBlocks,
                                     kmax<int64_t>(kFlatRowsMinBlocks, rows * cols * (int64_t)es / kFlatRowsWgBytes));
  return kmin<int64_t>((cols + cpb - 1) / cpb, want);
}
// The dims=2 flat path pays for the 8-byte types, and for the 4-byte types
// whose rows are not a multiple of the vector width (the narrow kernel's
// element path): n x 10^9/n matvec, n = 10, Float32 1052 -> 851 us, Float64
// 1666 -> 1354; n = 100 Float64 1567 -> 1322, but Float32 (16-byte row units
// in the narrow kernel) 706 -> 762, and UInt8, one LDS byte per element, lost
// 10-40 % at every size.
// UInt8 + (identity, abs2, x*y) over rows that are a multiple of 4 takes it
// with packed 16-bit accumulators over 32-bit words (flat_rows_u8_words).
// 4- and 8-byte types take it for columns of 2-8 KiB too, whatever their
// row count (HIP graphs, us, narrow or strip kernels -> flat: Float64 matvec
// 300 x 10^6 604 -> 380, 500 x 10^6 791 -> 665, 511 x 10^6 947 -> 666, 700 x
// 5*10^5 581 -> 429, 1000 x 10^6 1526 -> 1276, 1000 x 10^5 195 -> 148;
// Float32 600 x 10^6 492 -> 378, 1000 x 10^6 720 -> 655, 513 x 10^6 611 ->
// 351, 1200 x 10^6 839 -> 745, 1500 x 5*10^5 613 -> 487, 2000 x 5*10^5 712
// -> 641; the one loss seen, Float64 1023 x 5*10^5, 692 -> 711)
constexpr int64_t kFlatRowsMaxColBytes = 8192;  // two columns per 16 KiB block, 8 rows per thread
inline int64_t flat_rows_max_bytes(size_t es) { return es >= 4 ? kFlatRowsMaxColBytes : kFlatMaxColBytes; }
inline bool flat_rows_shape_ok(const void* A, int64_t rows, int64_t cs, size_t es, int64_t batch) {
  return batch == 1 && cs == rows && (uintptr_t)A % 16 == 0 && rows * (int64_t)es <= flat_rows_max_bytes(es) &&
         flat_cols_per_block(es, rows) > 0;
}
template <class T, class Op, class F>
inline bool use_flat_rows(const void* A, int64_t rows, int64_t cols, int64_t cs, int64_t batch) {
  constexpr int64_t ev = 16 / (int64_t)sizeof(T);
  const bool words = Dot4<T, Op, F>::kind >= 0 && (rows % 4 == 0 || flat_period_ok<F::kHasX>(rows, cols));
  // (rows >= 2: each block's slice of x must fit the kernel's LDS for it)
  return rows >= 2 &&
         (words || (sizeof(T) >= 4 && (sizeof(T) == 8 || rows % ev != 0 || rows * (int64_t)sizeof(T) > kFlatMaxColBytes))) &&
         flat_rows_shape_ok(A, rows, cs, sizeof(T), batch);
}

template <class T, class Op, class F>
int launch_flat_rows(const T* A, int64_t rows, int64_t cols, int S, T* scratch, T* dst, int64_t ds, const T* x,
                     int64_t xs, hipStream_t stream);

// dims=1 blocks also end on a 128-byte line of a contiguous destination:
// each workgroup then writes whole lines of results, where blocks of 408
// Float32 / 204 Float64 columns (10 rows) split lines between workgroups
// (10 x 10^8 Float32 vecmat 843 -> 784 us, Float64 10 x 5*10^7 845 -> 808,
// 100 x 10^6 Float32 66 -> 59, Float64 125 -> 115).
inline int64_t flat_cols_per_block_out(size_t es, int64_t rows, int64_t ds) {
  const int64_t cpb = flat_cols_per_block(es, rows);
  if (ds != 1) return cpb;
  int64_t q = 128 / (int64_t)es;  // results per line; a multiple of the block's alignment unit
  const int64_t cb = rows * (int64_t)es;
  int64_t g = 16;
  while (cb % g) g >>= 1;
  const int64_t ca = 16 / g;
  while (q % ca) q <<= 1;
  return cpb >= q ? cpb / q * q : cpb;
}
constexpr int64_t kFlatMinPassBytes = 8192;
template <class T, class Op, class F>
int launch_flat_cols(const T* A, int64_t rows, int64_t cols, T* dst, int64_t ds, const T* x, int64_t xs,
                     hipStream_t stream) {
  // about kFlatRowsPerLane rows per lane; UInt8 takes at least 2 lanes per
  // column (one lane per column reads LDS bytes at the column stride, with
  // bank conflicts: 10 x 10^7 UInt8 vecmat 44.9 us at 1 lane, 37.6 at 2)
  int L = sizeof(T) == 1 && rows >= 4 ? 2 : 1;
  // UInt8 dot4 columns: rows counted in 4-row words
  const int64_t units = Dot4<T, Op, F>::kind >= 0 ? (rows + 3) / 4 + (rows % 4 != 0) : rows;
  const int per = units != rows ? kFlatWordsPerLane : kFlatRowsPerLane;
  if (units != rows) L = 1;
  while (L < kWave && (int64_t)L * per < units) L <<= 1;
  int64_t cpb = flat_cols_per_block_out(sizeof(T), rows, ds);
  // 4-byte columns: a block takes one pass of the lanes when that still
  // leaves at least 8 KiB per block (HIP graphs, us, sums over 10^9
  // Float32: 8 rows 818 -> 727, 10 rows 824 -> 763, 12 rows 798 -> 731, 24
  // rows 681 -> 656; 4 rows, 4 KiB blocks, 831 -> 970 is left as it was;
  // Float64 4 rows 828 -> 841, the one 8-byte case it would change)
  if (sizeof(T) == 4 && cpb * L > kDimBlock && (int64_t)(kDimBlock / L) * rows * (int64_t)sizeof(T) >= kFlatMinPassBytes)
    cpb = kDimBlock / L;
  const int64_t nblk = (cols + cpb - 1) / cpb;
  const int64_t cap = sizeof(T) != 1 ? kFlatMaxBlocks : rows >= 256 ? kFlatMaxBlocksU8Long : kFlatMaxBlocksU8;
  const dim3 grid((unsigned)kmin<int64_t>(nblk, cap));
#define KF_FLAT(LL)                                                                                            \
  hipLaunchKernelGGL((reduce_cols_flat_kernel<T, Op, F, LL>), grid, dim3(kDimBlock), 0, stream, A, rows, cols, cpb, \
                     dst, ds, x, xs)
  switch (L) {
    case 1: KF_FLAT(1); break;
    case 2: KF_FLAT(2); break;
    case 4: KF_FLAT(4); break;
    case 8: KF_FLAT(8); break;
    case 16: KF_FLAT(16); break;
    case 32: KF_FLAT(32); break;
    default: KF_FLAT(64); break;
  }
#undef KF_FLAT
  return kf_check_launch("reduce_cols_flat_kernel");
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
  // Vector launches have rows % EPV == 0; the last strip may be partial: its
  // vectors past the end load nothing and store nothing (the rows beyond the
  // last column's end may lie past the allocation)
  bool in_strip[kRowVecs];
#pragma unroll
  for (int u = 0; u < kRowVecs; ++u) in_strip[u] = strip + (int64_t)(u * kDimBlock + tid) * EPV < rows;
  if constexpr (VEC && Dot4<T, Op, F>::kind >= 0) {
    // UInt8 +: packed 16-bit accumulators
    constexpr int K = Dot4<T, Op, F>::kind;
    uint32_t ae[kRowVecs][4] = {}, ao[kRowVecs][4] = {};
    const T* p = A + strip;
    int64_t c = c0;
    for (; c + kColUnroll <= c1; c += kColUnroll) {
      uint4 r[kColUnroll][kRowVecs];
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q)
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u)
          r[q][u] = in_strip[u] ? ld_stream(reinterpret_cast<const uint4*>(p + (c + q) * col_stride) + u * kDimBlock + tid)
                                : uint4{0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q) {
        const uint32_t w16 = F::kHasX ? 0x00010001u * (uint32_t)xv[(c + q) * xs] : 0u;
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u) pk16_vec<K>(ae[u], ao[u], r[q][u], w16);
      }
    }
    for (; c < c1; ++c) {
      const uint32_t w16 = F::kHasX ? 0x00010001u * (uint32_t)xv[c * xs] : 0u;
#pragma unroll
      for (int u = 0; u < kRowVecs; ++u)
        pk16_vec<K>(ae[u], ao[u],
                    in_strip[u] ? ld_stream(reinterpret_cast<const uint4*>(p + c * col_stride) + u * kDimBlock + tid)
                                : uint4{0, 0, 0, 0},
                    w16);
    }
#pragma unroll
    for (int u = 0; u < kRowVecs; ++u) {
      const uint32_t wd[4] = {pk16_bytes(ae[u][0], ao[u][0]), pk16_bytes(ae[u][1], ao[u][1]),
                              pk16_bytes(ae[u][2], ao[u][2]), pk16_bytes(ae[u][3], ao[u][3])};
      __builtin_memcpy(a[u], wd, sizeof(wd));
    }
  } else if constexpr (VEC) {
  {
    const T* p = A + strip;
    int64_t c = c0;
    for (; c + kColUnroll <= c1; c += kColUnroll) {
      uint4 r[kColUnroll][kRowVecs];
#pragma unroll
      for (int q = 0; q < kColUnroll; ++q)
#pragma unroll
        for (int u = 0; u < kRowVecs; ++u)
          r[q][u] = in_strip[u] ? ld_stream(reinterpret_cast<const uint4*>(p + (c + q) * col_stride) + u * kDimBlock + tid)
                                : uint4{0, 0, 0, 0};
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
        const uint4 r = in_strip[u] ? ld_stream(reinterpret_cast<const uint4*>(p + c * col_stride) + u * kDimBlock + tid)
                                    : uint4{0, 0, 0, 0};
        T x[EPV];
        __builtin_memcpy(x, &r, sizeof(x));
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], F::apply(x[e], w));
      }
    }
  }
  } else {
    // element path (unaligned): kColUnroll columns of loads in flight; rows
    // past the end read row 0's element and drop it
    int64_t c = c0;
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
  for (int u = 0; u < kRowVecs; ++u) {
    const int64_t r0 = strip + (int64_t)(u * kDimBlock + tid) * EPV;
    if (r0 >= rows) continue;
    T* o = gridDim.y == 1 ? out + r0 * out_stride : out + (int64_t)s * rows + r0;
    if (VEC && (gridDim.y > 1 || out_stride == 1) && (uintptr_t)o % 16 == 0) {
      // a whole vector of rows, contiguous aligned outputs: one 16-byte store
      uint4 v;
      __builtin_memcpy(&v, a[u], sizeof(v));
      *reinterpret_cast<uint4*>(o) = v;
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e)
        if (r0 + e < rows) o[gridDim.y == 1 ? e * out_stride : e] = a[u][e];
    }
  }
}


// dim = 2 over few columns (2..kFewMaxCols, rows a multiple of the vector
// width, 16-byte aligned columns) of matrices up to kFewMaxBytes: thread i
// reads vector i of every column in one batch of loads and stores one
// output vector, grid-stride over the rows. The strip kernel above carries
// at most kColUnroll columns of loads per pass and takes the remainder one
// column at a time (10 columns at 8 vectors per thread: 4, 4, 1, 1).
// Measured (HIP graphs, us, strip kernel -> this): matvec 10^6 x 10 Float32
// 11.5 -> 9.6, Float64 21.2 -> 15.8, UInt8 10.9 -> 8.0; 10^7 x 10 Float32
// 85.8 -> 80.7, Float64 156 -> 146, UInt8 31.1 -> 25.4. Larger matrices
// stream better through the strips, whose threads read 1-2 KiB runs per
// column (10^8 x 10 Float32 771 us there, 893 here), and UInt8 x*y keeps its
// 16 packed operands in VGPRs (129, 3 waves per SIMD): up to 32 MiB only.
constexpr int kFewMaxCols = 16;
constexpr int kFewBlocks = 4096;
constexpr int64_t kFewMaxBytes = 512LL << 20;
// a single column (a scaled copy) streams better through the strips beyond
// 128 MiB (10^8 x 1 Float32 169 against 146 us; 10^7 x 1 17.5 against 21.1)
constexpr int64_t kFewMaxBytesOne = 128LL << 20;
constexpr int64_t kFewMaxBytesU8X = 32LL << 20;
template <class T, class Op, class F>
__global__ __launch_bounds__(kDimBlock) void reduce_rows_few_kernel(
    const T* A, int64_t rows, int cols, int64_t col_stride, T* out, int64_t out_stride, const T* xv, int64_t xs) {
  constexpr int EPV = 16 / (int)sizeof(T);
  constexpr int C = kFewMaxCols;
  constexpr int K = Dot4<T, Op, F>::kind;
  const T id = Op::template identity<T>();
  T w[C];
#pragma unroll
  for (int c = 0; c < C; ++c) w[c] = F::kHasX && c < cols ? xv[c * xs] : id;
  const int64_t nv = rows / EPV;
  for (int64_t i = (int64_t)blockIdx.x * kDimBlock + threadIdx.x; i < nv; i += (int64_t)gridDim.x * kDimBlock) {
    uint4 r[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (c < cols) r[c] = ld_stream(reinterpret_cast<const uint4*>(A + c * col_stride) + i);
    T a[EPV];
    if constexpr (K >= 0) {
      // UInt8 +: packed 16-bit accumulators, two rows per instruction
      uint32_t ae[4] = {}, ao[4] = {};
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (c < cols) pk16_vec<K>(ae, ao, r[c], F::kHasX ? 0x00010001u * (uint32_t)w[c] : 0u);
      const uint32_t wd[4] = {pk16_bytes(ae[0], ao[0]), pk16_bytes(ae[1], ao[1]), pk16_bytes(ae[2], ao[2]),
                              pk16_bytes(ae[3], ao[3])};
      __builtin_memcpy(a, wd, sizeof(wd));
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = id;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c >= cols) continue;
        T x[EPV];
        __builtin_memcpy(x, &r[c], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], F::apply(x[e], w[c]));
      }
    }
    T* o = out + i * EPV * out_stride;
    if (out_stride == 1 && (uintptr_t)o % 16 == 0) {
      uint4 v;
      __builtin_memcpy(&v, a, sizeof(v));
      *reinterpret_cast<uint4*>(o) = v;
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) o[e * out_stride] = a[e];
    }
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
// Workgroups over batch x column ranges: 512 to 2048 by matrix size (n x p
// Float32 matrices, n = 10 / 100 / 1000, p = 10^9 / n: 2817 / 901 / 855 us
// at 512, 1052 / 701 / 692 at 2048; the combine of 2048 ranges cost UInt8
// n x 10^7 / n matrices 3-6 us).
constexpr int kNarrowBlocks = 2048;
constexpr int kNarrowMinBlocks = 512;
constexpr int64_t kNarrowWgBytes = 32 << 10;
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
  int multi_split; // dim 1, at most kMultiMaxCols columns: workgroups of reduce_cols_multi_kernel
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
      if (vec && cols <= kMultiMaxCols && rows * cols * (int64_t)es >= kMultiMinBytes) {
        // one vector per thread up to kMultiBlocks workgroups (10^6 x 10
        // Float32 vecmat: 14.6 us at the wave-per-column split's 244)
        const int64_t nv = rows / epv;
        p.multi_split = (int)kmax<int64_t>(1, kmin<int64_t>(kMultiBlocks, (nv + kDimBlock - 1) / kDimBlock));
      }
    }
  } else if (row_units(es, rows, vec) <= kDimBlock) {
    // Narrow: one strip covers every row; column ranges fill the GPU.
    const int64_t nu = row_units(es, rows, vec);
    p.narrow = true;
    p.unit_vec = vec && nu != rows;
    p.groups = 1;
    const int64_t P = kDimBlock / kmax<int64_t>(nu, 1);
    // workgroups: one per kNarrowWgBytes of the matrix, within
    // [kNarrowMinBlocks, kNarrowBlocks], so large matrices keep enough loads
    // in flight and small ones a short combine
    const int64_t target = kmin<int64_t>(kNarrowBlocks, kmax<int64_t>(kNarrowMinBlocks, rows * cols * (int64_t)es * nb /
                                                                                         kNarrowWgBytes));
    int64_t S = (target + nb - 1) / nb;
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
        if (rows / rsc * nb >= kDim2Blocks) {  // whole strips only
          rv = c;
          break;
        }
      }
    }
    if (vec) {
      // UInt8: at most 2 vectors per thread (10^7 x 100 matvec 199 -> 180
      // us, 1000 x 10^6 at 8 and 4 vectors 242 / 230 against 174); few
      // columns (larger than reduce_rows_few_kernel takes): one vector per
      // thread, more strips in flight (10^8 x 10 Float32 826 -> 771 us,
      // Float64 1676 -> 1544)
      if (es == 1) rv = kmin(rv, kDim2MaxRowVecsU8);
      if (cols <= kFewMaxCols) rv = es == 1 ? kmin(rv, 2) : 1;
    }
    p.row_vecs = rv;
    const int cu = vec ? col_unroll_for(rv) : kColUnrollDefault;
    const int64_t rs = (int64_t)kDimBlock * rv * epv;
    p.groups = (rows + rs - 1) / rs;
    int64_t S = 1;
    // few strips: split columns until kDim2SplitBlocks workgroups (10^4 x
    // 10^4 Float32 98.9 -> 77.5 us at 10 strips), else until kDim2Blocks
    // (65536 x 4096, 64 strips: 159 us at S = 4, 172 at S = 16)
    const int64_t want = p.groups * nb < kDim2FewStrips ? kDim2SplitBlocks : kDim2Blocks;
    const int64_t g = p.groups * nb;
    const int64_t smax = kmin<int64_t>(256, kmax<int64_t>(cols / (2 * cu), 1));
    if (g < want) S = kmin<int64_t>((want + g - 1) / g, smax);
    // whole rounds of workgroups over the CUs: the fewest splits from S up
    // whose grid is within 7 % of a multiple of the CU count (HIP graphs,
    // us, matvec: 10^5 x 10^4 Float32, 97 strips, 741 at S = 3 (291
    // workgroups, 35 CUs with two) -> 587 at S = 5, Float64 1305 -> 1262;
    // 3*10^5 x 3000 Float32, 292 strips, 689 at S = 1 -> 581; 10^4 x 10^5
    // Float64 1308 -> 1220; 10^5 x 10^3 Float32 90 -> 75; UInt8 10^5 x 10^4
    // 206 -> 194)
    const auto over = [&](int64_t t) {
      const int64_t w = g * t;
      return (w + kDim2Blocks - 1) / kDim2Blocks * kDim2Blocks * 100 > w * 107;
    };
    if (over(S))
      for (int64_t t = S + 1; t <= kmin<int64_t>(8 * S, smax); ++t)
        if (!over(t)) {
          S = t;
          break;
        }
    p.split = (int)S;
  }
  const int64_t parts = kmax<int64_t>(p.split, p.multi_split);
  if (parts > 1) p.partial_bytes = round256((size_t)parts * (size_t)(dim == 1 ? cols : rows) * es * (size_t)nb);
  return p;
}

// A single row reduced along dim 2, or a single column along dim 1: the
// entry points hand these to the 1-D reductions (kf_reduce, kf_reduce2),
// which stream them with every workgroup reading contiguous memory (one row
// of a 1 x 10^8 Float32 matrix: 2.2 TB/s through the narrow dim-2 kernel).
inline bool dim_is_1d(int64_t rows, int64_t cols, int dim) { return dim == 2 ? rows == 1 : cols == 1; }

inline bool dim_vec_ok(const void* A, int64_t cs, size_t es) {
  return ((uintptr_t)A % 16 == 0) && ((cs * (int64_t)es) % 16 == 0);
}

// Alignment decisions of a dims launch, shared by the entry-point scratch
// checks and the launch itself. vec: 16-byte paths. peel (dim 2): A is
// misaligned but every column (and batch entry) shares its misalignment, so
// the first `peel` rows go to an element-path launch and the rest, from an
// aligned A + peel, to the vector paths.
// Shorter columns stay on the element path: split-off head and tail rows
// would fetch each column's first and last lines again (16 rows: 2.0 TB/s
// split against 2.9 unsplit).
constexpr int64_t kPeelMinColumnBytes = 2048;
struct DimVec {
  bool vec;
  int64_t head, tail;  // dim 2 rows split off to element-path launches
};
inline DimVec dim_vec(const void* A, int64_t rows, int64_t cs, size_t es, int dim, int64_t batch,
                      int64_t a_bstride, bool has_x, const void* x, int64_t xs) {
  const bool strides16 = (cs * (int64_t)es) % 16 == 0 && (batch <= 1 || (a_bstride * (int64_t)es) % 16 == 0);
  DimVec v{strides16 && (uintptr_t)A % 16 == 0, 0, 0};
  // vecmat (dim 1 with an operand) reads x along the rows: vector path only if x is too
  if (has_x && dim == 1) v.vec = v.vec && xs == 1 && (uintptr_t)x % 16 == 0;
  if (dim == 2 && strides16) {
    // head: rows before the first 16-byte boundary; tail: rows after the
    // last whole vector. The vector launch in between has rows % EPV == 0.
    const int64_t ev = (int64_t)(16 / es);
    const int64_t h = (int64_t)(((16 - (uintptr_t)A % 16) % 16) / es);
    if (h < rows && rows * (int64_t)es >= kPeelMinColumnBytes) {
      const int64_t t = (rows - h) % ev;
      if (rows - h - t > 0 && (h > 0 || t > 0)) v = {true, h, t};
    }
  }
  // an unsplit dim-2 vector launch needs rows % EPV == 0
  if (dim == 2 && v.vec && !v.head && !v.tail && rows % (int64_t)(16 / es) != 0) v.vec = false;
  return v;
}

// Partial bytes of a dim-2 vector launch (one launch, the last strip
// possibly partial).
inline size_t dim2_vec_need(size_t es, int64_t rows, int64_t cols, int64_t batch) {
  return plan_dim(es, rows, cols, 2, true, batch).partial_bytes;
}

// Partial bytes the launch will use for this alignment (0: no scratch).
inline size_t dim_need(size_t es, int64_t rows, int64_t cols, int dim, int64_t batch, DimVec v) {
  if (v.head || v.tail) {
    size_t b = dim2_vec_need(es, rows - v.head - v.tail, cols, batch);
    if (v.head) b = kmax(b, plan_dim(es, v.head, cols, 2, false, batch).partial_bytes);
    if (v.tail) b = kmax(b, plan_dim(es, v.tail, cols, 2, false, batch).partial_bytes);
    return b;
  }
  if (dim == 2 && v.vec) return dim2_vec_need(es, rows, cols, batch);
  return plan_dim(es, rows, cols, dim, v.vec, batch).partial_bytes;
}
// Scratch query: the largest need over every alignment case.
inline size_t dim_query(size_t es, int64_t rows, int64_t cols, int dim, int64_t batch) {
  size_t b = kmax(plan_dim(es, rows, cols, dim, true, batch).partial_bytes,
                  plan_dim(es, rows, cols, dim, false, batch).partial_bytes);
  if (dim == 2) {
    const int64_t ev = (int64_t)(16 / es);
    if (rows % ev == 0) b = kmax(b, dim2_vec_need(es, rows, cols, batch));
    if (flat_rows_shape_ok(nullptr, rows, rows, es, batch))
      b = kmax(b, round256((size_t)flat_rows_grid(es, rows, cols) * (size_t)rows * es));  // the flat path's partials
    for (int64_t h = 0; h < ev && h < rows; ++h) {
      const int64_t t = (rows - h) % ev;  // the tail a head of h rows leaves
      if (rows - h - t > 0 && (h > 0 || t > 0)) b = kmax(b, dim_need(es, rows, cols, 2, batch, {true, h, t}));
    }
  }
  return kRedReserved + kmax<size_t>(256, b);
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

// combine_cols_kernel from kCombMinSplits partial columns of more than
// kCombMinUnits row units (fewer rows leave most of its lanes idle, where
// the narrow kernel's phases use them)
constexpr int kCombMinSplits = 16;
constexpr int kCombMinUnits = 16;
// Second stage of a split dims reduction: nz batches of an m x S partial
// matrix (column s at s*m, batch z at z*S*m; the scratch is 256-byte
// aligned) reduced along dim 2 into dst[i*ds + z*dst_bstride].
template <class T, class Op>
void launch_combine(const T* part, int S, int64_t m, T* dst, int64_t ds, int64_t dst_bstride, unsigned nz,
                    hipStream_t stream) {
  const int64_t nu = row_units(sizeof(T), m, true);
  if (nu > kCombMinUnits && S >= kCombMinSplits)
    hipLaunchKernelGGL((combine_cols_kernel<T, Op>), dim3((unsigned)((m + kWave - 1) / kWave), nz),
                       dim3(kCombWaves * kWave), 0, stream, part, S, m, dst, ds, dst_bstride);
  else if (nu <= kDimBlock)
    launch_narrow<T, Op, Unary<MapIdentity>>(nu != m, dim3(1, 1, nz), part, m, S, m, dst, ds, S, (int64_t)S * m,
                                             dst_bstride, nullptr, 0, stream);
  else
    hipLaunchKernelGGL((combine_split_kernel<T, Op>), dim3((unsigned)((m + kRedBlock - 1) / kRedBlock), nz),
                       dim3(kRedBlock), 0, stream, part, S, m, dst, ds, dst_bstride);
}

// S persistent workgroups write S partial rows-vectors into the scratch,
// combined by launch_combine (S = 1: straight into dst).
// UInt8 takes at most 6 workgroups per CU (HIP graphs, us, at 3 / 4 / 5 /
// 6 / 8 per CU): 100 x 10^7 sum 219 / 183 / 163 / 158 / 178, 1000 x 10^6
// sum 213 / 176 / 158 / 163 / 180, 128 x 7812500 sum 215 / 177 / 158 / 157
// / 175; matvec 100 x 10^7 254 / 215 / 193 / 197 / 196.
constexpr int kFlatRowsU8PerCu = 6;
template <class T, class Op, class F>
int launch_flat_rows(const T* A, int64_t rows, int64_t cols, int S, T* scratch, T* dst, int64_t ds, const T* x,
                     int64_t xs, hipStream_t stream) {
  const int64_t cpb = flat_cols_per_block(sizeof(T), rows);
  const int R = (int)((rows + kDimBlock - 1) / kDimBlock);
  // persistent: at most the workgroups the GPU holds at once, each one
  // partial rows-vector (10 x 10^8 matvec Float32 859 -> 768 us, 100 x 10^7
  // UInt8 211 -> 176 us, Float64 1323 -> 1263 us; the dims=1 flat kernel
  // keeps its 4096 workgroups, 1-10 % faster than a resident-sized grid)
#define KF_FLATR(RR)                                                                                          \
  do {                                                                                                        \
    constexpr auto kernel = reduce_rows_flat_kernel<T, Op, F, RR>;                                            \
    S = (int)kmin<int64_t>(S, resident_blocks<kernel>(kDimBlock));                                            \
    if (sizeof(T) == 1) S = (int)kmin<int64_t>(S, kFlatRowsU8PerCu * kf_device_cu_count());                \
    hipLaunchKernelGGL(kernel, dim3((unsigned)S), dim3(kDimBlock), 0, stream, A, rows, cols, cpb,             \
                       S > 1 ? scratch : dst, ds, x, xs);                                                     \
  } while (0)
  if (R <= 1) KF_FLATR(1);
  else if (R <= 2) KF_FLATR(2);
  else if (R <= 4) KF_FLATR(4);
  else KF_FLATR(8);
#undef KF_FLATR
  if (S > 1) launch_combine<T, Op>(scratch, S, rows, dst, ds, 0, 1, stream);
  return kf_check_launch("reduce_rows_flat_kernel");
}

// A reduction over a dimension of length 1 (dims=1 over one row, dims=2
// over one column): every output is f of one element, out[k*os] =
// f(A[k*as], x[0]), a streaming map (16-byte loads and stores when both
// sides are contiguous and aligned). Through the flat dims=1 kernel one
// 1-byte column per lane had taken 1 x 10^8 UInt8 vecmat to 136 us.
constexpr int kMapOneBlocks = 8192;  // element path: grid-stride
// vector path: one-shot workgroups of kMapOneVecs vectors per lane (HIP
// graphs, us, 1, 2, 4 vectors: Float64 10^8 x 1 matvec 245 / 263 / 268,
// 1 x 10^8 vecmat 243 / 266 / 266; Float32 122 / 129 / 132)
constexpr int kMapOneVecs = 1;
template <class T, class F>
__global__ __launch_bounds__(kDimBlock) void map_one_kernel(const T* A, int64_t n, int64_t as, T* out, int64_t os,
                                                            const T* xv, int vec) {
  constexpr int EPV = 16 / (int)sizeof(T);
  constexpr int U = kMapOneVecs;
  const T x0 = F::kHasX ? xv[0] : T();
  const int tid = threadIdx.x;
  if (vec) {
    // workgroup b maps vectors [b*U*256, (b+1)*U*256), its loads in flight
    // before any store; workgroup 0 also maps the tail elements
    const int64_t nv = n / EPV;
    const uint4* src = reinterpret_cast<const uint4*>(A);
    uint4* dst = reinterpret_cast<uint4*>(out);
    const int64_t base = (int64_t)blockIdx.x * (U * kDimBlock) + tid;
    uint4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kDimBlock < nv) r[u] = ld_stream(src + base + u * kDimBlock);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kDimBlock < nv) {
        T a[EPV];
        __builtin_memcpy(a, &r[u], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[e] = F::apply(a[e], F::kHasX ? x0 : a[e]);
        uint4 w;
        __builtin_memcpy(&w, a, 16);
        st_stream(dst + base + u * kDimBlock, w);
      }
    if (blockIdx.x == 0)
      for (int64_t k = nv * EPV + tid; k < n; k += kDimBlock) out[k] = F::apply(A[k], F::kHasX ? x0 : A[k]);
    return;
  }
  const int64_t step = (int64_t)gridDim.x * kDimBlock;
  for (int64_t k = (int64_t)blockIdx.x * kDimBlock + tid; k < n; k += step) {
    const T a = A[k * as];
    out[k * os] = F::apply(a, F::kHasX ? x0 : a);
  }
}

template <class T, class F>
int launch_map_one(const T* A, int64_t n, int64_t as, T* out, int64_t os, const T* x, hipStream_t stream) {
  const int vec = as == 1 && os == 1 && (uintptr_t)A % 16 == 0 && (uintptr_t)out % 16 == 0;
  const int64_t per = vec ? (int64_t)kDimBlock * kMapOneVecs * (16 / (int64_t)sizeof(T)) : kDimBlock;
  int64_t grid = (n + per - 1) / per;
  if (!vec) grid = kmin<int64_t>(grid, kMapOneBlocks);
  if (grid > (int64_t)(0xffffffffu / kDimBlock))  // threads of one launch: fewer than 2^32
    return kf_set_error(KF_EINVAL, "map_one_kernel: %lld elements exceed one launch", (long long)n);
  hipLaunchKernelGGL((map_one_kernel<T, F>), dim3((unsigned)kmax<int64_t>(grid, 1)), dim3(kDimBlock), 0, stream, A,
                     n, as, out, os, x, vec);
  return kf_check_launch("map_one_kernel");
}

template <class T, class Op, class F>
int launch_reduce_dim(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst,
                      int64_t ds, void* scratch, hipStream_t stream, int64_t batch = 1, int64_t a_bstride = 0,
                      const void* x = nullptr, int64_t xs = 0, int64_t dst_bstride = -1, bool may_peel = true) {
  if (dst_bstride < 0) dst_bstride = rows * ds;
  if (batch <= 1 && (dim == 1 ? rows == 1 && cols > 1 : cols == 1 && rows > 1))
    return dim == 1 ? launch_map_one<T, F>((const T*)A, cols, cs, (T*)dst, ds, (const T*)x, stream)
                    : launch_map_one<T, F>((const T*)A, rows, 1, (T*)dst, ds, (const T*)x, stream);
  const DimVec dv = dim_vec(A, rows, cs, sizeof(T), dim, batch, a_bstride, F::kHasX, x, xs);
  if (dim == 2 && !dv.head && !dv.tail && use_flat_rows<T, Op, F>(A, rows, cols, cs, batch)) {
    // short contiguous columns: the LDS-staged flat kernel, with as many
    // workgroups (and partial rows-vectors) as the plan's column splits
    const DimPlan pf = plan_dim(sizeof(T), rows, cols, 2, dv.vec, batch);
    // workgroups: the plan's column splits or the flat grid, whichever is
    // larger (the scratch query covers both partial sets)
    if (pf.split >= kFlatRowsMinSplit)
      return launch_flat_rows<T, Op, F>((const T*)A, rows, cols,
                                        (int)kmax<int64_t>(pf.split, flat_rows_grid(sizeof(T), rows, cols)),
                                        (T*)scratch, (T*)dst, ds, (const T*)x, xs, stream);
  }
  if (may_peel && (dv.head || dv.tail)) {
    // element-path launches for the head and tail rows around the vector
    // launch; stream order lets all of them use the same scratch
    const int64_t body = rows - dv.head - dv.tail;
    int rc = KF_OK;
    if (dv.head)
      rc = launch_reduce_dim<T, Op, F>(A, dv.head, cols, cs, 2, dst, ds, scratch, stream, batch, a_bstride, x, xs,
                                       dst_bstride, false);
    if (!rc)
      rc = launch_reduce_dim<T, Op, F>((const T*)A + dv.head, body, cols, cs, 2, (T*)dst + dv.head * ds, ds, scratch,
                                       stream, batch, a_bstride, x, xs, dst_bstride, false);
    if (!rc && dv.tail)
      rc = launch_reduce_dim<T, Op, F>((const T*)A + dv.head + body, dv.tail, cols, cs, 2,
                                       (T*)dst + (dv.head + body) * ds, ds, scratch, stream, batch, a_bstride, x, xs,
                                       dst_bstride, false);
    return rc;
  }
  const bool vec = dv.vec;
  if (dim == 2 && vec && batch <= 1 && cols <= kFewMaxCols && rows % (int64_t)(16 / sizeof(T)) == 0 &&
      row_units(sizeof(T), rows, true) > kDimBlock &&
      rows * cols * (int64_t)sizeof(T) <=
          (Dot4<T, Op, F>::kind == 2 ? kFewMaxBytesU8X : cols == 1 ? kFewMaxBytesOne : kFewMaxBytes)) {
    const int64_t nv = rows / (int64_t)(16 / sizeof(T));
    const unsigned grid = (unsigned)kmin<int64_t>((nv + kDimBlock - 1) / kDimBlock, kFewBlocks);
    hipLaunchKernelGGL((reduce_rows_few_kernel<T, Op, F>), dim3(grid), dim3(kDimBlock), 0, stream, (const T*)A,
                       rows, (int)cols, cs, (T*)dst, ds, (const T*)x, xs);
    return kf_check_launch("reduce_rows_few_kernel");
  }
  const DimPlan p = plan_dim(sizeof(T), rows, cols, dim, vec, batch);
  if (dim == 1) {
    if (use_flat_cols_dim1(A, rows, cs, sizeof(T), batch))
      return launch_flat_cols<T, Op, F>((const T*)A, rows, cols, (T*)dst, ds, (const T*)x, xs, stream);
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
    if constexpr (F::kHasX) {
      if (p.multi_split > 0) {
        const int S = p.multi_split;
        int64_t mseg = (rows + S - 1) / S;
        mseg = (mseg + EPV - 1) / EPV * EPV;
        hipLaunchKernelGGL((reduce_cols_multi_kernel<T, Op, F>), dim3((unsigned)S), dim3(kDimBlock), 0, stream,
                           (const T*)A, rows, (int)cols, cs, S > 1 ? (T*)scratch : (T*)dst, ds, mseg, (const T*)x);
        if (S > 1) launch_combine<T, Op>((const T*)scratch, S, cols, (T*)dst, ds, 0, 1, stream);
        return kf_check_launch("reduce_cols_multi_kernel");
      }
    }
    hipLaunchKernelGGL((reduce_cols_kernel<T, Op, F>), dim3((unsigned)p.groups, p.split), dim3(kDimBlock), 0,
                       stream, (const T*)A, rows, cols, cs, out, ds, seg, (int)vec, (const T*)x, xs);
    if (p.split > 1) launch_combine<T, Op>((const T*)scratch, p.split, cols, (T*)dst, ds, 0, 1, stream);
    return kf_check_launch("reduce_cols_kernel");
  }
  // dim 2, batched: dst[i*ds + z*dst_bstride] = op_j f(A[i + j*cs + z*a_bstride])
  const int64_t seg = (cols + p.split - 1) / p.split;
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

template <class T, class Op, class Map> struct ReduceDimL {
  static int run(const void* A, int64_t rows, int64_t cols, int64_t cs, int dim, void* dst, int64_t ds,
                 void* scratch, hipStream_t s, int64_t batch, int64_t a_bstride) {
    return launch_reduce_dim<T, Op, Unary<Map>>(A, rows, cols, cs, dim, dst, ds, red_work(scratch), s, batch,
                                                a_bstride);
  }
};

}  // namespace kf
