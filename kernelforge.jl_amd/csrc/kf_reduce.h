// Definitions shared by kf_reduce.hip (full and multi-array reductions) and
// kf_reduce_dims.hip (reductions along dims, matvec / vecmat).
#pragma once
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

// Two-operand element maps: reduce2 (dot product, squared distance and the
// asymmetric maps) and the matvec / vecmat operand map.
// v_dot4_u32_u8 folds: K 0 = sum of the four bytes, 1 = sum of their
// squares, 2 = dot product with the operand's four bytes. The low byte of a
// 32-bit sum of UInt8 terms is their mod-256 (Julia UInt8) sum.
template <int K> __device__ inline uint32_t dot4_word(uint32_t acc, uint32_t a, uint32_t x) {
  return __builtin_amdgcn_udot4(a, K == 0 ? 0x01010101u : K == 1 ? a : x, acc, false);
}
template <int K> __device__ inline uint32_t dot4_vec(uint32_t acc, uint4 a, uint4 x) {
  acc = dot4_word<K>(acc, a.x, x.x);
  acc = dot4_word<K>(acc, a.y, x.y);
  acc = dot4_word<K>(acc, a.z, x.z);
  return dot4_word<K>(acc, a.w, x.w);
}

// Per-lane fold of 16-byte vectors of T for the 1-D reductions: one
// accumulator per element slot, combined in slot order at the end; UInt8 +
// over identity or abs2 keeps one 32-bit dot4 sum instead (four bytes per
// instruction rather than sixteen byte operations per vector).
template <class T, class Op, class Map> struct VecFold {
  static constexpr int EPV = 16 / (int)sizeof(T);
  static constexpr int K = !__is_same(T, uint8_t) || !__is_same(Op, OpAdd) ? -1
                           : __is_same(Map, MapIdentity)                  ? 0
                           : __is_same(Map, MapAbs2)                      ? 1
                                                                          : -1;
  T a[K >= 0 ? 1 : EPV];
  uint32_t d = 0;
  __device__ VecFold() {
#pragma unroll
    for (int e = 0; e < (K >= 0 ? 1 : EPV); ++e) a[e] = Op::template identity<T>();
  }
  __device__ void add(uint4 r) {
    if constexpr (K >= 0) {
      d = dot4_vec<K>(d, r, r);
    } else {
      T x[EPV];
      __builtin_memcpy(x, &r, 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[e] = Op::combine(a[e], Map::apply(x[e]));
    }
  }
  __device__ T total() const {
    if constexpr (K >= 0) {
      return (T)d;
    } else {
      T acc = a[0];
#pragma unroll
      for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, a[e]);
      return acc;
    }
  }
};

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

}  // namespace kf
