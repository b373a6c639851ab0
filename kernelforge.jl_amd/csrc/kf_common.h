// Shared device-side vocabulary for the scan / mapreduce kernels on gfx950:
// element types, the fixed operator set, wave64 DPP primitives and the
// launch-error plumbing used by every entry point.
//
// Operator semantics follow Julia Base as used by KernelForge
// (reference: src/helpers.jl:133-175 for the left fold, src/scan/scan_kernel.jl:1-7
// for prefix application `op(prefix, v)`):
//   +      IEEE add for floats, wrap-around (mod 2^bits) for integers
//   max    NaN-propagating, -0.0 < +0.0 (Julia `max` on IEEE floats)
//   min    NaN-propagating, -0.0 < +0.0
//   affine (a1,b1) o (a2,b2) = (a2*a1, a2*b1 + b2)  (left operand is older)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/kf.h"

namespace kf {

constexpr int kWave = 64;

template <class T> __host__ __device__ constexpr T kmin(T a, T b) { return a < b ? a : b; }
template <class T> __host__ __device__ constexpr T kmax(T a, T b) { return a < b ? b : a; }

// (a, b) pair of the affine recurrence x_t = a_t * x_{t-1} + b_t.
struct __attribute__((aligned(8))) f32x2 {
  float a, b;
};

// Quaternions s + v1 i + v2 j + v3 k, laid out as Julia's Quaternion{T}
// (fields s, v1, v2, v3): QuaternionF32 16 bytes, QuaternionF64 32 bytes.
template <class F> struct quat {
  F s, v1, v2, v3;
};
using q32 = quat<float>;
using q64 = quat<double>;
template <class T> constexpr bool is_quat = __is_same(T, q32) || __is_same(T, q64);

// ---------------------------------------------------------------------------
// Operators. Each provides identity<T>() and combine(older, newer).
// ---------------------------------------------------------------------------
struct OpAdd {
  template <class T> __device__ static T identity();
  __device__ static float combine(float x, float y) { return x + y; }
  __device__ static double combine(double x, double y) { return x + y; }
  __device__ static int32_t combine(int32_t x, int32_t y) {
    return (int32_t)((uint32_t)x + (uint32_t)y);
  }
  __device__ static int64_t combine(int64_t x, int64_t y) {
    return (int64_t)((uint64_t)x + (uint64_t)y);
  }
  __device__ static uint8_t combine(uint8_t x, uint8_t y) { return (uint8_t)(x + y); }
};
// -0.0 is the exact additive identity: -0.0 + x == x bit-for-bit for every x.
template <> __device__ inline float OpAdd::identity<float>() { return -0.0f; }
template <> __device__ inline double OpAdd::identity<double>() { return -0.0; }
template <> __device__ inline int32_t OpAdd::identity<int32_t>() { return 0; }
template <> __device__ inline int64_t OpAdd::identity<int64_t>() { return 0; }
template <> __device__ inline uint8_t OpAdd::identity<uint8_t>() { return 0; }

struct OpMax {
  template <class T> __device__ static T identity();
  // IEEE 754-2019 maximum (v_maximum3_f32 on gfx950): NaN-propagating and
  // orders -0.0 below +0.0, which is exactly Julia's `max` on floats.
  __device__ static float combine(float x, float y) { return __builtin_elementwise_maximum(x, y); }
  __device__ static double combine(double x, double y) { return __builtin_elementwise_maximum(x, y); }
  __device__ static int32_t combine(int32_t x, int32_t y) { return x > y ? x : y; }
  __device__ static int64_t combine(int64_t x, int64_t y) { return x > y ? x : y; }
  __device__ static uint8_t combine(uint8_t x, uint8_t y) { return x > y ? x : y; }
};
template <> __device__ inline float OpMax::identity<float>() { return -__builtin_inff(); }
template <> __device__ inline double OpMax::identity<double>() { return -__builtin_inf(); }
template <> __device__ inline int32_t OpMax::identity<int32_t>() { return INT32_MIN; }
template <> __device__ inline int64_t OpMax::identity<int64_t>() { return INT64_MIN; }
template <> __device__ inline uint8_t OpMax::identity<uint8_t>() { return 0; }

struct OpMin {
  template <class T> __device__ static T identity();
  __device__ static float combine(float x, float y) { return __builtin_elementwise_minimum(x, y); }
  __device__ static double combine(double x, double y) { return __builtin_elementwise_minimum(x, y); }
  __device__ static int32_t combine(int32_t x, int32_t y) { return x < y ? x : y; }
  __device__ static int64_t combine(int64_t x, int64_t y) { return x < y ? x : y; }
  __device__ static uint8_t combine(uint8_t x, uint8_t y) { return x < y ? x : y; }
};
template <> __device__ inline float OpMin::identity<float>() { return __builtin_inff(); }
template <> __device__ inline double OpMin::identity<double>() { return __builtin_inf(); }
template <> __device__ inline int32_t OpMin::identity<int32_t>() { return INT32_MAX; }
template <> __device__ inline int64_t OpMin::identity<int64_t>() { return INT64_MAX; }
template <> __device__ inline uint8_t OpMin::identity<uint8_t>() { return 255; }

// Julia `*`: IEEE products; integers wrap (computed unsigned); quaternions
// multiply by the Hamilton product, older operand on the left.
struct OpMul {
  template <class T> __device__ static T identity() {
    if constexpr (is_quat<T>)
      return T{1, 0, 0, 0};
    else
      return T(1);
  }
  // Each component is one product and three fused multiply-adds (the sign
  // of a term is a free source negation): 16 VALU operations per Hamilton
  // product instead of 28, and each component rounded at most four times.
  template <class F> __device__ static F fma_(F a, F b, F c) {
    if constexpr (__is_same(F, float))
      return __builtin_fmaf(a, b, c);
    else
      return __builtin_fma(a, b, c);
  }
  template <class F> __device__ static quat<F> combine(quat<F> p, quat<F> q) {
    quat<F> o;
    o.s = fma_(-p.v3, q.v3, fma_(-p.v2, q.v2, fma_(-p.v1, q.v1, p.s * q.s)));
    o.v1 = fma_(-p.v3, q.v2, fma_(p.v2, q.v3, fma_(p.v1, q.s, p.s * q.v1)));
    o.v2 = fma_(p.v3, q.v1, fma_(p.v2, q.s, fma_(-p.v1, q.v3, p.s * q.v2)));
    o.v3 = fma_(p.v3, q.s, fma_(-p.v2, q.v1, fma_(p.v1, q.v2, p.s * q.v3)));
    return o;
  }
  __device__ static float combine(float x, float y) { return x * y; }
  __device__ static double combine(double x, double y) { return x * y; }
  __device__ static int32_t combine(int32_t x, int32_t y) { return (int32_t)((uint32_t)x * (uint32_t)y); }
  __device__ static int64_t combine(int64_t x, int64_t y) { return (int64_t)((uint64_t)x * (uint64_t)y); }
  __device__ static uint8_t combine(uint8_t x, uint8_t y) { return (uint8_t)(x * y); }
};

// Composition of affine maps, older map on the left. Non-commutative: every
// combine site in the kernels keeps the older operand first.
struct OpAffine {
  template <class T> __device__ static T identity();
  __device__ static f32x2 combine(f32x2 l, f32x2 r) {
    f32x2 o;
    o.a = r.a * l.a;
    o.b = __builtin_fmaf(r.a, l.b, r.b);
    return o;
  }
};
template <> __device__ inline f32x2 OpAffine::identity<f32x2>() { return f32x2{1.0f, 0.0f}; }

// ---------------------------------------------------------------------------
// Element maps f (applied once per loaded element).
// ---------------------------------------------------------------------------
struct MapIdentity {
  template <class T> __device__ static T apply(T x) { return x; }
};
struct MapAbs2 {
  __device__ static float apply(float x) { return x * x; }
  __device__ static double apply(double x) { return x * x; }
  __device__ static int32_t apply(int32_t x) { return (int32_t)((uint32_t)x * (uint32_t)x); }
  __device__ static int64_t apply(int64_t x) { return (int64_t)((uint64_t)x * (uint64_t)x); }
  __device__ static uint8_t apply(uint8_t x) { return (uint8_t)(x * x); }
};

// ---------------------------------------------------------------------------
// Register-word view of a value: W 32-bit words (a uint8 occupies one word).
// ---------------------------------------------------------------------------
template <class T> struct Words {
  static constexpr int W = sizeof(T) >= 4 ? (int)(sizeof(T) / 4) : 1;
  uint32_t w[W];
};

template <class T> __device__ inline Words<T> to_words(T v) {
  Words<T> r;
  if constexpr (sizeof(T) >= 4) {
    __builtin_memcpy(r.w, &v, sizeof(T));
  } else {
    r.w[0] = (uint32_t)v;
  }
  return r;
}

template <class T> __device__ inline T from_words(const Words<T>& r) {
  T v;
  if constexpr (sizeof(T) >= 4) {
    __builtin_memcpy(&v, r.w, sizeof(T));
  } else {
    v = (T)r.w[0];
  }
  return v;
}

// v_mov_b32_dpp on every word. Lanes whose DPP source is invalid or whose row
// is masked off keep `old` (bound_ctrl = 0).
template <int CTRL, int ROW_MASK, class T>
__device__ inline T dpp_move(T old, T v) {
  Words<T> o = to_words(old), s = to_words(v), r;
#pragma unroll
  for (int i = 0; i < Words<T>::W; ++i)
    r.w[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)o.w[i], (int)s.w[i], CTRL, ROW_MASK, 0xf, false);
  return from_words<T>(r);
}

template <class T> __device__ inline T read_lane(T v, int lane) {
  Words<T> s = to_words(v), r;
#pragma unroll
  for (int i = 0; i < Words<T>::W; ++i) r.w[i] = (uint32_t)__builtin_amdgcn_readlane((int)s.w[i], lane);
  return from_words<T>(r);
}

// DPP control codes (GFX9 encoding).
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143, kWaveShr1 = 0x138;

// Inclusive wave64 scan in lane order (lane 0 is the oldest element).
// Hillis-Steele within 16-lane rows, then the two row broadcasts; every step
// combines (lower lanes) o (own value), so it is valid for non-commutative ops.
template <class Op, class T> __device__ inline T wave_inclusive_scan(T x) {
  const T id = Op::template identity<T>();
  x = Op::combine(dpp_move<kRowShr1, 0xf>(id, x), x);
  x = Op::combine(dpp_move<kRowShr2, 0xf>(id, x), x);
  x = Op::combine(dpp_move<kRowShr4, 0xf>(id, x), x);
  x = Op::combine(dpp_move<kRowShr8, 0xf>(id, x), x);
  x = Op::combine(dpp_move<kRowBcast15, 0xa>(id, x), x);
  x = Op::combine(dpp_move<kRowBcast31, 0xc>(id, x), x);
  return x;
}

// Exclusive value for each lane given the inclusive scan (identity in lane 0).
template <class Op, class T> __device__ inline T wave_shift_right(T incl) {
  return dpp_move<kWaveShr1, 0xf>(Op::template identity<T>(), incl);
}

// Wave-wide reduction in lane order, result broadcast to all lanes.
template <class Op, class T> __device__ inline T wave_reduce(T x) {
  return read_lane(wave_inclusive_scan<Op>(x), kWave - 1);
}

__device__ inline int lane_id() { return (int)__lane_id(); }

// Device-scope (agent) relaxed 64-bit atomics: single-copy atomic and coherent
// across the 8 XCD L2s.
__device__ inline uint64_t ld_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Give-up report: a kernel that stopped waiting on its scratch buffer (a
// scan lookback or a reduction fold past its poll budget) stores 1 into the
// library's host-mapped report word, which every later entry point reads
// on the host without synchronising (kf_async_status). Null: no report.
__device__ inline void report_giveup(uint32_t* mbox) {
  if (mbox) __hip_atomic_store(mbox, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// 16-byte streaming accesses.
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld_stream(const uint4* p) {
  const v4u32 v = __builtin_nontemporal_load(reinterpret_cast<const v4u32*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ inline void st_stream(uint4* p, uint4 v) {
  const v4u32 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<v4u32*>(p));
}

// Type tag mapping (host enum -> C++ type) -------------------------------------
template <kf_dtype D> struct DT;
template <> struct DT<KF_F32> { using T = float; };
template <> struct DT<KF_F64> { using T = double; };
template <> struct DT<KF_I32> { using T = int32_t; };
template <> struct DT<KF_I64> { using T = int64_t; };
template <> struct DT<KF_U8> { using T = uint8_t; };
template <> struct DT<KF_F32X2> { using T = f32x2; };
template <> struct DT<KF_Q32> { using T = q32; };
template <> struct DT<KF_Q64> { using T = q64; };

}  // namespace kf

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by the entry points (defined in kf_api.hip).
// ---------------------------------------------------------------------------
int kf_set_error(int code, const char* fmt, ...);
int kf_check_launch(const char* what);
size_t kf_dtype_size(kf_dtype dt);
int kf_validate_op(kf_op op, kf_map f, kf_dtype dt, int allow_affine);
int kf_device_cu_count();
// Host-mapped give-up report word (allocated on first use outside stream
// capture; null if that failed or the stream is capturing). kf_mailbox_peek
// never allocates (for kf_reduce_noalloc).
uint32_t* kf_mailbox(hipStream_t stream);
uint32_t* kf_mailbox_peek();
// KF_EGIVEUP (and clears the report) if a kernel queued by an earlier call
// has given up since the last report; KF_OK otherwise. Non-blocking.
int kf_take_giveup(const char* who);
