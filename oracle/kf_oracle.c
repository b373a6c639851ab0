/*
 * kf_oracle.c — CPU restatement of KernelForge.jl's scan / mapreduce
 * semantics. TEST INFRASTRUCTURE ONLY: used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, as the checker
 * and as the timed CPU baseline. Nothing in the product links it.
 *
 * Two families of functions:
 *
 *  (1) Checkers (kfo_*): the reference's results as its own tests define
 *      them — Julia Base `accumulate(op, x)` for scan!
 *      (reference test/tests/scan/scan_test.jl:10,54,81,99,119) and Base
 *      `mapreduce` / `sum` for mapreduce
 *      (test/tests/mapreduce/mapreduce1d_test.jl:20-29,
 *      test/tests/mapreduce/mapreduce2d_test.jl:8-35). Float inputs are
 *      accumulated in double (the Float64 host accumulation the tolerance
 *      is stated against); integer inputs are computed exactly in their own
 *      width with wrap-around, which is Julia's Int32/Int64/UInt8 `+`.
 *      The in-thread left fold follows src/helpers.jl:170-174
 *      (a_i = op(a_{i-1}, v_i)); prefixes compose as op(older, newer)
 *      (src/scan/scan_kernel.jl:1-7, :396-412).
 *
 *  (2) CPU baseline (kfb_*): the same operations in the element's own
 *      arithmetic (what Base.accumulate! / Base.mapreduce compute on the
 *      host), single-threaded and OpenMP-chunked, for the bench's
 *      cpu_baseline figure.
 *
 * Codes: dtype 0 f32, 1 f64, 2 i32, 3 i64, 4 u8, 5 (a,b) f32 pairs;
 *        op 0 +, 1 max, 2 min, 3 affine, 4 * (Julia `*`: IEEE product,
 *        integers wrap); map 0 identity, 1 abs2.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { D_F32 = 0, D_F64 = 1, D_I32 = 2, D_I64 = 3, D_U8 = 4, D_F32X2 = 5 };
enum { OP_ADD = 0, OP_MAX = 1, OP_MIN = 2, OP_AFFINE = 3, OP_MUL = 4 };

/* Julia `max`/`min` on IEEE floats: NaN-propagating, -0.0 < +0.0. */
static double jl_max(double x, double y) {
  if (isnan(x) || isnan(y)) return NAN;
  if (x == y) return signbit(x) ? y : x;
  return x > y ? x : y;
}
static double jl_min(double x, double y) {
  if (isnan(x) || isnan(y)) return NAN;
  if (x == y) return signbit(x) ? x : y;
  return x < y ? x : y;
}

static double fop(int op, double x, double y) {
  switch (op) {
    case OP_ADD: return x + y;
    case OP_MAX: return jl_max(x, y);
    case OP_MUL: return x * y;
    default: return jl_min(x, y);
  }
}

static double fload(const void* p, int dt, int64_t i, int map) {
  double v = dt == D_F32 ? (double)((const float*)p)[i] : ((const double*)p)[i];
  return map ? v * v : v;
}

/* Integers are carried as uint64 and truncated to the element width after
 * every operation (wrap-around); max/min compare in the signed (or, for u8,
 * unsigned) domain of the element type. */
static uint64_t wrap(int dt, uint64_t v) {
  switch (dt) {
    case D_I32: return (uint64_t)(int64_t)(int32_t)(uint32_t)v;
    case D_U8: return v & 0xffu;
    default: return v;
  }
}
static uint64_t iload(const void* p, int dt, int64_t i, int map) {
  uint64_t v;
  switch (dt) {
    case D_I32: v = (uint64_t)(int64_t)((const int32_t*)p)[i]; break;
    case D_I64: v = (uint64_t)((const int64_t*)p)[i]; break;
    default: v = ((const uint8_t*)p)[i]; break;
  }
  if (map) v = wrap(dt, v * v);
  return v;
}
static uint64_t iop(int dt, int op, uint64_t x, uint64_t y) {
  if (op == OP_ADD) return wrap(dt, x + y);
  if (op == OP_MUL) return wrap(dt, x * y);
  if (dt == D_U8) {
    if (op == OP_MAX) return x > y ? x : y;
    return x < y ? x : y;
  }
  if (op == OP_MAX) return (int64_t)x > (int64_t)y ? x : y;
  return (int64_t)x < (int64_t)y ? x : y;
}
static uint64_t iidentity(int dt, int op) {
  if (op == OP_ADD) return 0;
  if (op == OP_MUL) return 1;
  if (dt == D_U8) return op == OP_MAX ? 0 : 255;
  if (dt == D_I32) return op == OP_MAX ? (uint64_t)(int64_t)INT32_MIN : (uint64_t)(int64_t)INT32_MAX;
  return op == OP_MAX ? (uint64_t)INT64_MIN : (uint64_t)INT64_MAX;
}
static void istore(void* p, int dt, int64_t i, uint64_t v) {
  switch (dt) {
    case D_I32: ((int32_t*)p)[i] = (int32_t)(uint32_t)v; break;
    case D_I64: ((int64_t*)p)[i] = (int64_t)v; break;
    default: ((uint8_t*)p)[i] = (uint8_t)v; break;
  }
}

/* ---------------------------------------------------------------- scan ---- */

/* Float scan, double accumulation. Exclusive: out[0] = identity (+0.0 for
 * +, -Inf for max, +Inf for min, 1 for *), out[i] = inclusive[i-1]. */
void kfo_scan_f(const void* src, int dt, int64_t n, int64_t stride, int op, int map, int excl, double* out) {
  double acc = 0.0;
  const double id = op == OP_ADD ? 0.0 : op == OP_MUL ? 1.0 : (op == OP_MAX ? -INFINITY : INFINITY);
  for (int64_t i = 0; i < n; ++i) {
    const double v = fload(src, dt, i * stride, map);
    const double prev = i == 0 ? id : acc;
    acc = i == 0 ? v : fop(op, acc, v);
    out[i] = excl ? prev : acc;
  }
}

/* Integer scan, exact, result in the element type. */
void kfo_scan_i(const void* src, int dt, int64_t n, int64_t stride, int op, int map, int excl, void* out) {
  uint64_t acc = 0;
  const uint64_t id = iidentity(dt, op);
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t v = iload(src, dt, i * stride, map);
    const uint64_t prev = i == 0 ? id : acc;
    acc = i == 0 ? v : iop(dt, op, acc, v);
    istore(out, dt, i, excl ? prev : acc);
  }
}

/* Affine-composition scan of (a, b) float pairs in double:
 * (a1,b1) o (a2,b2) = (a2*a1, a2*b1 + b2). The b-component of the inclusive
 * result is the recurrence x_t = a_t x_{t-1} + b_t with x_0 = 0, the
 * a-component the running product. Exclusive: out[0] = (1, 0). */
void kfo_scan_affine(const float* ab, int64_t n, int excl, double* out) {
  double A = 1.0, B = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double a = ab[2 * i], b = ab[2 * i + 1];
    if (excl) {
      out[2 * i] = A;
      out[2 * i + 1] = B;
    }
    const double nA = a * A, nB = a * B + b;
    A = nA;
    B = nB;
    if (!excl) {
      out[2 * i] = A;
      out[2 * i + 1] = B;
    }
  }
}

/* Quaternion product scan in double: q[4*i .. 4*i+3] = (s, v1, v2, v3) as
 * float (f64 == 0) or double (f64 == 1); prefixes multiply older on the
 * left (Base.accumulate(*, x) on Quaternions.jl values, reference
 * test/tests/scan/scan_test.jl:22-33), by the Hamilton product
 * (s1 + v1 i + ...)(s2 + w1 i + ...) with i^2 = j^2 = k^2 = ijk = -1.
 * Exclusive: out[0] = (1, 0, 0, 0). */
void kfo_scan_quat(const void* q, int f64, int64_t n, int excl, double* out) {
  double p[4] = {1.0, 0.0, 0.0, 0.0};
  for (int64_t i = 0; i < n; ++i) {
    double x[4];
    for (int c = 0; c < 4; ++c) x[c] = f64 ? ((const double*)q)[4 * i + c] : (double)((const float*)q)[4 * i + c];
    if (excl)
      for (int c = 0; c < 4; ++c) out[4 * i + c] = p[c];
    const double s = p[0] * x[0] - p[1] * x[1] - p[2] * x[2] - p[3] * x[3];
    const double a = p[0] * x[1] + p[1] * x[0] + p[2] * x[3] - p[3] * x[2];
    const double b = p[0] * x[2] - p[1] * x[3] + p[2] * x[0] + p[3] * x[1];
    const double c = p[0] * x[3] + p[1] * x[2] - p[2] * x[1] + p[3] * x[0];
    p[0] = s;
    p[1] = a;
    p[2] = b;
    p[3] = c;
    if (!excl)
      for (int k = 0; k < 4; ++k) out[4 * i + k] = p[k];
  }
}

/* -------------------------------------------------------------- reduce ---- */

double kfo_reduce_f(const void* src, int dt, int64_t n, int64_t stride, int op, int map) {
  double acc = fload(src, dt, 0, map);
  for (int64_t i = 1; i < n; ++i) acc = fop(op, acc, fload(src, dt, i * stride, map));
  return acc;
}

/* Also writes the element-typed result to *out (an int32/int64/uint8). */
void kfo_reduce_i(const void* src, int dt, int64_t n, int64_t stride, int op, int map, void* out) {
  uint64_t acc = iload(src, dt, 0, map);
  for (int64_t i = 1; i < n; ++i) acc = iop(dt, op, acc, iload(src, dt, i * stride, map));
  istore(out, dt, 0, acc);
}

/* Two-array maps: f2 = 0 -> x*y, 1 -> (x-y)^2, 2 -> x*y*y, 3 -> exp(x-y). */
static double fmap2(int f2, double a, double b) {
  switch (f2) {
    case 0: return a * b;
    case 1: return (a - b) * (a - b);
    case 2: return a * b * b;
    default: return exp(a - b);
  }
}

/* Two-array reduction op_i f2(x[i], y[i]) (the reference's
 * mapreduce(f, op, (x, y)), src/mapreduce/1D/mapreduce1d.jl:186-204). */
double kfo_reduce2_f(const void* x, const void* y, int dt, int64_t n, int op, int f2) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double a = fload(x, dt, i, 0), b = fload(y, dt, i, 0);
    const double v = fmap2(f2, a, b);
    acc = i == 0 ? v : fop(op, acc, v);
  }
  return acc;
}

void kfo_reduce2_i(const void* x, const void* y, int dt, int64_t n, int op, int f2, void* out) {
  uint64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t a = iload(x, dt, i, 0), b = iload(y, dt, i, 0);
    uint64_t v;
    if (f2 == 1) {
      const uint64_t d = wrap(dt, a - b);
      v = wrap(dt, d * d);
    } else if (f2 == 2) {
      v = wrap(dt, wrap(dt, a * b) * b);
    } else {
      v = wrap(dt, a * b);
    }
    acc = i == 0 ? v : iop(dt, op, acc, v);
  }
  istore(out, dt, 0, acc);
}

/* Three-array reduction op_i x[i]*y[i]*z[i] (the reference's
 * mapreduce1d(f, op, (a, b, c)), src/mapreduce/1D/mapreduce1d.jl:186-204,
 * tested with f = a*b*c, test/tests/mapreduce/mapreduce1d_test.jl:180-194). */
double kfo_reduce3_f(const void* x, const void* y, const void* z, int dt, int64_t n, int op) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double v = fload(x, dt, i, 0) * fload(y, dt, i, 0) * fload(z, dt, i, 0);
    acc = i == 0 ? v : fop(op, acc, v);
  }
  return acc;
}

void kfo_reduce3_i(const void* x, const void* y, const void* z, int dt, int64_t n, int op, void* out) {
  uint64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t v = wrap(dt, wrap(dt, iload(x, dt, i, 0) * iload(y, dt, i, 0)) * iload(z, dt, i, 0));
    acc = i == 0 ? v : iop(dt, op, acc, v);
  }
  istore(out, dt, 0, acc);
}

/* matvec (dim 2): out[i] = op_j f(A[i,j], x[j]); vecmat (dim 1):
 * out[j] = op_i f(x[i], A[i,j]); f2 = 0 -> product, 1 -> squared difference
 * (reference src/mapreduce/2D/matvec.jl:393-474, vecmat.jl:328-405). */
void kfo_reduce_dim_x_f(const void* A, const void* x, int dt, int64_t rows, int64_t cols, int64_t cs, int dim,
                        int op, int f2, double* out) {
  const int64_t m = dim == 2 ? rows : cols, k = dim == 2 ? cols : rows;
  for (int64_t o = 0; o < m; ++o) {
    double acc = 0.0;
    for (int64_t q = 0; q < k; ++q) {
      const int64_t i = dim == 2 ? o : q, j = dim == 2 ? q : o;
      const double a = fload(A, dt, i + j * cs, 0), b = fload(x, dt, q, 0);
      const double v = f2 ? (a - b) * (a - b) : a * b;
      acc = q == 0 ? v : fop(op, acc, v);
    }
    out[o] = acc;
  }
}

void kfo_reduce_dim_x_i(const void* A, const void* x, int dt, int64_t rows, int64_t cols, int64_t cs, int dim,
                        int op, int f2, void* out) {
  const int64_t m = dim == 2 ? rows : cols, k = dim == 2 ? cols : rows;
  for (int64_t o = 0; o < m; ++o) {
    uint64_t acc = 0;
    for (int64_t q = 0; q < k; ++q) {
      const int64_t i = dim == 2 ? o : q, j = dim == 2 ? q : o;
      const uint64_t a = iload(A, dt, i + j * cs, 0), b = iload(x, dt, q, 0);
      uint64_t v;
      if (f2) {
        const uint64_t d = wrap(dt, a - b);
        v = wrap(dt, d * d);
      } else {
        v = wrap(dt, a * b);
      }
      acc = q == 0 ? v : iop(dt, op, acc, v);
    }
    istore(out, dt, o, acc);
  }
}

/* Column-major A[i, j] = A[i + j*col_stride]. dim 1 -> cols outputs, dim 2
 * -> rows outputs (reference src/mapreduce/2D/mapreduce2d.jl:49-64). */
void kfo_reduce_dim_f(const void* A, int dt, int64_t rows, int64_t cols, int64_t col_stride, int dim, int op,
                      int map, double* out) {
  if (dim == 1) {
    for (int64_t j = 0; j < cols; ++j) {
      double acc = fload(A, dt, j * col_stride, map);
      for (int64_t i = 1; i < rows; ++i) acc = fop(op, acc, fload(A, dt, i + j * col_stride, map));
      out[j] = acc;
    }
  } else {
    for (int64_t i = 0; i < rows; ++i) out[i] = fload(A, dt, i, map);
    for (int64_t j = 1; j < cols; ++j)
      for (int64_t i = 0; i < rows; ++i) out[i] = fop(op, out[i], fload(A, dt, i + j * col_stride, map));
  }
}

void kfo_reduce_dim_i(const void* A, int dt, int64_t rows, int64_t cols, int64_t col_stride, int dim, int op,
                      int map, void* out) {
  if (dim == 1) {
    for (int64_t j = 0; j < cols; ++j) {
      uint64_t acc = iload(A, dt, j * col_stride, map);
      for (int64_t i = 1; i < rows; ++i) acc = iop(dt, op, acc, iload(A, dt, i + j * col_stride, map));
      istore(out, dt, j, acc);
    }
  } else {
    for (int64_t i = 0; i < rows; ++i) {
      uint64_t acc = iload(A, dt, i, map);
      for (int64_t j = 1; j < cols; ++j) acc = iop(dt, op, acc, iload(A, dt, i + j * col_stride, map));
      istore(out, dt, i, acc);
    }
  }
}

/* ------------------------------------------------------- CPU baseline ---- */
/* Compiled at -O3 so that the independent partial sums vectorise, as Base's
 * @simd blocks do. */
#pragma GCC push_options
#pragma GCC optimize("O3")

/* Base.accumulate!(+, dst, src) on Float32: sequential, Float32 arithmetic. */
void kfb_scan_add_f32_seq(const float* x, float* y, int64_t n) {
  float acc = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    acc = i == 0 ? x[0] : acc + x[i];
    y[i] = acc;
  }
}

/* Two-pass chunked scan on `threads` threads (per-chunk totals, exclusive
 * scan of the totals, then a re-scan with the chunk offset). */
void kfb_scan_add_f32_par(const float* x, float* y, int64_t n, int threads) {
#ifdef _OPENMP
  if (threads < 1) threads = 1;
  float totals[1024];
  if (threads > 1024) threads = 1024;
  const int64_t chunk = (n + threads - 1) / threads;
#pragma omp parallel num_threads(threads)
  {
    const int t = omp_get_thread_num();
    const int64_t lo = t * chunk, hi = lo + chunk < n ? lo + chunk : n;
    float s = 0.0f;
    for (int64_t i = lo; i < hi; ++i) s += x[i];
    totals[t] = s;
#pragma omp barrier
    float off = 0.0f;
    for (int k = 0; k < t; ++k) off += totals[k];
    float acc = off;
    for (int64_t i = lo; i < hi; ++i) {
      acc += x[i];
      y[i] = acc;
    }
  }
#else
  (void)threads;
  kfb_scan_add_f32_seq(x, y, n);
#endif
}

/* Base.mapreduce(identity, +, x) on Float32 (single thread, Float32
 * arithmetic, 8 independent partial sums like Base's pairwise blocks). */
float kfb_sum_f32_seq(const float* x, int64_t n) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int k = 0; k < 8; ++k) s[k] += x[i + k];
  for (; i < n; ++i) s[0] += x[i];
  float r = 0.0f;
  for (int k = 0; k < 8; ++k) r += s[k];
  return r;
}

float kfb_sum_f32_par(const float* x, int64_t n, int threads) {
  double total = 0.0;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
  const int64_t chunk = (n + threads - 1) / threads;
#pragma omp parallel num_threads(threads) reduction(+ : total)
  {
    const int t = omp_get_thread_num();
    const int64_t lo = t * chunk, hi = lo + chunk < n ? lo + chunk : n;
    if (hi > lo) total += kfb_sum_f32_seq(x + lo, hi - lo);
  }
#else
  (void)threads;
  total = kfb_sum_f32_seq(x, n);
#endif
  return (float)total;
}

/* ---- CPU baseline of every BASELINE configuration -----------------------
 * Each function runs on `threads` host threads (<= 1: the sequential left
 * fold Base.accumulate! / Base.mapreduce computes; > 1: the chunked
 * Threads.@threads variant: per-chunk folds, then for scans an ordered
 * combine of the chunk totals and a second pass that re-scans each chunk
 * from its prefix). Element arithmetic throughout (Int32 wraps, Float32 and
 * Float64 stay in their width); sums keep 8 independent partials per
 * thread, as Base's vectorised blocks do. */
static int clamp_threads(int threads) { return threads < 1 ? 1 : threads > 1024 ? 1024 : threads; }

/* Base.accumulate!(+, dst, src) on Int32 (wrap-around); exclusive shifts
 * by one with 0 first. */
static void scan_i32_range(const int32_t* x, int32_t* y, int64_t lo, int64_t hi, uint32_t acc, int exclusive) {
  if (exclusive)
    for (int64_t i = lo; i < hi; ++i) {
      y[i] = (int32_t)acc;
      acc += (uint32_t)x[i];
    }
  else
    for (int64_t i = lo; i < hi; ++i) {
      acc += (uint32_t)x[i];
      y[i] = (int32_t)acc;
    }
}

void kfb_scan_add_i32(const int32_t* x, int32_t* y, int64_t n, int exclusive, int threads) {
  threads = clamp_threads(threads);
  if (threads == 1) {
    scan_i32_range(x, y, 0, n, 0u, exclusive);
    return;
  }
  uint32_t totals[1024];
  const int64_t chunk = (n + threads - 1) / threads;
#pragma omp parallel num_threads(threads)
  {
    const int t = omp_get_thread_num();
    const int64_t lo = t * chunk < n ? t * chunk : n, hi = lo + chunk < n ? lo + chunk : n;
    uint32_t s = 0;
    for (int64_t i = lo; i < hi; ++i) s += (uint32_t)x[i];
    totals[t] = s;
#pragma omp barrier
    uint32_t off = 0;
    for (int k = 0; k < t; ++k) off += totals[k];
    scan_i32_range(x, y, lo, hi, off, exclusive);
  }
}

/* The affine recurrence's scan on interleaved Float32 pairs: (A, B) <-
 * (a*A, a*B + b), inclusive, in Float32. */
static void affine_range(const float* ab, float* out, int64_t lo, int64_t hi, float A, float B) {
  for (int64_t i = lo; i < hi; ++i) {
    const float a = ab[2 * i], b = ab[2 * i + 1];
    A = a * A;
    B = a * B + b;
    out[2 * i] = A;
    out[2 * i + 1] = B;
  }
}

void kfb_scan_affine_f32(const float* ab, float* out, int64_t n, int threads) {
  threads = clamp_threads(threads);
  if (threads == 1 || n < 2) {
    if (n > 0) {
      out[0] = ab[0];
      out[1] = ab[1];
      affine_range(ab, out, 1, n, ab[0], ab[1]);
    }
    return;
  }
  float tA[1024], tB[1024];
  const int64_t chunk = (n + threads - 1) / threads;
#pragma omp parallel num_threads(threads)
  {
    const int t = omp_get_thread_num();
    const int64_t lo = t * chunk < n ? t * chunk : n, hi = lo + chunk < n ? lo + chunk : n;
    float A = 1.0f, B = 0.0f;  /* the chunk's composition, older first */
    for (int64_t i = lo; i < hi; ++i) {
      const float a = ab[2 * i], b = ab[2 * i + 1];
      A = a * A;
      B = a * B + b;
    }
    tA[t] = A;
    tB[t] = B;
#pragma omp barrier
    float pA = 1.0f, pB = 0.0f;
    for (int k = 0; k < t; ++k) {
      pA = tA[k] * pA;
      pB = tA[k] * pB + tB[k];
    }
    affine_range(ab, out, lo, hi, pA, pB);
  }
}

#define KFB_FOLD8(T, NAME, INIT, STEP, JOIN)                                        \
  static T NAME##_seq(const T* x, int64_t n) {                                      \
    T s[8];                                                                         \
    for (int k = 0; k < 8; ++k) s[k] = INIT;                                        \
    int64_t i = 0;                                                                  \
    for (; i + 8 <= n; i += 8)                                                      \
      for (int k = 0; k < 8; ++k) s[k] = STEP(s[k], x[i + k]);                      \
    for (; i < n; ++i) s[0] = STEP(s[0], x[i]);                                     \
    T r = s[0];                                                                     \
    for (int k = 1; k < 8; ++k) r = JOIN(r, s[k]);                                  \
    return r;                                                                       \
  }                                                                                 \
  T NAME(const T* x, int64_t n, int threads) {                                      \
    threads = clamp_threads(threads);                                               \
    if (threads == 1) return NAME##_seq(x, n);                                      \
    T part[1024];                                                                   \
    const int64_t chunk = (n + threads - 1) / threads;                              \
    _Pragma("omp parallel num_threads(threads)") {                                  \
      const int t = omp_get_thread_num();                                           \
      const int64_t lo = t * chunk < n ? t * chunk : n;                             \
      const int64_t hi = lo + chunk < n ? lo + chunk : n;                           \
      part[t] = NAME##_seq(x + lo, hi - lo);                                        \
    }                                                                               \
    T r = part[0];                                                                  \
    for (int k = 1; k < threads; ++k) r = JOIN(r, part[k]);                         \
    return r;                                                                       \
  }

#define KFB_ADD(a, b) ((a) + (b))
#define KFB_ADDSQ(a, v) ((a) + (v) * (v))
#define KFB_MAX(a, b) ((a) > (b) ? (a) : (b))
/* Base.mapreduce(abs2, +, x) on Float32 / Float64 and maximum(x) on Int32 */
KFB_FOLD8(float, kfb_sum_abs2_f32, 0.0f, KFB_ADDSQ, KFB_ADD)
KFB_FOLD8(double, kfb_sum_abs2_f64, 0.0, KFB_ADDSQ, KFB_ADD)
KFB_FOLD8(int32_t, kfb_max_i32, INT32_MIN, KFB_MAX, KFB_MAX)

/* Base.mapreduce(identity, +, A; dims) on a column-major Float32 matrix
 * A[i, j] = A[i + j*cs]: dims=1 sums each column (columns split across
 * threads), dims=2 adds the columns into the row sums (rows split across
 * threads, each thread walking every column over its rows). */
void kfb_sum_dims_f32(const float* A, int64_t rows, int64_t cols, int64_t cs, int dim, float* out, int threads) {
  threads = clamp_threads(threads);
  if (dim == 1) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t j = 0; j < cols; ++j) {
      const float* c = A + j * cs;
      float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      int64_t i = 0;
      for (; i + 8 <= rows; i += 8)
        for (int k = 0; k < 8; ++k) s[k] += c[i + k];
      for (; i < rows; ++i) s[0] += c[i];
      float r = s[0];
      for (int k = 1; k < 8; ++k) r += s[k];
      out[j] = r;
    }
    return;
  }
  const int64_t chunk = (rows + threads - 1) / threads;
#pragma omp parallel num_threads(threads)
  {
    const int t = omp_get_thread_num();
    const int64_t lo = t * chunk < rows ? t * chunk : rows, hi = lo + chunk < rows ? lo + chunk : rows;
    for (int64_t i = lo; i < hi; ++i) out[i] = A[i];
    for (int64_t j = 1; j < cols; ++j) {
      const float* c = A + j * cs;
      for (int64_t i = lo; i < hi; ++i) out[i] += c[i];
    }
  }
}
#pragma GCC pop_options

int kfo_omp_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
