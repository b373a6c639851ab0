/*
 * kf.h — C ABI of libkfhip.so, the gfx950 (MI355X) implementation of
 * KernelForge.jl's scan / mapreduce hot path.
 *
 * Every entry point takes plain device pointers, element counts and strides
 * (in elements), and a hipStream_t (passed as void*; NULL = default stream).
 * Calls are stream-ordered and non-blocking; the library never allocates
 * device memory (its one allocation is a 256-byte pinned host word for
 * give-up reports, see kf_async_status) and never synchronises. Scratch memory is caller-owned:
 * size it with the matching *_scratch_bytes query and zero-fill it ONCE
 * before its first use (kf_scratch_reset does that on a stream). After that
 * the kernels keep it valid themselves (epoch-tagged tile descriptors and
 * epoch-tagged reduction fold slots), so one scratch buffer may be reused across calls,
 * dtypes, operators and sizes without clearing. A buffer serves one family:
 * scan calls (kf_scan), or reduction calls (kf_reduce, kf_reduce2, kf_reduce3,
 * kf_reduce_dim*). Reduction partials written over scan descriptors could
 * read as current ones, so never share one buffer between the two.
 * Calls that share a scratch buffer must be ordered on one stream;
 * concurrent calls need distinct buffers.
 *
 * Return codes: KF_OK, KF_EINVAL (bad enum, shape, stride or alignment),
 * KF_ENOSCRATCH (scratch missing or too small), KF_EHIP (a HIP error; the
 * text is in kf_last_error()), KF_EGIVEUP (an earlier call's kernel gave
 * up waiting on its scratch buffer: see kf_async_status; the call that
 * returns it queued nothing). n == 0 is a successful no-op.
 *
 * Semantics follow Julia Base, as the reference's tests require
 * (reference test/tests/scan/scan_test.jl:1-125 compares against
 * `accumulate`, the test/tests/mapreduce files against `mapreduce`/`sum`).
 */
#ifndef KF_H
#define KF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_VERSION 100 /* 1.0.0 */

typedef enum {
  KF_OK = 0,
  KF_EINVAL = 1,
  KF_ENOSCRATCH = 2,
  KF_EHIP = 3,
  KF_EGIVEUP = 4
} kf_status;

/* Binary operator `op` of scan!/mapreduce. KF_OP_AFFINE is the
 * non-commutative composition (a1,b1) o (a2,b2) = (a2*a1, a2*b1 + b2) on
 * KF_F32X2 pairs; it is accepted by kf_scan only. KF_OP_MUL is Julia `*`
 * (IEEE product for floats, wrap-around for integers), the operator of the
 * reference's product-scan tests (test/tests/scan/scan_test.jl:1-19). */
typedef enum {
  KF_OP_ADD = 0,
  KF_OP_MAX = 1,
  KF_OP_MIN = 2,
  KF_OP_AFFINE = 3,
  KF_OP_MUL = 4
} kf_op;

/* Element map `f` (applied to each element before `op`). */
typedef enum {
  KF_MAP_IDENTITY = 0,
  KF_MAP_ABS2 = 1
} kf_map;

/* Post-map `g` applied to results (the reference's `g` keyword). */
typedef enum {
  KF_POST_IDENTITY = 0,
  KF_POST_SQRT = 1,   /* floating-point types only */
  KF_POST_ABS2 = 2
} kf_post;

/* Two-argument element map of kf_reduce2: f(x, y). */
typedef enum {
  KF_MAP2_MUL = 0,     /* x * y       (dot product)       */
  KF_MAP2_SQDIFF = 1,  /* (x - y)^2   (squared distance)  */
  KF_MAP2_WSQ = 2,     /* x * y * y   (weighted sum of squares; kf_reduce2 only) */
  KF_MAP2_EXPDIFF = 3  /* exp(x - y)  (floating-point types; kf_reduce2 only)    */
} kf_map2;

/* Three-argument element map of kf_reduce3: f(x, y, z). */
typedef enum {
  KF_MAP3_MUL = 0     /* x * y * z */
} kf_map3;

/* Element types. KF_F32X2 is an interleaved (a, b) pair of float32.
 * KF_Q32 / KF_Q64 are quaternions (s, v1, v2, v3) of float32 / float64, the
 * memory layout of Julia's QuaternionF32 / QuaternionF64 (Quaternions.jl,
 * used by the reference's non-commutative scan test,
 * test/tests/scan/scan_test.jl:22-33); they take KF_OP_MUL (the Hamilton
 * product) in kf_scan only. */
typedef enum {
  KF_F32 = 0,
  KF_F64 = 1,
  KF_I32 = 2,
  KF_I64 = 3,
  KF_U8 = 4,
  KF_F32X2 = 5,
  KF_Q32 = 6,
  KF_Q64 = 7
} kf_dtype;

int kf_version(void);

/* Text of the last error raised on the calling host thread ("" if none). */
const char* kf_last_error(void);

/* Zero-fill `bytes` of scratch on `stream` with a fill kernel (no memset
 * node, so it is safe inside captured graphs). */
int kf_scratch_reset(void* scratch, size_t bytes, void* stream);

/* Give-up reports (no counterpart in the reference, whose kernels spin
 * without bound). The scan's lookback and the reduction's fold wait on
 * other workgroups through the scratch buffer; only out-of-order dispatch,
 * a corrupted buffer or overlapping calls on one buffer can keep them
 * waiting, and then they stop after a poll budget instead of hanging the
 * GPU. A kernel that stops stores nothing as a result and raises a flag in
 * its scratch header (kf_scan_scratch_status / kf_reduce_scratch_status)
 * and in a pinned, host-mapped report word of the library. The report
 * surfaces without any synchronisation: the next compute entry point
 * (kf_scan*, kf_reduce*) called after the failed kernel has finished
 * returns KF_EGIVEUP without queuing anything and clears the report, and
 * kf_async_status reads and clears it (after a stream synchronisation it
 * covers every kernel queued before it). Like the asynchronous errors of
 * HIP itself, the report belongs to the process, not to one buffer or
 * stream. The report word is allocated (pinned host memory, 256 bytes,
 * once per process) by kf_init or by the first call of any compute entry
 * point except kf_reduce_noalloc, which never allocates, and never while
 * the call's stream is being captured into a graph: kernels launched before
 * the word exists carry none. Call kf_init at set-up to have every kernel,
 * captured and kf_reduce_noalloc ones included, report. */
int kf_init(void);
int kf_async_status(int* gave_up);

/* ---------------------------------------------------------------- scan ----
 * dst[i] = g(f(src[0]) op ... op f(src[i]))           (exclusive = 0)
 * dst[0] = g(identity(op)); dst[i] = g(incl[i-1])      (exclusive = 1)
 * g (KF_POST_*) is applied to each stored value only, never to the running
 * prefix, as the reference's kernels do (scan_kernel.jl:284-295); sqrt
 * needs a floating-point type, the affine scan takes no g.
 * Strides are in elements (1 = contiguous). src and dst may alias only
 * exactly (in-place scan, same pointer and stride).
 *
 * Replaces the reference's
 *   scan!(f, op, dst, src; g, tmp, Nitem, workgroup, family, arch)
 *     src/scan/scan.jl:251-284 (host) -> _scan_impl! src/scan/scan.jl:414-479
 *     -> scan_kernel_packed! / scan_kernel! src/scan/scan_kernel.jl:94-478
 * and get_allocation(Scan1D, ...) src/scan/scan.jl:156-211 (scratch size).
 * The exclusive variant has no reference counterpart (CUB/rocPRIM
 * ExclusiveSum semantics, used by the reference's vendor benchmarks
 * perfs/rocm_cpp/hipcub_hipcc/rocprim_scan_benchmark.cpp). */
size_t kf_scan_scratch_bytes(kf_dtype dt, kf_op op, int64_t n);

int kf_scan(kf_op op, kf_map f, kf_post g, kf_dtype dt, int exclusive,
            const void* src, int64_t src_stride,
            void* dst, int64_t dst_stride, int64_t n,
            void* scratch, size_t scratch_bytes, void* stream);

/* kf_scan with the reference's launch-shape keywords: `workgroup` threads
 * per workgroup and `nitem` elements per thread (reference
 * src/scan/scan.jl:261-284, where `Nitem` / `workgroup` override
 * default_nitem / default_workgroup; <= 0 means not given). The kernels are
 * compiled for a fixed set of tile shapes (1024 threads x 1, 2, 4 or 8
 * 16-byte vectors per thread, 768 x 8 for 4- and 8-byte elements, 512 x 1,
 * 2, 4, 8, 12 or 16 for UInt8; quaternions 1024 x 1, 2 or 4 units
 * (QuaternionF64: 1 or 2) and 768 x 8 (QuaternionF32) or 1024 x 8
 * (QuaternionF64)), so a request takes the nearest shape: the smallest
 * |log2(threads / workgroup)| + |log2(elements per thread / nitem)|, a
 * keyword not given standing for the size-based default shape's value;
 * ties go to the default shape, then to the smaller tile. kf_scan_shape
 * reports the shape chosen; the scratch size depends on it
 * (kf_scan_shaped_scratch_bytes, which replaces the reference's
 * get_allocation(Scan1D, f, op, src, workgroup, blocks) sizing,
 * src/scan/scan.jl:187-211). With both keywords <= 0 these are kf_scan and
 * kf_scan_scratch_bytes. Results do not depend on the shape for integer
 * elements; floating-point sums are regrouped. */
size_t kf_scan_shaped_scratch_bytes(kf_dtype dt, kf_op op, int64_t n, int workgroup, int nitem);

int kf_scan_shape(kf_dtype dt, int64_t n, int workgroup, int nitem, int* threads, int* items);

int kf_scan_shaped(kf_op op, kf_map f, kf_post g, kf_dtype dt, int exclusive,
                   const void* src, int64_t src_stride,
                   void* dst, int64_t dst_stride, int64_t n, int workgroup, int nitem,
                   void* scratch, size_t scratch_bytes, void* stream);

/* Diagnostics (no counterpart in the reference). KF_OK from kf_scan means
 * the launch was queued; it does not cover a lookback give-up. Tiles are
 * numbered by workgroup id, and a tile waits only on lower-numbered tiles,
 * which is deadlock-free because the GPU dispatches each XCD's workgroups
 * in increasing id order. Should a predecessor never publish (dispatch out
 * of that order, a corrupted scratch buffer, or overlapping calls on one
 * buffer), a tile stops after 2^24 lookback polls and raises the give-up
 * flag in the scratch header; every waiting tile of that grid then stops
 * too, no stopped tile stores, and the results are invalid. The flag is
 * sticky: until it is cleared, every later kf_scan on that scratch stores
 * nothing (dst untouched), and each such call is reported like the give-up
 * itself (kf_async_status). kf_scan_scratch_status synchronises `stream`,
 * sets *gave_up = 1 if the flag is raised and then clears it and moves the
 * buffer's epoch past every descriptor of the failed call, so the buffer is
 * valid again; kf_scratch_reset (a zero fill) also clears it. The status
 * queries leave the process-wide report alone (it may stand for another
 * buffer): read it with kf_async_status. */
int kf_scan_scratch_status(void* scratch, void* stream, int* gave_up);


/* -------------------------------------------------------------- reduce ----
 * dst[0] = f(src[0]) op f(src[stride]) op ... (n terms), written on device.
 * op must be commutative (ADD, MAX, MIN). The result is deterministic: the
 * combine tree depends only on n and the pointer alignment.
 *
 * Replaces the reference's mapreduce1d!(f, op, dst, src; tmp, ...)
 *   src/mapreduce/1D/mapreduce1d.jl:259-345 -> mapreduce1d_kernel!
 *   src/mapreduce/1D/mapreduce1d_kernel.jl:5-93, and
 * get_allocation(MapReduce1D, ...) src/mapreduce/1D/mapreduce1d.jl:140-170. */
size_t kf_reduce_scratch_bytes(kf_dtype dt, int64_t n);

int kf_reduce(kf_op op, kf_map f, kf_dtype dt,
              const void* src, int64_t n, int64_t stride,
              void* dst, void* scratch, size_t scratch_bytes, void* stream);

/* After a fold give-up (see kf_async_status) dst is left untouched and the
 * buffer is already valid for the next call (the fold's epoch skips past
 * every slot of the failed call). kf_reduce_scratch_status synchronises
 * `stream`, sets *gave_up = 1 if a call on this reduction scratch buffer
 * gave up since the last query, and clears that flag. No counterpart in the
 * reference (whose finisher, mapreduce1d_kernel.jl:58-92, spins unbounded). */
int kf_reduce_scratch_status(void* scratch, void* stream, int* gave_up);

/* ------------------------------------------------------------- reduce2 ----
 * dst[0] = f(x[0], y[0]) op ... op f(x[n-1], y[n-1]) (element strides xs, ys).
 * The two-array form of the reference's
 *   mapreduce(f, op, (x, y))  src/mapreduce/mapreduce.jl:228-239 ->
 *   mapreduce1d(f, op, srcs::NTuple)  src/mapreduce/1D/mapreduce1d.jl:186-204
 * for the maps x*y and (x-y)^2 (its tests' dot products and distances,
 * test/tests/mapreduce/mapreduce1d_test.jl:231-319), x*y*y and exp(x-y)
 * (its weighted sum of squares and sum(exp(a - b)), same file :117-131). */
size_t kf_reduce2_scratch_bytes(kf_dtype dt, int64_t n);

int kf_reduce2(kf_op op, kf_map2 f, kf_dtype dt,
               const void* x, int64_t x_stride, const void* y, int64_t y_stride, int64_t n,
               void* dst, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------- reduce3 ----
 * dst[0] = f(x[0], y[0], z[0]) op ... op f(x[n-1], y[n-1], z[n-1]) with
 * f = x*y*z: the three-array form of the same reference entry point
 *   mapreduce1d(f, op, srcs::NTuple)  src/mapreduce/1D/mapreduce1d.jl:186-204
 * (its test: sum(a .* b .* c), test/tests/mapreduce/mapreduce1d_test.jl:180-194).
 * Scratch as kf_reduce2. */
size_t kf_reduce3_scratch_bytes(kf_dtype dt, int64_t n);

int kf_reduce3(kf_op op, kf_map3 f, kf_dtype dt,
               const void* x, int64_t x_stride, const void* y, int64_t y_stride,
               const void* z, int64_t z_stride, int64_t n,
               void* dst, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------ reduce_noalloc ----
 * No counterpart in the reference: kf_reduce for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and result as
 * kf_reduce without the scratch pair: the partials live in a static device
 * array of KF_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.
 * Sizes whose kf_reduce_scratch_bytes exceeds it are refused with
 * KF_EINVAL (Float32 up to about 2^30 elements fits). The call allocates
 * nothing (its first call on a device looks the array's address up once).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams, or host threads, without ordering) race and give
 * wrong results; order them on one stream. */
#define KF_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

int kf_reduce_noalloc(kf_op op, kf_map f, kf_dtype dt,
                      const void* src, int64_t n, int64_t stride,
                      void* dst, void* stream);

/* ---------------------------------------------------------- reduce_dim ----
 * A is a column-major rows x cols matrix: A[i, j] at A + i + j*col_stride
 * (col_stride >= rows; col_stride = 2*rows is the view A[:, 1:2:end]).
 *   dim = 1: dst[j * dst_stride] = op_i f(A[i, j])   (cols outputs)
 *   dim = 2: dst[i * dst_stride] = op_j f(A[i, j])   (rows outputs)
 * op must be commutative (ADD, MAX, MIN).
 * Scratch holds split partials; whether a call splits depends on the shape
 * and on the alignment of A (and of x for vecmat), and the query returns the
 * largest need over every alignment, so one buffer of that size serves any
 * A of this shape. A call that does not split accepts a null scratch; one
 * that does is refused with KF_ENOSCRATCH before any launch.
 *
 * Replaces the reference's mapreduce2d!(f, op, dst, src, dim)
 *   src/mapreduce/2D/mapreduce2d.jl:111-126, which routes dim=1 to
 *   vecmat! (src/mapreduce/2D/vecmat.jl:411-531, vecmat_kernel.jl:1-169)
 *   and dim=2 to matvec! (src/mapreduce/2D/matvec.jl:480-611,
 *   matvec_kernel.jl:1-239). */
size_t kf_reduce_dim_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int dim);

int kf_reduce_dim(kf_op op, kf_map f, kf_dtype dt,
                  const void* A, int64_t rows, int64_t cols, int64_t col_stride,
                  int dim, void* dst, int64_t dst_stride,
                  void* scratch, size_t scratch_bytes, void* stream);

/* Reduction along a dim with a vector operand x (scratch:
 * kf_reduce_dim_scratch_bytes with the same shape and dim):
 *   dim = 2 (matvec): dst[i * dst_stride] = op_j f(A[i, j], x[j * x_stride])
 *   dim = 1 (vecmat): dst[j * dst_stride] = op_i f(x[i * x_stride], A[i, j])
 * with f = x*y (A*x, x'*A) or (x-y)^2. Replaces the reference's
 *   matvec(f, op, A, x) src/mapreduce/2D/matvec.jl:393-474 and
 *   vecmat(f, op, x, A) src/mapreduce/2D/vecmat.jl:328-405. */
int kf_reduce_dim_x(kf_op op, kf_map2 f, kf_dtype dt,
                    const void* A, int64_t rows, int64_t cols, int64_t col_stride, int dim,
                    const void* x, int64_t x_stride, void* dst, int64_t dst_stride,
                    void* scratch, size_t scratch_bytes, void* stream);

/* Batched dim-2 reduction: `batch` column-major rows x cols matrices, the
 * z-th starting at A + z*batch_stride:
 *   dst[(i + z*rows) * dst_stride] = op_j f(A[i + j*col_stride + z*batch_stride])
 * This reduces the middle block of dims of an array viewed as
 * (pre = rows, mid = cols, post = batch); with it the host reduces any set
 * of dims one contiguous block at a time. Replaces the reference's general
 * fallback mapreducedims!(f, op, dst, src, dims)
 *   src/mapreduce/ND/mapreducedims.jl:90-140 (kernel mapreducedims_kernel.jl:1-23). */
size_t kf_reduce_dim_batched_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int64_t batch);

int kf_reduce_dim_batched(kf_op op, kf_map f, kf_dtype dt,
                          const void* A, int64_t rows, int64_t cols, int64_t col_stride,
                          int64_t batch, int64_t batch_stride,
                          void* dst, int64_t dst_stride,
                          void* scratch, size_t scratch_bytes, void* stream);

/* x[i*stride] = g(x[i*stride]) for i < n, in place. Applies the reference's
 * post-map `g` (mapreduce(f, op, x; dims, g), src/mapreduce/mapreduce.jl:51-58)
 * to reduction outputs (kf_scan applies g itself as it stores). */
int kf_post_map(kf_post g, kf_dtype dt, void* x, int64_t n, int64_t stride, void* stream);

/* ---------------------------------------------------------------- copy ----
 * dst[0:bytes] = src[0:bytes] with 16-byte streaming loads/stores (when dst
 * and src are equally misaligned, after a byte head): the bandwidth
 * ceiling the scan/reduce kernels are measured against. Any element type:
 * the copy is of bytes. Replaces the reference's vcopy!
 * src/copy/copy.jl:24-28 / copy_kernel! src/copy/copy_kernel.jl:3-18. */
int kf_copy(void* dst, const void* src, size_t bytes, void* stream);

/* dst[i] = value for i < count, elements of value_bytes (1..64) bytes each;
 * `value` is a host pointer, read before the call returns. 16-byte
 * streaming stores when value_bytes divides 16 and dst is aligned to it,
 * element-wise stores otherwise. Replaces the reference's setvalue!
 * src/copy/copy.jl:52-56 / setvalue_kernel! src/copy/copy_kernel.jl:20-35. */
int kf_fill(void* dst, int64_t count, const void* value, size_t value_bytes, void* stream);

/* ----------------------------------------------------------- bandwidth ----
 * Measurement probes (no counterpart in the reference's library; they play
 * the part of its vendor copy benchmark,
 * perfs/cuda_cpp/cub_nvcc/cub_memcpy_benchmark.cu, bytes = 2N): the copy
 * and read ceilings the scan and reduction kernels are measured against,
 * and the write rate of the read+write bound. src, dst and bytes must be
 * multiples of 16. The copies write dst[0:bytes]; the reads load
 * src[0:bytes] and use dst only as a 4-byte sink; the write stores to
 * dst[0:bytes] and reads nothing (src unused).
 * KF_BW_COPY_ORDERED needs kf_bw_probe_scratch_bytes(bytes) of scratch (no
 * zeroing needed; its epoch comes from a host counter, so it must not be
 * captured into a graph). */
typedef enum {
  KF_BW_COPY = 0,          /* kf_copy: one 16-byte vector per lane, 256 threads    */
  KF_BW_COPY_TILED = 1,    /* the scan's tile shape: 768 threads x 8 striped vectors */
  KF_BW_COPY_ORDERED = 2,  /* one vector per lane; tile t stores after tile t-1 loaded */
  KF_BW_READ = 3,          /* read: one vector per lane                            */
  KF_BW_READ_TILED = 4,    /* read: two vectors per lane, 256 apart (reduction level 0) */
  KF_BW_WRITE = 5          /* write: one vector per lane, plain (temporal) 16-byte stores */
} kf_bw_kind;

size_t kf_bw_probe_scratch_bytes(size_t bytes);

int kf_bw_probe(int kind, void* dst, const void* src, size_t bytes,
                void* scratch, size_t scratch_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KF_H */
