// matvec / vecmat (a reduction along dims with a vector operand) through
// the C ABI; the kernels and launch plan are in kf_reduce_dims.h.
#include "kf_reduce_dims.h"

using namespace kf;

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
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce_dim_x"))) return rc;
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
  if (dim_is_1d(rows, cols, dim))  // a dot product of one row or column with x
    return kf_reduce2(op, f, dt, A, dim == 2 ? col_stride : 1, x, x_stride, dim == 2 ? cols : rows, dst, scratch,
                      scratch_bytes, stream);
  const DimVec dv = dim_vec(A, rows, col_stride, es, dim, 1, 0, true, x, x_stride);
  const DimPlan p = plan_dim(es, rows, cols, dim, dv.vec);
  if (dim_need(es, rows, cols, dim, 1, dv) > 0) {
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
