// mapreduce along dims (plain and batched) through the C ABI; the kernels
// and launch plan are in kf_reduce_dims.h.
#include "kf_reduce_dims.h"

using namespace kf;


extern "C" size_t kf_reduce_dim_scratch_bytes(kf_dtype dt, int64_t rows, int64_t cols, int dim) {
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || rows <= 0 || cols <= 0 || (dim != 1 && dim != 2)) return 256;
  const size_t b = dim_query(es, rows, cols, dim, 1);  // the plan depends on alignment: every case
  // one row reduced along dim 2, or one column along dim 1, is a 1-D reduction
  if (dim_is_1d(rows, cols, dim)) return kmax(b, kf_reduce_scratch_bytes(dt, dim == 2 ? cols : rows));
  return b;
}

extern "C" int kf_reduce_dim(kf_op op, kf_map f, kf_dtype dt, const void* A, int64_t rows, int64_t cols,
                             int64_t col_stride, int dim, void* dst, int64_t dst_stride, void* scratch,
                             size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce_dim"))) return rc;
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
  if (dim_is_1d(rows, cols, dim))  // the 1-D kernels stream it as one vector (strided for one row)
    return kf_reduce(op, f, dt, A, dim == 2 ? cols : rows, dim == 2 ? col_stride : 1, dst, scratch, scratch_bytes,
                     stream);
  const size_t need = kf_reduce_dim_scratch_bytes(dt, rows, cols, dim);
  const DimVec dv = dim_vec(A, rows, col_stride, es, dim, 1, 0, false, nullptr, 0);
  const DimPlan p = plan_dim(es, rows, cols, dim, dv.vec);
  if (dim_need(es, rows, cols, dim, 1, dv) > 0) {
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
  return dim_query(es, rows, cols, 2, batch);
}

extern "C" int kf_reduce_dim_batched(kf_op op, kf_map f, kf_dtype dt, const void* A, int64_t rows, int64_t cols,
                                     int64_t col_stride, int64_t batch, int64_t batch_stride, void* dst,
                                     int64_t dst_stride, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce_dim_batched"))) return rc;
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
  const DimVec dv = dim_vec(A, rows, col_stride, es, 2, batch, batch_stride, false, nullptr, 0);
  const DimPlan p = plan_dim(es, rows, cols, 2, dv.vec, batch);
  if (dim_need(es, rows, cols, 2, batch, dv) > 0) {
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
