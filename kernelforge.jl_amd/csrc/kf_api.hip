// Error reporting, validation and device queries shared by the entry points.
#include <stdarg.h>
#include <stdio.h>

#include "kf_common.h"

namespace {
thread_local char g_last_error[512] = "";
constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};  // 0 = not queried yet (benign race: same value)
}  // namespace

int kf_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int kf_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kf_set_error(KF_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return KF_OK;
}

size_t kf_dtype_size(kf_dtype dt) {
  switch (dt) {
    case KF_F32: return 4;
    case KF_F64: return 8;
    case KF_I32: return 4;
    case KF_I64: return 8;
    case KF_U8: return 1;
    case KF_F32X2: return 8;
    case KF_Q32: return 16;
    case KF_Q64: return 32;
  }
  return 0;
}

int kf_validate_op(kf_op op, kf_map f, kf_dtype dt, int allow_affine) {
  if (kf_dtype_size(dt) == 0) return kf_set_error(KF_EINVAL, "unknown dtype %d", (int)dt);
  if (f != KF_MAP_IDENTITY && f != KF_MAP_ABS2) return kf_set_error(KF_EINVAL, "unknown map %d", (int)f);
  if (op == KF_OP_AFFINE || dt == KF_F32X2) {
    if (!allow_affine)
      return kf_set_error(KF_EINVAL, "the affine operator is non-commutative and is supported by kf_scan only");
    if (op != KF_OP_AFFINE || dt != KF_F32X2)
      return kf_set_error(KF_EINVAL, "the affine operator requires KF_F32X2 elements and vice versa");
    if (f != KF_MAP_IDENTITY) return kf_set_error(KF_EINVAL, "abs2 is not defined on affine pairs");
    return KF_OK;
  }
  if (dt == KF_Q32 || dt == KF_Q64) {
    if (!allow_affine)
      return kf_set_error(KF_EINVAL, "the quaternion product is non-commutative and is supported by kf_scan only");
    if (op != KF_OP_MUL) return kf_set_error(KF_EINVAL, "quaternion elements take KF_OP_MUL only");
    if (f != KF_MAP_IDENTITY) return kf_set_error(KF_EINVAL, "abs2 is not defined on quaternions here");
    return KF_OK;
  }
  if (op != KF_OP_ADD && op != KF_OP_MAX && op != KF_OP_MIN && op != KF_OP_MUL)
    return kf_set_error(KF_EINVAL, "unknown op %d", (int)op);
  return KF_OK;
}

int kf_device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices && g_cu_count[dev] > 0) return g_cu_count[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < kMaxDevices) g_cu_count[dev] = cus;
  return cus;
}

extern "C" int kf_version(void) { return KF_VERSION; }

extern "C" const char* kf_last_error(void) { return g_last_error; }
