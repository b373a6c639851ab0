// Error reporting, validation and device queries shared by the entry points.
#include <atomic>
#include <mutex>
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

// The give-up report word: pinned, host-mapped and coherent, so a kernel's
// system-scope store is visible to a plain host read once it lands. One per
// process, shared by every device (pinned host memory is portable).
namespace {
std::mutex g_mbox_mu;
std::atomic<uint32_t*> g_mbox{nullptr};
bool g_mbox_failed = false;
}  // namespace

uint32_t* kf_mailbox_peek() { return g_mbox.load(std::memory_order_acquire); }

uint32_t* kf_mailbox(hipStream_t stream) {
  uint32_t* p = g_mbox.load(std::memory_order_acquire);
  if (p) return p;
  // never allocate while the caller's stream is being captured into a graph
  // (an allocation there can invalidate the capture): the captured kernels
  // then carry no report word; kf_init before the capture avoids that
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (cap != hipStreamCaptureStatusNone) return nullptr;
  std::lock_guard<std::mutex> lock(g_mbox_mu);
  p = g_mbox.load(std::memory_order_relaxed);
  if (p || g_mbox_failed) return p;
  void* q = nullptr;
  if (hipHostMalloc(&q, 256, hipHostMallocPortable | hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
      !q) {
    (void)hipGetLastError();
    g_mbox_failed = true;
    return nullptr;
  }
  *(volatile uint32_t*)q = 0;
  p = (uint32_t*)q;
  g_mbox.store(p, std::memory_order_release);
  return p;
}

int kf_take_giveup(const char* who) {
  uint32_t* p = kf_mailbox_peek();
  if (!p || __atomic_load_n(p, __ATOMIC_ACQUIRE) == 0) return KF_OK;
  if (__atomic_exchange_n(p, 0u, __ATOMIC_ACQ_REL) == 0) return KF_OK;
  return kf_set_error(KF_EGIVEUP,
                      "%s: not run: a kernel queued by an earlier call gave up waiting on its scratch buffer, so "
                      "that call's results are invalid (a scan buffer stays inert until kf_scan_scratch_status "
                      "clears it)",
                      who);
}

extern "C" int kf_init(void) {
  if (!kf_mailbox(nullptr)) return kf_set_error(KF_EHIP, "kf_init: could not allocate the pinned give-up report word");
  return KF_OK;
}

extern "C" int kf_async_status(int* gave_up) {
  if (!gave_up) return kf_set_error(KF_EINVAL, "kf_async_status: null pointer");
  uint32_t* p = kf_mailbox_peek();
  *gave_up = p && __atomic_exchange_n(p, 0u, __ATOMIC_ACQ_REL) != 0;
  return KF_OK;
}

extern "C" int kf_version(void) { return KF_VERSION; }

extern "C" const char* kf_last_error(void) { return g_last_error; }
