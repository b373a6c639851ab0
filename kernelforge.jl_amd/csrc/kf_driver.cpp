// kf_driver: calls libkfhip.so through the C ABI of include/kf.h from a plain
// host program (no Python, no torch): device memory from hipMalloc, scratch
// sized by the *_scratch_bytes queries and zero-filled once with
// kf_scratch_reset, results checked exactly against host loops, then the
// Float32 scan timed with HIP events. It is what a Julia ccall (or any other
// FFI) binding does, minus the language.
//
//   kf_driver [n]     (default n = 2^24; the timing runs at n = 2^28)
//
// Prints one line per check and "kf_driver: ok" at the end; exits 1 on the
// first mismatch or error.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "kf.h"

namespace {

int fail(const char* what) {
  std::printf("kf_driver: FAIL %s (%s)\n", what, kf_last_error());
  return 1;
}

#define HIP_OK(call)                                                         \
  do {                                                                       \
    if ((call) != hipSuccess) {                                              \
      std::printf("kf_driver: HIP error in %s\n", #call);                    \
      return 1;                                                              \
    }                                                                        \
  } while (0)

uint32_t lcg(uint64_t& s) {
  s = s * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(s >> 33);
}

}  // namespace

int main(int argc, char** argv) {
  const int64_t n = argc > 1 ? std::atoll(argv[1]) : (int64_t)1 << 24;
  if (n < 1) return fail("n must be >= 1");
  std::printf("kf_driver: libkfhip version %d, n = %lld\n", kf_version(), (long long)n);

  // ---- Int32 inclusive / exclusive scan, exact -------------------------
  std::vector<int32_t> h(n), out(n);
  uint64_t seed = 20261201;
  for (auto& v : h) v = (int32_t)(lcg(seed) % 16);
  int32_t *src = nullptr, *dst = nullptr;
  HIP_OK(hipMalloc(&src, n * sizeof(int32_t)));
  HIP_OK(hipMalloc(&dst, n * sizeof(int32_t)));
  HIP_OK(hipMemcpy(src, h.data(), n * sizeof(int32_t), hipMemcpyHostToDevice));
  const size_t sbytes = kf_scan_scratch_bytes(KF_I32, KF_OP_ADD, n);
  void* scratch = nullptr;
  HIP_OK(hipMalloc(&scratch, sbytes));
  if (kf_scratch_reset(scratch, sbytes, nullptr)) return fail("kf_scratch_reset");
  for (int exclusive = 0; exclusive < 2; ++exclusive) {
    if (kf_scan(KF_OP_ADD, KF_MAP_IDENTITY, KF_POST_IDENTITY, KF_I32, exclusive, src, 1, dst, 1, n, scratch, sbytes,
                nullptr))
      return fail("kf_scan");
    HIP_OK(hipMemcpy(out.data(), dst, n * sizeof(int32_t), hipMemcpyDeviceToHost));
    uint32_t acc = 0;
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t incl = acc + (uint32_t)h[i];
      if ((uint32_t)out[i] != (exclusive ? acc : incl)) {
        std::printf("kf_driver: scan mismatch at %lld\n", (long long)i);
        return fail(exclusive ? "exclusive scan" : "inclusive scan");
      }
      acc = incl;
    }
    std::printf("kf_driver: Int32 %s scan exact\n", exclusive ? "exclusive" : "inclusive");
  }

  // ---- full reductions (+ wraps, max), exact ---------------------------
  const size_t rbytes = kf_reduce_scratch_bytes(KF_I32, n);
  void* rscratch = nullptr;
  HIP_OK(hipMalloc(&rscratch, rbytes));
  if (kf_scratch_reset(rscratch, rbytes, nullptr)) return fail("kf_scratch_reset");
  int32_t* d1 = nullptr;
  HIP_OK(hipMalloc(&d1, sizeof(int32_t)));
  for (kf_op op : {KF_OP_ADD, KF_OP_MAX}) {
    if (kf_reduce(op, KF_MAP_ABS2, KF_I32, src, n, 1, d1, rscratch, rbytes, nullptr)) return fail("kf_reduce");
    int32_t got = 0;
    HIP_OK(hipMemcpy(&got, d1, sizeof got, hipMemcpyDeviceToHost));
    uint32_t sum = 0;
    int32_t mx = INT32_MIN;
    for (int64_t i = 0; i < n; ++i) {
      const int32_t sq = (int32_t)((uint32_t)h[i] * (uint32_t)h[i]);
      sum += (uint32_t)sq;
      mx = sq > mx ? sq : mx;
    }
    if (got != (op == KF_OP_ADD ? (int32_t)sum : mx)) return fail("kf_reduce value");
    std::printf("kf_driver: mapreduce(abs2, %s) exact\n", op == KF_OP_ADD ? "+" : "max");
  }

  // ---- dims reductions of a column-major matrix (a view: every 2nd column)
  const int64_t rows = 1000, cols = 300, cs = 2 * rows;  // columns 0, 2, 4, ... of a rows x 2*cols matrix
  if (rows * 2 * cols <= n) {
    std::vector<int32_t> col(cols), row(rows);
    int32_t* dd = nullptr;
    HIP_OK(hipMalloc(&dd, (rows > cols ? rows : cols) * sizeof(int32_t)));
    for (int dim = 1; dim <= 2; ++dim) {
      const size_t dbytes = kf_reduce_dim_scratch_bytes(KF_I32, rows, cols, dim);
      void* ds = nullptr;
      HIP_OK(hipMalloc(&ds, dbytes));
      if (kf_scratch_reset(ds, dbytes, nullptr)) return fail("kf_scratch_reset");
      if (kf_reduce_dim(KF_OP_ADD, KF_MAP_IDENTITY, KF_I32, src, rows, cols, cs, dim, dd, 1, ds, dbytes, nullptr))
        return fail("kf_reduce_dim");
      std::vector<int32_t>& got = dim == 1 ? col : row;
      HIP_OK(hipMemcpy(got.data(), dd, got.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
      for (int64_t k = 0; k < (int64_t)got.size(); ++k) {
        uint32_t s = 0;
        if (dim == 1)
          for (int64_t i = 0; i < rows; ++i) s += (uint32_t)h[i + k * cs];
        else
          for (int64_t j = 0; j < cols; ++j) s += (uint32_t)h[k + j * cs];
        if ((int32_t)s != got[k]) return fail("kf_reduce_dim value");
      }
      std::printf("kf_driver: mapreduce(identity, +; dims=%d) on a column view exact\n", dim);
      HIP_OK(hipFree(ds));
    }
    HIP_OK(hipFree(dd));
  }
  HIP_OK(hipFree(src));
  HIP_OK(hipFree(dst));
  HIP_OK(hipFree(d1));
  HIP_OK(hipFree(scratch));
  HIP_OK(hipFree(rscratch));

  // ---- timing: scan!(+) Float32 n = 2^28 on a stream ---------------------
  const int64_t nt = (int64_t)1 << 28;
  float *fs = nullptr, *fd = nullptr;
  HIP_OK(hipMalloc(&fs, nt * sizeof(float)));
  HIP_OK(hipMalloc(&fd, nt * sizeof(float)));
  HIP_OK(hipMemset(fs, 0, nt * sizeof(float)));
  const size_t tb = kf_scan_scratch_bytes(KF_F32, KF_OP_ADD, nt);
  void* ts = nullptr;
  HIP_OK(hipMalloc(&ts, tb));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  if (kf_scratch_reset(ts, tb, stream)) return fail("kf_scratch_reset");
  for (int i = 0; i < 5; ++i)
    if (kf_scan(KF_OP_ADD, KF_MAP_IDENTITY, KF_POST_IDENTITY, KF_F32, 0, fs, 1, fd, 1, nt, ts, tb, stream))
      return fail("kf_scan");
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  const int reps = 20;
  HIP_OK(hipEventRecord(e0, stream));
  for (int i = 0; i < reps; ++i)
    if (kf_scan(KF_OP_ADD, KF_MAP_IDENTITY, KF_POST_IDENTITY, KF_F32, 0, fs, 1, fd, 1, nt, ts, tb, stream))
      return fail("kf_scan");
  HIP_OK(hipEventRecord(e1, stream));
  HIP_OK(hipEventSynchronize(e1));
  float ms = 0.f;
  HIP_OK(hipEventElapsedTime(&ms, e0, e1));
  const double us = 1e3 * ms / reps;
  std::printf("kf_driver: scan!(+) Float32 n=2^28: %.1f us, %.0f GB/s\n", us, 8.0 * nt / us / 1e3);
  HIP_OK(hipStreamDestroy(stream));
  HIP_OK(hipFree(fs));
  HIP_OK(hipFree(fd));
  HIP_OK(hipFree(ts));
  std::printf("kf_driver: ok\n");
  return 0;
}
