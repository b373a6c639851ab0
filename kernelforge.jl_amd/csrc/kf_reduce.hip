// Full reductions (mapreduce) for gfx950 over one, two or three arrays;
// the reductions along dims are in kf_reduce_dims.hip.
//
// Same two stages as the reference's kernel (reference
// src/mapreduce/1D/mapreduce1d_kernel.jl:5-93): partial results per
// workgroup, then a combine. MI355X design:
//  * Stage 1 streams with 16-byte nontemporal loads, several in flight per
//    lane, every vector element folded into its own accumulator (16
//    independent Float32 sums per lane: accurate and dependency-free).
//  * The combine is an atomic-free fold inside the last launch: the
//    reference's single launch lets workgroup 1 spin on per-workgroup flags
//    (mapreduce1d_kernel.jl:66-92); here the last level's workgroups (at
//    most kFoldMax) publish epoch-tagged partial slots with relaxed
//    device-scope stores and the last workgroup gathers them
//    (fold_partial). Every contiguous reduction takes one launch: up to
//    16*256*kFoldMax vectors (128 MiB) one-shot workgroups of 2-16 vectors
//    per lane, from 256 MiB kFoldMax persistent workgroups over contiguous
//    chunks; in between, a one-shot level 0 that writes partials and a
//    folding level 1. A "last workgroup done" ticket was measured to
//    serialise same-address device atomics at the end of the grid (1.8
//    TB/s with 8192 workgroups), and fences cost more than the launch they
//    save.
//  * Combine orders depend only on the shape and pointer alignment, so every
//    result is bit-for-bit reproducible run to run.
#include <mutex>

#include "kf_reduce.h"

namespace kf {
#ifdef KF_TIMELINE
// Instrumented build only: every workgroup of a folding one-launch
// reduction records, by thread 0, three 100 MHz realtime stamps (start,
// its loads folded into its partial, slot published or fold done), its XCD
// and its HW_ID word at g_red_timeline + workgroup * kRedTimelineWords.
__device__ uint64_t* g_red_timeline = nullptr;
constexpr int kRedTimelineWords = 6;
__device__ inline void red_timeline(uint64_t t0, uint64_t t1) {
  if (threadIdx.x == 0 && g_red_timeline) {
    uint64_t* w = g_red_timeline + (int64_t)blockIdx.x * kRedTimelineWords;
    w[0] = t0;
    w[1] = t1;
    w[2] = __builtin_amdgcn_s_memrealtime();
    w[3] = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // HW_REG_XCC_ID[3:0]
    w[4] = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID
    w[5] = gridDim.x;
  }
}
#define KF_RED_STAMP(v) const uint64_t v = __builtin_amdgcn_s_memrealtime()
#else
#define KF_RED_STAMP(v)
#endif
// ---------------------------------------------------------------------------
// Full reduction, stage 1: grid-stride over 16-byte vectors. An unaligned
// head and the ragged tail are folded in by workgroup 0, so any
// element-aligned contiguous view takes the vector path.
// ---------------------------------------------------------------------------
template <class T, class Op, class Map>
__global__ __launch_bounds__(kRedBlock) void reduce_kernel(const T* src, int64_t n, int64_t stride,
                                                           T* out, int vec) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const int64_t gtid = (int64_t)blockIdx.x * kRedBlock + tid;
  const int64_t gsize = (int64_t)gridDim.x * kRedBlock;

  T acc = id;
  if (vec) {
    const int64_t head = kmin<int64_t>(n, (int64_t)(((16 - ((uintptr_t)src & 15)) & 15) / sizeof(T)));
    const int64_t nvec = (n - head) / EPV;
    const int64_t tail0 = head + nvec * EPV;
    const uint4* v = reinterpret_cast<const uint4*>(src + head);
    T a[kRedUnroll][EPV];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[u][e] = id;
    int64_t i = gtid;
    for (; i + (kRedUnroll - 1) * gsize < nvec; i += kRedUnroll * gsize) {
      uint4 r[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) r[u] = ld_stream(v + i + u * gsize);
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) {
        T x[EPV];
        __builtin_memcpy(x, &r[u], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e) a[u][e] = Op::combine(a[u][e], Map::apply(x[e]));
      }
    }
    for (; i < nvec; i += gsize) {
      const uint4 r = ld_stream(v + i);
      T x[EPV];
      __builtin_memcpy(x, &r, 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) a[0][e] = Op::combine(a[0][e], Map::apply(x[e]));
    }
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc = Op::combine(acc, a[u][e]);
    if (blockIdx.x == 0) {
      if (tid < head) acc = Op::combine(acc, Map::apply(src[tid]));
      if (tail0 + tid < n) acc = Op::combine(acc, Map::apply(src[tail0 + tid]));
    }
  } else {
    T a[kRedUnroll];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) a[u] = id;
    int64_t i = gtid;
    for (; i + (kRedUnroll - 1) * gsize < n; i += kRedUnroll * gsize) {
      T x[kRedUnroll];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) x[u] = src[(i + u * gsize) * stride];
#pragma unroll
      for (int u = 0; u < kRedUnroll; ++u) a[u] = Op::combine(a[u], Map::apply(x[u]));
    }
    for (; i < n; i += gsize) a[0] = Op::combine(a[0], Map::apply(src[i * stride]));
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) acc = Op::combine(acc, a[u]);
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if (tid == 0) out[blockIdx.x] = part;  // a partial, or the result when gridDim.x == 1
}

// Full reduction, stage 1 (vector path): one-shot workgroups. Workgroup b
// reads the kOnceVecs 16-byte vectors [b*kOnceVecs, (b+1)*kOnceVecs) once and
// writes one partial; the grid covers the whole array. Many short-lived
// workgroups keep far more loads in flight than a grid-stride loop (measured
// 7.3 vs 6.1 TB/s for Float32 reads on MI355X). Workgroup 0 also folds in
// the unaligned head and the ragged tail. The same kernel (head = tail = 0,
// identity map) reduces the partials of the previous level.
constexpr int kOnceUnroll = 2;
constexpr int kOnceVecs = kRedBlock * kOnceUnroll;

// Single-level fold, replacing combine_all_kernel's launch for grids of
// 2..kFoldMax workgroups. Every workgroup but the last publishes its
// partial into its slot as W 64-bit words, each {tag:32, value bits:32},
// with relaxed device-scope stores. The last workgroup polls all slots
// (8 per thread, all in flight together) until every word carries the
// tag, then combines them in slot order with its own partial last, so
// the result does not depend on timing. It stores the result and the tag
// as the new epoch. The tag is epoch + 1, read by thread 0 with a plain
// load at kernel start, before the workgroup's data loads (`hdr0`), so its
// round trip overlaps them: the previous call's last workgroup wrote it before that kernel
// ended, and within a call every reader loads it before publishing,
// which the waiter's completion depends on. Slots of older calls never
// match. Only one workgroup ever waits, so progress needs no co-residency;
// a bounded spin (only a corrupted or concurrently shared buffer can
// exhaust it) keeps a bad buffer from hanging the GPU, and its exhaustion
// is reported, never passed off as a result (see the give-up branch).
constexpr uint32_t kFoldSpinLimit = 1u << 22;
// The fold's give-up controls: the host-mapped report word, the waiter's
// poll budget and, in the instrumented library only, a workgroup that
// withholds its slot (kf_debug_reduce_giveup) so that the give-up path can
// be tested with every kernel exiting normally.
struct FoldCtl {
  uint32_t* mbox;
  uint32_t limit;
  int withhold;
};
#ifdef KF_TIMELINE
thread_local int g_fold_withhold = -1;
thread_local uint32_t g_fold_limit = kFoldSpinLimit;
#else
constexpr int g_fold_withhold = -1;
constexpr uint32_t g_fold_limit = kFoldSpinLimit;
#endif
inline FoldCtl fold_ctl() { return FoldCtl{kf_mailbox_peek(), g_fold_limit, g_fold_withhold}; }
__device__ inline uint32_t fold_epoch(const uint64_t* hdr) { return threadIdx.x == 0 ? (uint32_t)hdr[0] : 0u; }
template <class T, class Op>
__device__ inline void fold_partial(T part, T* out, uint64_t* hdr, T* s_wave, uint32_t hdr0, FoldCtl ctl) {
  constexpr int W = Words<T>::W;
  constexpr int PER = kFoldMax / kRedBlock;
  __shared__ uint32_t s_tag;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const uint32_t t = hdr0 + 1u;
    s_tag = t == 0 ? 1u : t;
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  uint64_t* slots = hdr + 256 / sizeof(uint64_t);
  const int last = (int)gridDim.x - 1;
  if ((int)blockIdx.x != last) {
    if (tid == 0 && (int)blockIdx.x != ctl.withhold) {
      const Words<T> w = to_words(part);
#pragma unroll
      for (int i = 0; i < W; ++i) st_agent(slots + 2 * blockIdx.x + i, ((uint64_t)tag << 32) | w.w[i]);
    }
    return;
  }
  // the last workgroup: slot k * kRedBlock + tid of every k on this thread
  const T id = Op::template identity<T>();
  T v[PER];
  bool done[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = id;
    done[k] = k * kRedBlock + tid >= last;
  }
  bool complete = false;
  for (uint32_t polls = 0; polls < ctl.limit; ++polls) {
    uint64_t d[PER][W];
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (!done[k]) {
#pragma unroll
        for (int i = 0; i < W; ++i) d[k][i] = ld_agent(slots + 2 * (k * kRedBlock + tid) + i);
      }
    bool all = true;
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (!done[k]) {
        bool ok = true;
        Words<T> w;
#pragma unroll
        for (int i = 0; i < W; ++i) {
          ok &= (uint32_t)(d[k][i] >> 32) == tag;
          w.w[i] = (uint32_t)d[k][i];
        }
        if (ok) {
          v[k] = from_words<T>(w);
          done[k] = true;
        } else {
          all = false;
        }
      }
    if (__syncthreads_and(all)) {
      complete = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!complete) {
    // Gave up: out[0] keeps its old value. The flag (header word 1) stays
    // set for kf_reduce_scratch_status, the report word tells the host,
    // and the epoch skips one value so that no slot this call's workgroups
    // published (or publish late) reads as current in the next call.
    if (tid == 0) {
      hdr[1] = 1;
      hdr[0] = tag + 1u;
      report_giveup(ctl.mbox);
    }
    return;
  }
  T acc = v[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) acc = Op::combine(acc, v[k]);
  __syncthreads();  // s_wave still holds this workgroup's own partial sums
  const T others = block_reduce<T, Op>(acc, s_wave);
  if (tid == 0) {
    out[0] = Op::combine(others, part);
    hdr[0] = tag;
  }
}

template <class T, class Op, class Map, bool FOLD = false, int U = kOnceUnroll>
__global__ __launch_bounds__(kRedBlock) void reduce_once_kernel(const T* src, int64_t n, int64_t head,
                                                                int64_t nvec, T* out, uint64_t* fold_hdr, FoldCtl ctl) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const int tid = threadIdx.x;
  KF_RED_STAMP(tl_start);
  const uint32_t hdr0 = FOLD ? fold_epoch(fold_hdr) : 0u;  // fold tag, read ahead of the data
  const uint4* v = reinterpret_cast<const uint4*>(src + head);
  const int64_t base = (int64_t)blockIdx.x * (kRedBlock * U) + tid;
  uint4 r[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + u * kRedBlock < nvec) r[u] = ld_stream(v + base + u * kRedBlock);
  VecFold<T, Op, Map> f;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + u * kRedBlock < nvec) f.add(r[u]);
  T acc = f.total();
  KF_RED_STAMP(tl_loaded);
  if (blockIdx.x == 0) {
    const int64_t tail0 = head + nvec * EPV;
    if (tid < head) acc = Op::combine(acc, Map::apply(src[tid]));
    if (tail0 + tid < n) acc = Op::combine(acc, Map::apply(src[tail0 + tid]));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if constexpr (!FOLD) {
    if (tid == 0) out[blockIdx.x] = part;  // a partial, or the result when gridDim.x == 1
  } else {
    fold_partial<T, Op>(part, out, fold_hdr, s_wave, hdr0, ctl);  // out is the result
#ifdef KF_TIMELINE
    red_timeline(tl_start, tl_loaded);
#endif
  }
}

// Single-launch reduction for arrays of kChunkMinVecs vectors (256 MiB) or
// more: kFoldMax workgroups, workgroup b streaming the contiguous chunk
// [b*chunk, (b+1)*chunk) of vectors with U loads in flight per lane, then
// the fold. At 32 loads about three workgroups fit per CU, so the grid runs
// in rounds; the fold's waiter is the last workgroup, dispatched last, so
// every workgroup it waits for has started and none of them waits. The host makes `chunk` a whole number of
// U * kRedBlock-vector rounds, so only the last non-empty chunk ends in a
// partial round, which is one guarded round with every load in flight (a
// one-load-per-iteration remainder loop cost 13 serial memory latencies per
// workgroup at 10^9 Float32: 630 vs 590 us). Measured on MI355X against one-shot level 0 +
// folding level 1 (eager, us): Float32 2^26 41.0 vs 41.9-43.1, 2^28 154.0
// vs 156.9, 2^30 606 vs 622; Float64 2^26 79.1 vs 80.9, 2^28 305 vs 318;
// Int32 2^28 153.7 vs 156.7. At 200 MB (5*10^7 Float32, 1.5 loop
// iterations per lane) it lost (32.5 vs 31.6), hence the threshold. Loads
// in flight per lane (HIP graphs, median of 7, us, 16 / 8 / 24 / 32 / 48 /
// 64; 32 loads take 146 VGPRs, three workgroups per CU): Float32 2^28
// 154.6 / 157.2 / 161.7 / 153.2 / 161.3 / 153.8, 2^30 607.8 / 613.1 / 611.5
// / 602.5 / 610.9 / 603.2, 10^8 62.1 / 62.2 / 61.7 / 59.2 / 58.9 / 61.5;
// Float64 2^27 154.8 / 156.3 / 162.6 / 153.9 / 162.7 / 153.3; Int32 2^28
// 154.4 / 156.5 / 162.5 / 153.5 / 162.8 / 154.0 (24 and 48 do not divide
// the rounds evenly over the CUs' resident workgroups).
constexpr int64_t kChunkMinVecs = (int64_t)1 << 24;
constexpr int kChunkUnroll = 32;
template <class T, class Op, class Map, int U>
__global__ __launch_bounds__(kRedBlock) void reduce_chunk_kernel(const T* src, int64_t n, int64_t head, int64_t nvec,
                                                                 int64_t chunk, T* out, uint64_t* fold_hdr, FoldCtl ctl) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const int tid = threadIdx.x;
  KF_RED_STAMP(tl_start);
  const uint32_t hdr0 = fold_epoch(fold_hdr);  // fold tag, read ahead of the data
  const uint4* v = reinterpret_cast<const uint4*>(src + head);
  const int64_t b0 = (int64_t)blockIdx.x * chunk;
  const int64_t b1 = kmin<int64_t>(nvec, b0 + chunk);
  VecFold<T, Op, Map> f;
  int64_t i = b0 + tid;
  for (; i + (int64_t)(U - 1) * kRedBlock < b1; i += (int64_t)U * kRedBlock) {
    uint4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = ld_stream(v + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < U; ++u) f.add(r[u]);
  }
  if (i < b1) {  // the partial last round: fewer than U vectors per lane
    uint4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * kRedBlock < b1) r[u] = ld_stream(v + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * kRedBlock < b1) f.add(r[u]);
  }
  T acc = f.total();
  KF_RED_STAMP(tl_loaded);
  if (blockIdx.x == 0) {
    const int64_t tail0 = head + nvec * EPV;
    if (tid < head) acc = Op::combine(acc, Map::apply(src[tid]));
    if (tail0 + tid < n) acc = Op::combine(acc, Map::apply(src[tail0 + tid]));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  fold_partial<T, Op>(part, out, fold_hdr, s_wave, hdr0, ctl);
#ifdef KF_TIMELINE
  red_timeline(tl_start, tl_loaded);
#endif
}

// Strided views with short strides (stride * sizeof(T) <= kStrideVecBytes,
// e.g. x[1:2:end]): every 128-byte line of the view's span holds elements of
// the view, so HBM reads the whole span either way. Stream the span with
// 16-byte loads instead of element loads, combining only the elements at
// span offsets that are multiples of the stride. kFoldMax persistent
// workgroups over contiguous chunks (whole rounds but the last), folded in
// the same launch; workgroup 0 folds in the head (up to the first 128-byte
// line) and the tail of the span. The vector holding span offset q keeps the
// elements e with (q + e) % stride == 0: a bit pattern of period `stride`,
// shifted by the vector's residue, which each lane advances by a constant
// per vector instead of dividing.
constexpr int kStrideVecBytes = 32;
constexpr int kStrideUnroll = 8;
template <class T, class Op, class Map>
__global__ __launch_bounds__(kRedBlock) void reduce_stride_kernel(const T* src, int64_t span, int stride,
                                                                  int64_t head, int64_t nvec, int64_t chunk, T* out,
                                                                  uint64_t* fold_hdr, FoldCtl ctl) {
  constexpr int EPV = 16 / (int)sizeof(T);
  constexpr int U = kStrideUnroll;
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const uint32_t hdr0 = fold_epoch(fold_hdr);  // fold tag, read ahead of the data
  const uint4* v = reinterpret_cast<const uint4*>(src + head);
  const int64_t b0 = (int64_t)blockIdx.x * chunk;
  const int64_t b1 = kmin<int64_t>(nvec, b0 + chunk);
  // bits e = 0, stride, 2*stride, ... below EPV
  uint32_t pat = 0;
  for (int e = 0; e < EPV; e += stride) pat |= 1u << e;
  // residue of the span offset of this lane's vectors, and its steps
  int rr = (int)((head + (b0 + tid) * (int64_t)EPV) % stride);
  const int step_u = (int)(((int64_t)kRedBlock * EPV) % stride);
  const int step_round = (int)(((int64_t)U * kRedBlock * EPV) % stride);
  T a[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) a[e] = id;
  for (int64_t i = b0 + tid; i < b1; i += (int64_t)U * kRedBlock) {
    uint4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * kRedBlock < b1) r[u] = ld_stream(v + i + u * kRedBlock);
    int q = rr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i + u * kRedBlock < b1) {
        const uint32_t m = pat << (q == 0 ? 0 : stride - q);
        T x[EPV];
        __builtin_memcpy(x, &r[u], 16);
#pragma unroll
        for (int e = 0; e < EPV; ++e)
          if ((m >> e) & 1u) a[e] = Op::combine(a[e], Map::apply(x[e]));
      }
      q += step_u;
      if (q >= stride) q -= stride;
    }
    rr += step_round;
    if (rr >= stride) rr -= stride;
  }
  T acc = a[0];
#pragma unroll
  for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, a[e]);
  if (blockIdx.x == 0) {
    // head: span offsets [0, head); tail: [head + nvec * EPV, span)
    if (tid < head && tid % stride == 0) acc = Op::combine(acc, Map::apply(src[tid]));
    const int64_t t = head + nvec * EPV + tid;
    if (t < span && t % stride == 0) acc = Op::combine(acc, Map::apply(src[t]));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  fold_partial<T, Op>(part, out, fold_hdr, s_wave, hdr0, ctl);
}

// Full reduction, stage 2: one 1024-thread workgroup combines `count`
// partials; each thread issues all of its (at most kRedMaxBlocks/1024) loads
// before combining, so the stage costs about one memory latency.
constexpr int kCombineBlock = 1024;
template <class T, class Op>
__global__ __launch_bounds__(kCombineBlock) void combine_all_kernel(const T* partials, int count, T* dst) {
  constexpr int PER = kRedMaxBlocks / kCombineBlock;
  constexpr int WAVES = kCombineBlock / kWave;
  __shared__ T s_wave[WAVES];
  const T id = Op::template identity<T>();
  T v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = k * kCombineBlock + threadIdx.x;
    v[k] = j < count ? partials[j] : id;
  }
  T x = v[0];
#pragma unroll
  for (int k = 1; k < PER; ++k) x = Op::combine(x, v[k]);
  x = wave_reduce<Op>(x);
  if (lane_id() == 0) s_wave[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    T r = s_wave[0];
    for (int w = 1; w < WAVES; ++w) r = Op::combine(r, s_wave[w]);
    dst[0] = r;
  }
}


template <class T> int reduce_grid(int64_t n) {
  constexpr int64_t per_block = (int64_t)kRedBlock * kRedUnroll * 2;
  int64_t g = (n + per_block - 1) / per_block;
  const int64_t cap = kmin<int64_t>(kRedMaxBlocks, (int64_t)kf_device_cu_count() * 32);
  if (g > cap) g = cap;
  return (int)kmax<int64_t>(g, 1);
}

// Level sizes of the vector path. Level 0 reads the input with u0 16-byte
// vectors per lane; every later level reduces the previous level's partials
// (read as 16-byte vectors) with kOnceUnroll per lane, until at most
// kFoldMax partial-producing workgroups remain: the last level folds its
// partials into the result inside the same launch (fold_partial), so no
// separate combine launch is needed. u0 is the smallest of 2, 4, 8 and 16
// that brings level 0 itself under kFoldMax, so arrays of up to 128 MiB
// reduce in one launch; larger ones take u0 = 2 and a folding level 1.
// Measured on MI355X (HIP graphs, us; one launch at the adaptive width
// against level 0 at 2 vectors + a folding level 1): Float32 5*10^6 4.06
// vs 6.97, 10^7 6.80 vs 10.37, 2*10^7 12.3 vs 14.3; Float64 8*10^6 10.1 vs
// 14.2; UInt8 1.2*10^8 20.9 vs 20.3 (the one loss); eager calls gain the
// launch too (Float32 10^7 7.1 vs 10.7). At 2^28 Float32, 157 us in two
// launches; before, a third combine_all_kernel launch made it 160-162 us.
// Single-launch alternatives measured slower at 2^28: 2048 persistent
// workgroups over contiguous chunks (161 us), one-shot workgroups whose
// group leaders wait for their group's partials (165 us; 160 us with the
// groups formed per XCD), and a last-arriver fold by device-scope atomic
// counters (188 us: the atomics serialise).
constexpr int kOnceMaxUnroll = 16;
struct OnceLevels {
  int nlev;
  int u0;
  int64_t count[8];
};
inline OnceLevels once_levels(int64_t nvec, int epv, bool adaptive = true, int max_u = kOnceMaxUnroll) {
  OnceLevels L{};
  L.u0 = kOnceUnroll;
  if (adaptive) {
    for (int u = kOnceUnroll; u <= max_u; u *= 2)
      if ((nvec + (int64_t)kRedBlock * u - 1) / ((int64_t)kRedBlock * u) <= kFoldMax) {
        L.u0 = u;
        break;
      }
  }
  int64_t c = kmax<int64_t>(1, (nvec + (int64_t)kRedBlock * L.u0 - 1) / ((int64_t)kRedBlock * L.u0));
  L.count[L.nlev++] = c;
  while (c > kFoldMax && L.nlev < 8) {
    const int64_t cv = (c + epv - 1) / epv;  // partials read as 16-byte vectors
    c = (cv + kOnceVecs - 1) / kOnceVecs;
    L.count[L.nlev++] = c;
  }
  return L;
}

// Scratch for a full reduction of n elements of es bytes: two ping-pong
// partial buffers for the vector path, or kRedMaxBlocks partials for the
// strided path, whichever is larger.
inline size_t reduce_scratch(size_t es, int64_t n) {
  const int64_t nvec = n / (int64_t)(16 / es);
  const OnceLevels L = once_levels(nvec, (int)(16 / es));
  size_t a = 0, b = 0;
  for (int i = 0; i < L.nlev; ++i) {
    const size_t bytes = round256((size_t)L.count[i] * es + 16);
    if (i % 2 == 0) a = kmax(a, bytes); else b = kmax(b, bytes);
  }
  return kRedReserved + kmax<size_t>(a + b, round256((size_t)kRedMaxBlocks * es));
}

// Launch of reduce_once_kernel with the level's vectors per lane.
template <class T, class Op, class Map, bool FOLD>
void launch_once(int u, unsigned grid, const T* src, int64_t n, int64_t head, int64_t nvec, T* out, uint64_t* hdr,
                 hipStream_t stream) {
  if (u == 16)
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map, FOLD, 16>), dim3(grid), dim3(kRedBlock), 0, stream, src, n, head,
                       nvec, out, hdr, fold_ctl());
  else if (u == 8)
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map, FOLD, 8>), dim3(grid), dim3(kRedBlock), 0, stream, src, n, head,
                       nvec, out, hdr, fold_ctl());
  else if (u == 4)
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map, FOLD, 4>), dim3(grid), dim3(kRedBlock), 0, stream, src, n, head,
                       nvec, out, hdr, fold_ctl());
  else
    hipLaunchKernelGGL((reduce_once_kernel<T, Op, Map, FOLD, kOnceUnroll>), dim3(grid), dim3(kRedBlock), 0, stream, src,
                       n, head, nvec, out, hdr, fold_ctl());
}

constexpr uintptr_t kHeadAlign = 128;  // head elements, up to 127 (< kRedBlock)

template <class T, class Op, class Map>
int launch_reduce(const void* src, int64_t n, int64_t stride, void* dst, void* scratch,
                  hipStream_t stream) {
  constexpr int EPV = 16 / (int)sizeof(T);
  uint8_t* work = (uint8_t*)red_work(scratch);
  if (stride != 1 && n > 1 && stride * (int64_t)sizeof(T) <= kStrideVecBytes) {
    const int64_t span = (n - 1) * stride + 1;
    const int64_t head = kmin<int64_t>(span, (int64_t)(((kHeadAlign - ((uintptr_t)src & (kHeadAlign - 1))) &
                                                        (kHeadAlign - 1)) / sizeof(T)));
    const int64_t nvec = (span - head) / EPV;
    constexpr int64_t kRound = (int64_t)kStrideUnroll * kRedBlock;
    const int64_t grid = kmax<int64_t>(1, kmin<int64_t>(kFoldMax, (nvec + kRound - 1) / kRound));
    const int64_t chunk = ((nvec + grid - 1) / grid + kRound - 1) / kRound * kRound;
    if (grid == 1) {
      // one workgroup: its partial is the result (no fold)
      hipLaunchKernelGGL((reduce_kernel<T, Op, Map>), dim3(1), dim3(kRedBlock), 0, stream, (const T*)src, n, stride,
                         (T*)dst, 0);
      return kf_check_launch("reduce_kernel");
    }
    hipLaunchKernelGGL((reduce_stride_kernel<T, Op, Map>), dim3((unsigned)grid), dim3(kRedBlock), 0, stream,
                       (const T*)src, span, (int)stride, head, nvec, chunk, (T*)dst, (uint64_t*)scratch, fold_ctl());
    return kf_check_launch("reduce_stride_kernel");
  }
  if (stride != 1) {
    const int grid = reduce_grid<T>(n);
    T* out = grid == 1 ? (T*)dst : (T*)work;
    hipLaunchKernelGGL((reduce_kernel<T, Op, Map>), dim3(grid), dim3(kRedBlock), 0, stream,
                       (const T*)src, n, stride, out, 0);
    if (grid > 1)
      hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                         (const T*)work, grid, (T*)dst);
    return kf_check_launch("reduce_kernel");
  }
  // The vectors start at the first 128-byte line boundary: a vector stream
  // that starts mid-line makes every workgroup's first and last lines
  // shared with a neighbour, often on another XCD (and L2), and fetched
  // twice (2^28 Float32 at x[2:]: 159.9 us with a 16-byte head, 155.0 with a
  // 128-byte one; aligned 153.7). Workgroup 0 folds in the head elements.
  const int64_t head = kmin<int64_t>(n, (int64_t)(((kHeadAlign - ((uintptr_t)src & (kHeadAlign - 1))) &
                                                   (kHeadAlign - 1)) / sizeof(T)));
  const int64_t nvec = (n - head) / EPV;
  const OnceLevels L = once_levels(nvec, EPV);
  if (nvec >= kChunkMinVecs) {
    // kFoldMax persistent workgroups over contiguous chunks, folded in the
    // same launch
    constexpr int64_t kRound = (int64_t)kChunkUnroll * kRedBlock;
    const int64_t chunk = ((nvec + kFoldMax - 1) / kFoldMax + kRound - 1) / kRound * kRound;
    hipLaunchKernelGGL((reduce_chunk_kernel<T, Op, Map, kChunkUnroll>), dim3(kFoldMax), dim3(kRedBlock), 0, stream,
                       (const T*)src, n, head, nvec, chunk, (T*)dst, (uint64_t*)scratch, fold_ctl());
    return kf_check_launch("reduce_chunk_kernel");
  }
  size_t abytes = 0;
  for (int i = 0; i < L.nlev; i += 2) abytes = kmax(abytes, round256((size_t)L.count[i] * sizeof(T) + 16));
  T* buf[2] = {(T*)work, (T*)(work + abytes)};
  // level 0 reads the input (with map, head and tail); later levels reduce
  // partials; the last level writes the result (one workgroup) or folds
  const int last = L.nlev - 1;
  for (int i = 0; i <= last; ++i) {
    const unsigned grid = (unsigned)L.count[i];
    T* out = i == last ? (T*)dst : buf[i % 2];
    const bool fold = i == last && grid > 1;
    if (i == 0) {
      if (fold)
        launch_once<T, Op, Map, true>(L.u0, grid, (const T*)src, n, head, nvec, out, (uint64_t*)scratch, stream);
      else
        launch_once<T, Op, Map, false>(L.u0, grid, (const T*)src, n, head, nvec, out, nullptr, stream);
    } else {
      const int64_t m = L.count[i - 1];
      const T* in = buf[(i - 1) % 2];
      if (fold)
        launch_once<T, Op, MapIdentity, true>(kOnceUnroll, grid, in, m, 0, m / EPV, out, (uint64_t*)scratch, stream);
      else
        launch_once<T, Op, MapIdentity, false>(kOnceUnroll, grid, in, m, 0, m / EPV, out, nullptr, stream);
    }
  }
  return kf_check_launch("reduce_once_kernel");
}

// ---------------------------------------------------------------------------
// Two-array full reduction: dst = op_i f2(x[i], y[i]) with f2 = x*y (dot
// product) or (x-y)^2 (squared distance). Level 0 reads both arrays
// (one-shot when both are 16-byte aligned and contiguous, grid-stride
// otherwise); later levels reuse the partial reduction above.
// ---------------------------------------------------------------------------
struct Map3Mul {
  template <class T> __device__ static T apply(T a, T b, T c) { return Map2Mul::apply(Map2Mul::apply(a, b), c); }
};

// K operand arrays of one multi-array reduction (K = 2 or 3), passed by value.
template <class T, int K> struct Operands {
  const T* p[K];
  int64_t s[K];
};
template <class M, class T, int K> __device__ inline T apply_k(const T (&v)[K]) {
  if constexpr (K == 2)
    return M::apply(v[0], v[1]);
  else
    return M::apply(v[0], v[1], v[2]);
}

// Multi-array reduction, vector path: the one-shot workgroups of
// reduce_once_kernel, each loading the same 16-byte vectors of all K arrays.
template <class T, class Op, class M, int K, bool FOLD = false, int U = kOnceUnroll>
__global__ __launch_bounds__(kRedBlock) void reducek_once_kernel(Operands<T, K> a, int64_t n, T* out,
                                                                 uint64_t* fold_hdr, FoldCtl ctl) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const uint32_t hdr0 = FOLD ? fold_epoch(fold_hdr) : 0u;  // fold tag, read ahead of the data
  const int64_t nvec = n / EPV;
  const int64_t base = (int64_t)blockIdx.x * (kRedBlock * U) + tid;
  uint4 r[U][K];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + u * kRedBlock < nvec) {
#pragma unroll
      for (int k = 0; k < K; ++k) r[u][k] = ld_stream(reinterpret_cast<const uint4*>(a.p[k]) + base + u * kRedBlock);
    }
  T acc_e[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc_e[e] = id;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + u * kRedBlock < nvec) {
      T x[K][EPV];
#pragma unroll
      for (int k = 0; k < K; ++k) __builtin_memcpy(x[k], &r[u][k], 16);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        T v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] = x[k][e];
        acc_e[e] = Op::combine(acc_e[e], apply_k<M, T, K>(v));
      }
    }
  T acc = acc_e[0];
#pragma unroll
  for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, acc_e[e]);
  if (blockIdx.x == 0 && nvec * EPV + tid < n) {
    T v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = a.p[k][nvec * EPV + tid];
    acc = Op::combine(acc, apply_k<M, T, K>(v));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if constexpr (!FOLD) {
    if (tid == 0) out[blockIdx.x] = part;
  } else {
    fold_partial<T, Op>(part, out, fold_hdr, s_wave, hdr0, ctl);  // out is the result
  }
}

// Persistent multi-array reduction for large operands (K x 16-byte vectors
// of kChunkMinVecs or more): kFoldMax workgroups, workgroup b folding the
// contiguous chunk [b*chunk, (b+1)*chunk) of vectors of every array with U
// loads per array in flight per lane, then the in-kernel fold, as
// reduce_chunk_kernel does for one array. The host makes `chunk` a whole
// number of U * kRedBlock-vector rounds.
template <class T, class Op, class M, int K, int U>
__global__ __launch_bounds__(kRedBlock) void reducek_chunk_kernel(Operands<T, K> a, int64_t n, int64_t chunk, T* out,
                                                                  uint64_t* fold_hdr, FoldCtl ctl) {
  constexpr int EPV = 16 / (int)sizeof(T);
  __shared__ T s_wave[kRedWaves];
  const T id = Op::template identity<T>();
  const int tid = threadIdx.x;
  const uint32_t hdr0 = fold_epoch(fold_hdr);  // fold tag, read ahead of the data
  const int64_t nvec = n / EPV;
  const int64_t b0 = (int64_t)blockIdx.x * chunk;
  const int64_t b1 = kmin<int64_t>(nvec, b0 + chunk);
  T acc_e[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc_e[e] = id;
  auto fold = [&](const uint4 (&rv)[K]) {
    T x[K][EPV];
#pragma unroll
    for (int k = 0; k < K; ++k) __builtin_memcpy(x[k], &rv[k], 16);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      T v[K];
#pragma unroll
      for (int k = 0; k < K; ++k) v[k] = x[k][e];
      acc_e[e] = Op::combine(acc_e[e], apply_k<M, T, K>(v));
    }
  };
  int64_t i = b0 + tid;
  for (; i + (int64_t)(U - 1) * kRedBlock < b1; i += (int64_t)U * kRedBlock) {
    uint4 r[U][K];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int k = 0; k < K; ++k) r[u][k] = ld_stream(reinterpret_cast<const uint4*>(a.p[k]) + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < U; ++u) fold(r[u]);
  }
  if (i < b1) {  // the partial last round
    uint4 r[U][K];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * kRedBlock < b1) {
#pragma unroll
        for (int k = 0; k < K; ++k) r[u][k] = ld_stream(reinterpret_cast<const uint4*>(a.p[k]) + i + u * kRedBlock);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * kRedBlock < b1) fold(r[u]);
  }
  T acc = acc_e[0];
#pragma unroll
  for (int e = 1; e < EPV; ++e) acc = Op::combine(acc, acc_e[e]);
  if (blockIdx.x == 0 && nvec * EPV + tid < n) {
    T v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = a.p[k][nvec * EPV + tid];
    acc = Op::combine(acc, apply_k<M, T, K>(v));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  fold_partial<T, Op>(part, out, fold_hdr, s_wave, hdr0, ctl);
}

// Multi-array reduction, strided operands: grid-stride loop.
template <class T, class Op, class M, int K>
__global__ __launch_bounds__(kRedBlock) void reducek_kernel(Operands<T, K> a, int64_t n, T* out) {
  __shared__ T s_wave[kRedWaves];
  T acc = Op::template identity<T>();
  const int64_t gsize = (int64_t)gridDim.x * kRedBlock;
  for (int64_t i = (int64_t)blockIdx.x * kRedBlock + threadIdx.x; i < n; i += gsize) {
    T v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = a.p[k][i * a.s[k]];
    acc = Op::combine(acc, apply_k<M, T, K>(v));
  }
  const T part = block_reduce<T, Op>(acc, s_wave);
  if (threadIdx.x == 0) out[blockIdx.x] = part;
}

template <class T, class Op, class M, int K>
int launch_reducek(const Operands<T, K>& a, int64_t n, void* dst, void* scratch_base, hipStream_t stream) {
  constexpr int EPV = 16 / (int)sizeof(T);
  void* scratch = red_work(scratch_base);
  bool vec = true;
  for (int k = 0; k < K; ++k) vec = vec && a.s[k] == 1 && (uintptr_t)a.p[k] % 16 == 0;
  if (!vec) {
    const int grid = reduce_grid<T>(n);
    T* out = grid == 1 ? (T*)dst : (T*)scratch;
    hipLaunchKernelGGL((reducek_kernel<T, Op, M, K>), dim3(grid), dim3(kRedBlock), 0, stream, a, n, out);
    if (grid > 1)
      hipLaunchKernelGGL((combine_all_kernel<T, Op>), dim3(1), dim3(kCombineBlock), 0, stream,
                         (const T*)scratch, grid, (T*)dst);
    return kf_check_launch("reducek_kernel");
  }
  // Loads in flight per lane and array: 8 (three arrays at 4 per array:
  // x*y*z Float64 2^27 464.8 against 460.6 us, Float32 10^7 21.6 against
  // 20.8; two arrays at 16: no gain). From 1 GiB of operands the
  // persistent chunk kernel, below it the one-shot kernel with the fewest
  // loads per lane that fold in one launch, else two levels. Measured on
  // MI355X (HIP graphs, us, two levels -> this): dot products Float32 2^28
  // 314.9 -> 308.3, Float64 2^27 326.2 -> 320.2; x*y*z Float32 2^28 483.3 ->
  // 462.9, 10^8 182.0 -> 174.9, Float64 2^27 482.0 -> 461.6 (the Float32 10^8
  // dot product, 800 MB, stays on two levels: 120.4 against 123.1 chunked).
  constexpr int KU = 8;
  const int64_t nvec = n / EPV;
  if (nvec * K >= 4 * kChunkMinVecs) {
    constexpr int64_t kRound = (int64_t)KU * kRedBlock;
    const int64_t chunk = ((nvec + kFoldMax - 1) / kFoldMax + kRound - 1) / kRound * kRound;
    hipLaunchKernelGGL((reducek_chunk_kernel<T, Op, M, K, KU>), dim3(kFoldMax), dim3(kRedBlock), 0, stream, a, n,
                       chunk, (T*)dst, (uint64_t*)scratch_base, fold_ctl());
    return kf_check_launch("reducek_chunk_kernel");
  }
  const OnceLevels L = once_levels(nvec, EPV, /*adaptive=*/true, KU);
  if (L.nlev == 1 && L.count[0] > 1) {
    // the kernel's loads per lane must be the width the grid was sized for
    static_assert(KU == 8, "one-shot widths compiled below: 2, 4, 8");
    const dim3 grid((unsigned)L.count[0]);
    if (L.u0 == 8)
      hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K, true, 8>), grid, dim3(kRedBlock), 0, stream, a, n,
                         (T*)dst, (uint64_t*)scratch_base, fold_ctl());
    else if (L.u0 == 4)
      hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K, true, 4>), grid, dim3(kRedBlock), 0, stream, a, n,
                         (T*)dst, (uint64_t*)scratch_base, fold_ctl());
    else if (L.u0 == 2)
      hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K, true, 2>), grid, dim3(kRedBlock), 0, stream, a, n,
                         (T*)dst, (uint64_t*)scratch_base, fold_ctl());
    else
      return kf_set_error(KF_EINVAL, "kf_reduce2/3: internal: no kernel of width %d", L.u0);
    return kf_check_launch("reducek_once_kernel");
  }
  size_t abytes = 0;
  for (int i = 0; i < L.nlev; i += 2) abytes = kmax(abytes, round256((size_t)L.count[i] * sizeof(T) + 16));
  T* buf[2] = {(T*)scratch, (T*)((uint8_t*)scratch + abytes)};
  const int last = L.nlev - 1;
  hipLaunchKernelGGL((reducek_once_kernel<T, Op, M, K>), dim3((unsigned)L.count[0]), dim3(kRedBlock), 0, stream,
                     a, n, last == 0 ? (T*)dst : buf[0], (uint64_t*)nullptr, fold_ctl());
  for (int i = 1; i <= last; ++i) {
    const int64_t m = L.count[i - 1];
    const unsigned grid = (unsigned)L.count[i];
    T* out = i == last ? (T*)dst : buf[i % 2];
    if (i == last && grid > 1)
      launch_once<T, Op, MapIdentity, true>(kOnceUnroll, grid, buf[(i - 1) % 2], m, 0, m / EPV, out,
                                            (uint64_t*)scratch_base, stream);
    else
      launch_once<T, Op, MapIdentity, false>(kOnceUnroll, grid, buf[(i - 1) % 2], m, 0, m / EPV, out, nullptr,
                                             stream);
  }
  return kf_check_launch("reducek_once_kernel");
}

template <class T, class Op, class M2>
int launch_reduce2(const void* x, int64_t xs, const void* y, int64_t ys, int64_t n, void* dst, void* scratch,
                   hipStream_t stream) {
  return launch_reducek<T, Op, M2, 2>(Operands<T, 2>{{(const T*)x, (const T*)y}, {xs, ys}}, n, dst, scratch,
                                      stream);
}

template <class T, class Op, class Map> struct ReduceL {
  static int run(const void* src, int64_t n, int64_t stride, void* dst, void* scratch, hipStream_t s) {
    return launch_reduce<T, Op, Map>(src, n, stride, dst, scratch, s);
  }
};
template <class T, class Op, class Map2> struct Reduce2L {
  static int run(const void* x, int64_t xs, const void* y, int64_t ys, int64_t n, void* dst, void* scratch,
                 hipStream_t s) {
    return launch_reduce2<T, Op, Map2>(x, xs, y, ys, n, dst, scratch, s);
  }
};

// ---------------------------------------------------------------------------
// Post-map and scratch fill.
// ---------------------------------------------------------------------------
struct PostSqrt {
  __device__ static float apply(float x) { return __builtin_sqrtf(x); }
  __device__ static double apply(double x) { return __builtin_sqrt(x); }
};
template <class T, class G>
__global__ __launch_bounds__(256) void post_map_kernel(T* x, int64_t n, int64_t stride) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gsize)
    x[i * stride] = G::apply(x[i * stride]);
}

__global__ void fill_zero_kernel(uint8_t* p, int64_t n) {
  const int64_t gsize = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gsize) p[i] = 0;
}

}  // namespace kf

using namespace kf;

extern "C" size_t kf_reduce_scratch_bytes(kf_dtype dt, int64_t n) {
  (void)n;
  size_t es = kf_dtype_size(dt);
  if (es == 0) es = 8;
  return reduce_scratch(es, kmax<int64_t>(n, 1));
}

extern "C" int kf_reduce(kf_op op, kf_map f, kf_dtype dt, const void* src, int64_t n, int64_t stride,
                         void* dst, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce"))) return rc;
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!src || !dst) return kf_set_error(KF_EINVAL, "kf_reduce: null src or dst");
  if (stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce: stride must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)src % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce: src/dst not aligned to the element type");
  const size_t need = kf_reduce_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce: scratch must be 256-byte aligned");
  return dispatch_all<ReduceL>(dt, op, f, src, n, stride, dst, scratch, (hipStream_t)stream);
}

extern "C" size_t kf_reduce2_scratch_bytes(kf_dtype dt, int64_t n) { return kf_reduce_scratch_bytes(dt, n); }

template <class T, class M2, class... A> int dispatch_reduce2_op(kf_op op, A... args) {
  switch (op) {
    case KF_OP_ADD: return Reduce2L<T, OpAdd, M2>::run(args...);
    case KF_OP_MAX: return Reduce2L<T, OpMax, M2>::run(args...);
    case KF_OP_MUL: return Reduce2L<T, OpMul, M2>::run(args...);
    default: return Reduce2L<T, OpMin, M2>::run(args...);
  }
}

template <class T, class... A> int dispatch_reduce2(kf_op op, kf_map2 f, A... args) {
  switch (f) {
    case KF_MAP2_SQDIFF: return dispatch_reduce2_op<T, Map2SqDiff>(op, args...);
    case KF_MAP2_WSQ: return dispatch_reduce2_op<T, Map2WSq>(op, args...);
    case KF_MAP2_EXPDIFF:
      if constexpr (__is_same(T, float) || __is_same(T, double)) return dispatch_reduce2_op<T, Map2ExpDiff>(op, args...);
      return kf_set_error(KF_EINVAL, "kf_reduce2: exp(x - y) needs a floating-point type");
    default: return dispatch_reduce2_op<T, Map2Mul>(op, args...);
  }
}

extern "C" int kf_reduce2(kf_op op, kf_map2 f, kf_dtype dt, const void* x, int64_t x_stride, const void* y,
                          int64_t y_stride, int64_t n, void* dst, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, KF_MAP_IDENTITY, dt, /*allow_affine=*/0);
  if (rc) return rc;
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce2"))) return rc;
  if (f != KF_MAP2_MUL && f != KF_MAP2_SQDIFF && f != KF_MAP2_WSQ && f != KF_MAP2_EXPDIFF)
    return kf_set_error(KF_EINVAL, "kf_reduce2: unknown map %d", (int)f);
  if (f == KF_MAP2_EXPDIFF && dt != KF_F32 && dt != KF_F64)
    return kf_set_error(KF_EINVAL, "kf_reduce2: exp(x - y) needs a floating-point type");
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce2: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!x || !y || !dst) return kf_set_error(KF_EINVAL, "kf_reduce2: null pointer");
  if (x_stride < 1 || y_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce2: strides must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)x % es || (uintptr_t)y % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce2: pointers not aligned to the element type");
  const size_t need = kf_reduce2_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce2: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce2: scratch must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  switch (dt) {
    case KF_F32: return dispatch_reduce2<float>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_F64: return dispatch_reduce2<double>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_I32: return dispatch_reduce2<int32_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_I64: return dispatch_reduce2<int64_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    case KF_U8: return dispatch_reduce2<uint8_t>(op, f, x, x_stride, y, y_stride, n, dst, scratch, s);
    default: return kf_set_error(KF_EINVAL, "kf_reduce2: bad dtype %d", (int)dt);
  }
}

extern "C" size_t kf_reduce3_scratch_bytes(kf_dtype dt, int64_t n) { return kf_reduce_scratch_bytes(dt, n); }

template <class T>
int dispatch_reduce3(kf_op op, const Operands<T, 3>& a, int64_t n, void* dst, void* scratch, hipStream_t s) {
  switch (op) {
    case KF_OP_ADD: return launch_reducek<T, OpAdd, Map3Mul, 3>(a, n, dst, scratch, s);
    case KF_OP_MAX: return launch_reducek<T, OpMax, Map3Mul, 3>(a, n, dst, scratch, s);
    case KF_OP_MUL: return launch_reducek<T, OpMul, Map3Mul, 3>(a, n, dst, scratch, s);
    default: return launch_reducek<T, OpMin, Map3Mul, 3>(a, n, dst, scratch, s);
  }
}

extern "C" int kf_reduce3(kf_op op, kf_map3 f, kf_dtype dt, const void* x, int64_t x_stride, const void* y,
                          int64_t y_stride, const void* z, int64_t z_stride, int64_t n, void* dst, void* scratch,
                          size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, KF_MAP_IDENTITY, dt, /*allow_affine=*/0);
  if (rc) return rc;
  kf_mailbox((hipStream_t)stream);
  if ((rc = kf_take_giveup("kf_reduce3"))) return rc;
  if (f != KF_MAP3_MUL) return kf_set_error(KF_EINVAL, "kf_reduce3: unknown map %d", (int)f);
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce3: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!x || !y || !z || !dst) return kf_set_error(KF_EINVAL, "kf_reduce3: null pointer");
  if (x_stride < 1 || y_stride < 1 || z_stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce3: strides must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)x % es || (uintptr_t)y % es || (uintptr_t)z % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce3: pointers not aligned to the element type");
  const size_t need = kf_reduce3_scratch_bytes(dt, n);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_reduce3: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256) return kf_set_error(KF_EINVAL, "kf_reduce3: scratch must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
#define KF_R3(T) \
  dispatch_reduce3<T>(op, Operands<T, 3>{{(const T*)x, (const T*)y, (const T*)z}, {x_stride, y_stride, z_stride}}, \
                      n, dst, scratch, s)
  switch (dt) {
    case KF_F32: return KF_R3(float);
    case KF_F64: return KF_R3(double);
    case KF_I32: return KF_R3(int32_t);
    case KF_I64: return KF_R3(int64_t);
    case KF_U8: return KF_R3(uint8_t);
    default: return kf_set_error(KF_EINVAL, "kf_reduce3: bad dtype %d", (int)dt);
  }
#undef KF_R3
}

template <class T, class G> int launch_post(void* x, int64_t n, int64_t stride, hipStream_t s) {
  const int grid = (int)kmin<int64_t>(8192, kmax<int64_t>(1, (n + 255) / 256));
  hipLaunchKernelGGL((post_map_kernel<T, G>), dim3(grid), dim3(256), 0, s, (T*)x, n, stride);
  return kf_check_launch("post_map_kernel");
}

extern "C" int kf_post_map(kf_post g, kf_dtype dt, void* x, int64_t n, int64_t stride, void* stream) {
  if (g == KF_POST_IDENTITY || n == 0) return KF_OK;
  if (n < 0 || stride < 1) return kf_set_error(KF_EINVAL, "kf_post_map: bad n or stride");
  if (!x) return kf_set_error(KF_EINVAL, "kf_post_map: null pointer");
  const size_t es = kf_dtype_size(dt);
  if (es == 0 || dt == KF_F32X2) return kf_set_error(KF_EINVAL, "kf_post_map: unsupported dtype %d", (int)dt);
  if ((uintptr_t)x % es) return kf_set_error(KF_EINVAL, "kf_post_map: pointer not aligned to the element type");
  hipStream_t s = (hipStream_t)stream;
  if (g == KF_POST_SQRT) {
    if (dt == KF_F32) return launch_post<float, PostSqrt>(x, n, stride, s);
    if (dt == KF_F64) return launch_post<double, PostSqrt>(x, n, stride, s);
    return kf_set_error(KF_EINVAL, "kf_post_map: sqrt needs a floating-point type");
  }
  if (g == KF_POST_ABS2) {
    switch (dt) {
      case KF_F32: return launch_post<float, MapAbs2>(x, n, stride, s);
      case KF_F64: return launch_post<double, MapAbs2>(x, n, stride, s);
      case KF_I32: return launch_post<int32_t, MapAbs2>(x, n, stride, s);
      case KF_I64: return launch_post<int64_t, MapAbs2>(x, n, stride, s);
      default: return launch_post<uint8_t, MapAbs2>(x, n, stride, s);
    }
  }
  return kf_set_error(KF_EINVAL, "kf_post_map: unknown post-map %d", (int)g);
}

extern "C" int kf_scratch_reset(void* scratch, size_t bytes, void* stream) {
  if (bytes == 0) return KF_OK;
  if (!scratch) return kf_set_error(KF_EINVAL, "kf_scratch_reset: null scratch");
  const int grid = (int)kmin<int64_t>(1024, kmax<int64_t>(1, ((int64_t)bytes + 255) / 256));
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (uint8_t*)scratch,
                     (int64_t)bytes);
  return kf_check_launch("fill_zero_kernel");
}

namespace kf {
__global__ void clear_fold_flag_kernel(uint64_t* hdr) { hdr[1] = 0; }
}  // namespace kf

extern "C" int kf_reduce_scratch_status(void* scratch, void* stream, int* gave_up) {
  if (!scratch || !gave_up) return kf_set_error(KF_EINVAL, "kf_reduce_scratch_status: null pointer");
  hipStream_t s = (hipStream_t)stream;
  uint64_t w = 0;
  if (hipMemcpyAsync(&w, (uint64_t*)scratch + 1, sizeof w, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return kf_check_launch("kf_reduce_scratch_status");
  *gave_up = w != 0;
  // the epoch already moved past the failed call's slots; only the flag is
  // cleared (a kernel, not a memset node: the call may sit in a graph)
  if (w != 0) hipLaunchKernelGGL(clear_fold_flag_kernel, dim3(1), dim3(1), 0, s, (uint64_t*)scratch);
  return kf_check_launch("clear_fold_flag_kernel");
}

#ifdef KF_TIMELINE
extern "C" int kf_debug_reduce_timeline(void* buf) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_red_timeline), &buf, sizeof(buf)) != hipSuccess)
    return kf_check_launch("kf_debug_reduce_timeline");
  return KF_OK;
}

extern "C" int kf_debug_reduce_giveup(int workgroup, uint32_t spin_limit) {
  if (workgroup < 0) {
    g_fold_withhold = -1;
    g_fold_limit = kFoldSpinLimit;
    return KF_OK;
  }
  if (spin_limit == 0) return kf_set_error(KF_EINVAL, "kf_debug_reduce_giveup: spin_limit must be > 0");
  g_fold_withhold = workgroup;
  g_fold_limit = spin_limit;
  return KF_OK;
}
#endif

// ---------------------------------------------------------------------------
// Allocation-free full reduction: kf_reduce with its scratch in a static
// device array instead of a caller buffer.
// ---------------------------------------------------------------------------
namespace kf {
constexpr size_t kStaticScratchBytes = KF_NOALLOC_SCRATCH_BYTES;
}  // namespace kf

// One copy per GPU, alive until the process ends. Zero at load (static
// storage), which is the initial state the epoch-tagged fold slots need;
// after that the kernels keep it valid. In host code this name is only a
// stand-in for the symbol: the device address comes from
// hipGetSymbolAddress (static_scratch_ptr below).
static __device__ __align__(256) uint8_t scratch[kf::kStaticScratchBytes];

namespace {
constexpr int kMaxStaticDevices = 64;
std::mutex g_static_mu;
void* g_static_ptr[kMaxStaticDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device with that device current.
int static_scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxStaticDevices)
    return kf_set_error(KF_EHIP, "kf_reduce_noalloc: no current HIP device (or device id >= %d)", kMaxStaticDevices);
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (!g_static_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return kf_set_error(KF_EHIP, "kf_reduce_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_static_ptr[dev] = p;
  }
  *out = g_static_ptr[dev];
  return KF_OK;
}
}  // namespace

extern "C" int kf_reduce_noalloc(kf_op op, kf_map f, kf_dtype dt, const void* src, int64_t n, int64_t stride,
                                 void* dst, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/0);
  if (rc) return rc;
  if ((rc = kf_take_giveup("kf_reduce_noalloc"))) return rc;
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_reduce_noalloc: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!src || !dst) return kf_set_error(KF_EINVAL, "kf_reduce_noalloc: null src or dst");
  if (stride < 1) return kf_set_error(KF_EINVAL, "kf_reduce_noalloc: stride must be >= 1");
  const size_t es = kf_dtype_size(dt);
  if ((uintptr_t)src % es || (uintptr_t)dst % es)
    return kf_set_error(KF_EINVAL, "kf_reduce_noalloc: src/dst not aligned to the element type");
  const size_t need = kf_reduce_scratch_bytes(dt, n);
  if (need > kStaticScratchBytes)
    return kf_set_error(KF_EINVAL,
                        "kf_reduce_noalloc: n = %lld needs %zu bytes of scratch, more than the static %zu; "
                        "use kf_reduce with a caller buffer",
                        (long long)n, need, kStaticScratchBytes);
  void* p = nullptr;
  rc = static_scratch_ptr(&p);
  if (rc) return rc;
  return dispatch_all<ReduceL>(dt, op, f, src, n, stride, dst, p, (hipStream_t)stream);
}
