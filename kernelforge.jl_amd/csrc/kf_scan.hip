// Single-pass decoupled-lookback prefix scan for gfx950.
//
// Follows the algorithm of the reference's scan_kernel_packed! /
// scan_kernel! (reference src/scan/scan_kernel.jl:94-478): per-tile
// thread/wave/block scan, publish the tile aggregate (PARTIAL), look back
// over predecessor descriptors until an inclusive prefix (PREFIX) is found,
// publish the tile's own PREFIX, apply the prefix and store. The MI355X
// design differs from the reference in these ways:
//
//  * Large tiles: 8 16-byte vectors per lane x 1024 threads = 128 KiB (768
//    threads = 96 KiB for 4- and 8-byte types from 17 MiB on; 512 threads
//    x 8/12/16 vectors for UInt8; 2 or 4 vectors per lane for arrays too
//    small to make 160 such tiles), so 2^28 Float32 is 10923 tiles and the
//    per-tile lookback is amortised over a large streaming body. The tile
//    stays in registers in "striped" order: lane l of wave w holds vector
//    j*64 + l of the wave's contiguous chunk, so every load and store is a
//    fully coalesced 16-byte access and no LDS transpose is needed. Each
//    row j (64 lanes x 16 bytes) is scanned in-lane, then across the wave
//    with DPP row shifts/broadcasts, and rows are chained with a carry (the
//    affine pairs instead scan all row totals once through LDS,
//    wave_row_prefixes). A lane's unit is one 16-byte vector, or one element
//    for wider types (32-byte Float64 quaternions, moved as two halves).
//  * The lookback window lives in the top lanes of one wave: lane j reads
//    the descriptor of tile (t - 64 + j) for the last `win` lanes, so
//    lane order is tile order and a DPP scan combines the window in the
//    order a non-commutative op needs (lookback_all, for fully resident
//    grids, gives each lane a contiguous chunk of predecessors instead, and
//    for up to 2 * BLOCK + 1 resident tiles every wave of the workgroup
//    reads a share, the waves' folds combined through LDS).
//  * Each tile descriptor owns a 128-byte line (kDescWords words): tiles are
//    published from different XCDs, and packing several descriptors per line
//    made those writers and the pollers contend for one line (measured: 5.0
//    vs 5.8 TB/s for Float32 at 2^28).
//  * A descriptor is W 64-bit words (W = sizeof(T)/4, at least 1). Every
//    word carries a 32-bit tag {epoch:30, state:2} next to 32 bits of the
//    value, written and read with relaxed device-scope atomics: a reader
//    either sees all W words with one tag (a consistent value) or retries,
//    so no fences are needed for any element size (the reference uses one
//    packed word for <= 4-byte types and a split flag/partial layout with
//    fences otherwise, scan_kernel.jl:24-58, :94-299).
//  * Tiles are numbered by workgroup id. An atomic ticket per tile, the
//    usual way to number tiles in start order, serialised on its one
//    address (15-30 ns per ticket) and throttled the whole grid (2^28
//    Float32 337 -> 321 us, Float64 2^27 347 -> 324 us, 10^7 UInt8 16.3 ->
//    9.7 us without it). Waiting on lower-numbered tiles stays deadlock-free
//    because each XCD dispatches its workgroups in increasing id order: the
//    lowest tile not yet started only waits for a slot on its XCD, whose
//    resident tiles are all lower, depend only on tiles that already
//    started, and so finish. The bounded lookback spin (give-up flag) stays
//    as the backstop.
//  * The epoch lives in the scratch header (word 0, high half). Every tile
//    reads it with a plain load at its start, and the last tile advances it
//    once its lookback has completed, which needs every lower tile to have
//    published and so to have read it already. Descriptors of earlier calls
//    carry older epochs and read as INVALID, so the scratch buffer needs no
//    clearing between calls (the reference fill!s its descriptors before
//    every launch, src/scan/scan.jl:444-470).
#include <atomic>
#include <cmath>
#include <type_traits>

#include "kf_common.h"

#ifdef KF_TIMELINE
// Instrumented build only (build.py --timeline -> libkfhip_timeline.so):
// every tile records, by thread 0, four 100 MHz realtime stamps (start,
// tile scanned, prefix known, stores issued), its XCD and its HW_ID word
// into kKfTimelineWords words at g_scan_timeline + tile * kKfTimelineWords.
__device__ uint64_t* g_scan_timeline = nullptr;
constexpr int kKfTimelineWords = 6;
#endif

namespace kf {

constexpr int kScanBlock = 1024;       // large tiles (default)
// Tile shapes: 1024 threads x kTierV[t] 16-byte vectors per lane (32 KiB
// to 128 KiB; 512 threads for UInt8). An array takes the largest shape that
// still cuts it into at least min_tiles() tiles (scan_tier), but never fewer
// than 2 vectors per lane (UInt8: 1). Measured on MI355X with tiles
// numbered by workgroup id: 240 tiles rather than 120 gives Float32 2^21
// 7.68 -> 6.80 us, 2*10^6 7.55 -> 7.04 us, 4*10^6 10.4 -> 8.8 us, 10^6 6.06
// -> 6.16 us. Letting 10^6 drop to 16 KiB tiles to reach 240 cost 9 %,
// hence the floor. A later sweep with every shape forced in turn (the
// launch-shape keywords) lowered the minimum to 160: Float32 3.5*10^6
// 8.8 -> 8.1 us, Float64 1.6*10^6 10.2 -> 9.4 us (Float32 2.5*10^6 tied,
// Int32 3*10^6 8.2 -> 8.6 us the one loss).
// Threads per tile by element type (2^28 Float32 / Int32, 2^27 Float64,
// 2^26 affine pairs, 2^30 UInt8 over 512, 768 and 1024): UInt8 (16
// elements per vector, long in-tile work) gains most from co-resident
// workgroups, one computing while another streams (512: 5.74 vs 5.43 TB/s
// at 1024). Large Float32, Int32 and 8-byte arrays take 768-thread tiles,
// two workgroups per CU (the 8-byte types once wave 0 parks its tile in LDS
// during the lookback): Float32 2^28 320 vs 329 us at 1024, Int32 322 vs
// 335 us, Float64 2^27 324 vs 353 us.
constexpr int kTiers = 4;
constexpr int kTierV[kTiers] = {1, 2, 4, 8};
constexpr int64_t kMinTiles = 160;
// UInt8 tiles carry 4x the elements per byte of work: they need more tiles
// (480) before a larger shape pays (10^7 9.7 us at 480, 10.7 at 240, 18.2
// at 960).
// Quaternion tiles carry about three Hamilton products per element of
// in-tile work, so fewer, longer tiles pay off sooner: QuaternionF32 takes
// 1024 x 4 from 64 tiles (HIP graphs, us, 1024 x 2 -> 1024 x 4: 4*10^5
// 12.1 -> 11.4, 6*10^5 13.9 -> 12.4; 2*10^5 9.9 vs 9.8).
template <class T> constexpr int64_t min_tiles() { return sizeof(T) == 1 ? 480 : is_quat<T> ? 64 : kMinTiles; }
template <class T> constexpr int kMinTier = sizeof(T) == 1 ? 0 : 1;
// Arrays of at least kWideBytes take a wider shape: the 4- and 8-byte
// types 768 threads x 8 vectors (96 KiB); UInt8 (from kU8WideBytes) 512
// threads x 12 vectors (96 KiB), and from kHugeBytes on 512 x 16 (128 KiB). The UInt8 shapes
// halve or third the lookbacks per byte and still fit two workgroups per
// CU (96 and 120 VGPRs): 6*10^8 214 -> 207 us, 8*10^8 279 -> 269 us,
// 10^9 343 -> 329 us at 12; 2^30 361 -> 341 us, 2^31 702 -> 657 us at 16,
// where 12 gives 350 / 673 (20 and 24 vectors lose 8-10 %; at 32 the
// compiler no longer keeps the tile in registers).
// The 4- and 8-byte types take it from 17 MiB, where two co-resident 96 KiB
// tiles per CU balance the last round of tiles better than one 128 KiB tile
// (HIP graphs, us, 1024 x 8 -> 768 x 8): Float32 6*10^6 11.3 -> 9.9, 10^7
// 16.4 -> 14.6, 10^8 124.3 -> 122.7; Float64 6*10^6 24.6 -> 17.9, 10^7
// 35.6 -> 31.5, 2*10^7 64.5 -> 55.1, 5*10^7 142.0 -> 125.4; affine pairs
// 5*10^6 21.5 -> 17.0, 5*10^7 141.8 -> 125.6. Worst case Float32 2*10^7
// 29.7 -> 30.6. The forced-shape sweep moved the threshold from 20 down to
// 17 MiB: at 18 MiB Float32 9.6 -> 9.5 us, Int32 9.9 -> 9.2, Float64 and
// Int64 11.0 -> 10.9, affine pairs 10.6 -> 10.3 (Float32 5.2*10^6 10.4 ->
// 9.7); at 16 MiB the 1024-thread tiles are still 2-7 % ahead.
constexpr int64_t kWideBytes = 17LL << 20;
constexpr int64_t kHugeBytes = 1LL << 30;
// UInt8 takes the 12-vector shape from 384 MiB (forced-shape sweep: 3*10^8
// 106.5 us at 8 vectors vs 107.8 at 12, 3.5-4*10^8 tied, 4.5*10^8 153.7 vs
// 152.3, 5*10^8 169.7 vs 167.3).
constexpr int64_t kU8WideBytes = 384LL << 20;
constexpr int kTierWide = kTiers;      // tier index of the wide shape
constexpr int kTierHuge = kTiers + 1;  // UInt8 from kHugeBytes
template <class T> constexpr bool has_wide_tier() {
  return sizeof(T) == 4 || sizeof(T) == 8 || sizeof(T) == 1 || is_quat<T>;
}
// Quaternions take a wide shape of longer lane chunks from kWideBytes on:
// QuaternionF32 768 threads x 8 units (96 KiB), QuaternionF64 1024 x 8
// units (256 KiB, one workgroup per CU at 128 VGPRs). More units per lane spread the wave scan's six combines
// and the prefix combine over more elements (about 2.9 Hamilton products
// per element at 8 units, 3.75 at 4). Measured on MI355X (HIP graphs, us;
// tiles through the LDS transpose below): QuaternionF32 at 768 x 8 vs 1024
// x 4: 2*10^6 18.5 vs 19.6, 4*10^6 32.6 vs 33.6, 2^23 57.3 vs 61.8, 2^24
// 103.0 vs 115.0, 2^26 377.1 vs 434.7 (512 x 16 378, 768 x 16 402);
// QuaternionF64 at 1024 x 4 vs 1024 x 2: 10^6 28.4 vs 32.9, 2^22 87.4 vs
// 114.0, 2^24 335.4 vs 430.9 (512 x 4 349, 768 x 4 346, 512 x 8 341).
// With granule-striped loads and stores (below), QuaternionF64 at 1024 x 8
// / 768 x 8 / 1024 x 4 / 512 x 8: 10^6 23.1 / 22.8 / 23.1 / 22.6, 2^22
// 62.0 / 67.2 / 71.9 / 72.6, 2^24 220.1 / 229.3 / 288.2 / 290.6, 2^25
// 423.1 / 438.7 / 562.1 / 568.2. (Before
// the transpose, with blocked loads and stores, QuaternionF32 2^26 took
// 588.7 us at 1024 x 4 and 549.3 at 768 x 8.)
constexpr int kWideBlockQ32 = 768, kWideVQ32 = 8, kWideBlockQ64 = 1024, kWideVQ64 = 8;
template <class T> constexpr bool has_huge_tier() { return sizeof(T) == 1; }
// (Float32 and the 8-byte types measured 0.5-10 % slower at 512 x 12 or 16.)
constexpr int kWideBlockF32 = 768, kWideVF32 = 8, kWideBlock8 = 768, kWideV8 = 8;
template <class T> constexpr int scan_block(int tier) {
  if (is_quat<T> && tier == kTierWide) return sizeof(T) == 16 ? kWideBlockQ32 : kWideBlockQ64;
  if (sizeof(T) == 1) return 512;
  if (tier != kTierWide) return kScanBlock;
  return sizeof(T) == 4 ? kWideBlockF32 : kWideBlock8;
}
template <class T> constexpr int tier_v(int tier) {
  if (is_quat<T> && tier == kTierWide) return sizeof(T) == 16 ? kWideVQ32 : kWideVQ64;
  if (tier == kTierHuge) return 16;
  if (tier != kTierWide) return kTierV[tier];
  return sizeof(T) == 1 ? 12 : sizeof(T) == 4 ? kWideVF32 : kWideV8;
}
constexpr uint32_t kStatePartial = 1, kStatePrefix = 2;
constexpr size_t kScanHeaderBytes = 256;
constexpr int kDescWords = 16;             // 128 bytes per tile descriptor
constexpr uint32_t kSpinLimit = 1u << 24;  // lookback polls before giving up (seconds)
constexpr uint32_t kFlagPollMask = 1023;   // a waiting lookback re-reads the give-up flag every 1024 polls
// Predecessors polled per lookback round (lanes 64-win..63). Each
// descriptor is its own 128-byte line and a poll completes only when its
// slowest line returns, while in the steady state of a long scan (more
// tiles than fit on the GPU at once) the nearest predecessors mostly hold
// PREFIX already: the larger the tile, the fewer lines a poll needs.
// Measured with tiles numbered by workgroup id: 96 KiB tiles 4 (2^28
// Float32 320 us; 2: 330, 8: 333); 128 KiB tiles over 4+ generations 2
// (Float32 10^8 126.7 vs 129.6 us at 4); tiles of 64 KiB or less 8 (UInt8
// 10^8 40.9 vs 41.7 us). When every tile is resident at once they all
// publish PARTIAL together and walk back towards tile 0, and the full
// 64-tile window is faster.
// Grids of at most kWave * kAllChunk + 1 tiles, all resident at once, read
// every predecessor in one poll round (lookback_all, window code 0) instead
// of walking back one 64-tile window per round: Float32 10^6 6.09 -> 5.72
// us, 2*10^6 7.03 -> 6.70 us, 2^21 6.90 -> 6.53 us, affine 2^22 13.6 ->
// 13.2 us. Only for types of up to 4 bytes: the 8-byte types lost 1-3 %
// from the extra registers (Float64 10^6 8.41 -> 8.70 us), and a chunk of
// 8 lost 5 % at 10^7 Float32.
constexpr int kAllChunk = 4;
template <class T> constexpr bool kLookAllFor = sizeof(T) <= 4;
// Grids of up to BLOCK * kBlockChunk + 1 tiles, all resident, let every
// wave of the workgroup read a share of the predecessors (window code -1):
// one poll round where lookback_all does not apply (more than 257 tiles,
// or 8-byte types, which keep its registers out of their kernels).
// Measured with HIP graphs, us, 64-tile window -> whole workgroup: UInt8
// 3*10^6 7.2 -> 6.5, 5*10^6 8.5 -> 7.5, 10^7 9.9 -> 9.0; Float64 10^6 8.9 ->
// 8.1, 1.6*10^6 10.1 -> 9.4; affine pairs 10^6 9.0 -> 8.2; Float32 2*10^6
// 7.3 -> 7.0. Only for tiles of at most 2 vectors per lane (4 for the
// 8-byte types): 4-vector UInt8 tiles lost 7 % (2*10^7 13.2 -> 14.1 us,
// 3*10^7 16.0 -> 17.1), their longer loads overlapping more of the
// workgroup-wide polling.
constexpr int kBlockChunk = 2;
template <class T, int BLOCK, int VPL>
constexpr bool kLookBlockFor = sizeof(T) <= 8 && VPL <= (sizeof(T) == 8 ? 4 : 2);
// For grids of several generations the window code also carries, in its
// bits from 8 on, the number of tiles resident from the start (the first
// generation), for the staggered start below.
inline int look_window(int64_t ntiles, int64_t resident, int64_t tile_bytes, bool look_all, bool look_block,
                       int block) {
  if (ntiles <= resident) {
    if (look_all && ntiles <= (int64_t)kWave * kAllChunk + 1) return 0;
    if (look_block && ntiles <= (int64_t)block * kBlockChunk + 1) return -1;
    return kWave;
  }
  const int gen1 = (int)kmin<int64_t>(resident, 1 << 22) << 8;
  if (tile_bytes >= (128 << 10) && ntiles > 4 * resident) return 2 | gen1;
  if (tile_bytes <= (64 << 10)) return 8 | gen1;
  return 4 | gen1;
}
__device__ inline int window_of(int win) { return win > 0 ? (win & 0xff) : win; }

// Staggered start of the first generation: tile t of the R tiles resident
// from the start waits t/R x kFirstGenStaggerNs before its loads. All R
// tiles loading at once finish together, and the PREFIX front then walks
// through them (a tile of the first generation sees only tile 0's PREFIX
// and the others' PARTIALs), so the first stores start about one tile life
// late; spread out, the low tiles finish loading first and the front
// follows them. Measured on MI355X (median of 9 HIP graphs, us, as before /
// spread over 3, 4, 6 us): Float32 2^28 320.6 / 319.8 / 319.9 / 319.3,
// 10^8 124.5 / 123.8 / 123.8 / 123.2, 2.5*10^7 37.0 / 36.2 / 36.1 / 35.9;
// affine 2^26 167.9 / 167.7 / 167.5 / 167.3; QuaternionF64 2^24 220.4 /
// 219.1 / 218.0 / 217.0; UInt8 10^8 40.6 / 40.3 / 40.5 / 40.6 (8 us: 42.0).
// Grids of a single generation are not staggered: their last tile ends one
// load, one poll round trip and one store after the last load starts, and
// any delay adds to it (0.5 / 1 us spread: Float32 10^6 5.05 -> 5.61 / 6.19
// us, UInt8 10^7 8.41 -> 9.08 / 9.73).
constexpr uint64_t kFirstGenStaggerNs = 6000;
__device__ inline void first_gen_stagger(int win, int64_t tile) {
  const int64_t gen1 = win > 0 ? (int64_t)(win >> 8) : 0;
  if (tile >= gen1) return;
  const uint64_t ticks = (uint64_t)tile * (kFirstGenStaggerNs / 10) / (uint64_t)gen1;  // 100 MHz counter
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(4);
}

// The unit a lane loads and stores: 16 bytes, or one element of a wider
// type (a 32-byte QuaternionF64 moves as two 16-byte halves).
template <class T> constexpr int kVecBytes = sizeof(T) > 16 ? (int)sizeof(T) : 16;
struct uint4x2 {
  uint4 lo, hi;
};
template <class T> using VecT = std::conditional_t<(sizeof(T) > 16), uint4x2, uint4>;
// Loads of a source vector at any element-aligned address: the byte-aligned
// vector type still compiles to one global_load_dwordx4 (gfx950 serves
// unaligned global accesses), so a source that is misaligned differently
// from the destination streams as well (the tiles follow the destination's
// alignment, which keeps every store a whole aligned vector).
typedef uint32_t v4u32_u __attribute__((ext_vector_type(4), aligned(1)));
__device__ inline uint4 ld_stream_u(const void* p) {
  const v4u32_u v = __builtin_nontemporal_load(reinterpret_cast<const v4u32_u*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ inline uint4 ld_vec(const uint4* p) { return ld_stream_u(p); }
__device__ inline uint4x2 ld_vec(const uint4x2* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  return uint4x2{ld_stream_u(q), ld_stream_u(q + 1)};
}
__device__ inline void st_vec(uint4* p, uint4 v) { st_stream(p, v); }
// Cached (temporal) accesses of a whole unit, for the blocked layout, where
// one instruction touches every V-th unit and the lane's next instruction
// the units between: the line must stay in the cache in between.
__device__ inline uint4x2 ld_unit_cached(const uint4x2* p) { return *p; }
__device__ inline uint4 ld_unit_cached(const uint4* p) { return *p; }
__device__ inline void st_unit_cached(uint4x2* p, uint4x2 v) { *p = v; }
__device__ inline void st_unit_cached(uint4* p, uint4 v) { *p = v; }
__device__ inline void st_vec(uint4x2* p, uint4x2 v) {
  uint4* q = reinterpret_cast<uint4*>(p);
  st_stream(q, v.lo);
  st_stream(q + 1, v.hi);
}

template <class T, int BLOCK = kScanBlock, int VPL = 8> struct ScanShape {
  static constexpr int EPV = kVecBytes<T> / (int)sizeof(T);  // elements per vector
  static constexpr int V = VPL;                     // vectors per lane
  static constexpr int WAVE_ELEMS = kWave * V * EPV;
  static constexpr int TILE = BLOCK * V * EPV;
  static constexpr int W = Words<T>::W;
};

template <class T>
__device__ inline void publish(uint64_t* desc, int64_t tile, uint32_t tag, T v) {
  const Words<T> w = to_words(v);
#pragma unroll
  for (int i = 0; i < ScanShape<T>::W; ++i)
    st_agent(desc + tile * kDescWords + i, ((uint64_t)tag << 32) | w.w[i]);
}

// Give-up flag: header word 1. A lookback that has polled `limit` times
// without finding its prefix sets it and stops; so does one that sees it
// set (it re-reads it every kFlagPollMask + 1 polls), so that one give-up
// ends every waiting tile of the grid quickly.
__device__ inline uint64_t* giveup_flag(const uint64_t* desc) {
  return const_cast<uint64_t*>(desc) - kScanHeaderBytes / sizeof(uint64_t) + 1;
}
__device__ inline bool lookback_stop(const uint64_t* desc, uint32_t polls, uint32_t limit) {
  if (polls >= limit) {
    __hip_atomic_fetch_or(giveup_flag(desc), (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  if ((polls & kFlagPollMask) != kFlagPollMask) return false;
  const uint64_t f = ld_agent(giveup_flag(desc));
  return __builtin_amdgcn_readfirstlane((uint32_t)(f | (f >> 32))) != 0;  // wave-uniform
}

// Decoupled lookback, executed by one full wave. Returns the combination of
// every tile before `tile` (tile > 0), in tile order; sets gave_up (and
// returns garbage) when it stopped waiting.
template <class T, class Op>
__device__ inline T lookback(const uint64_t* desc, int64_t tile, uint32_t epoch30, int win, uint32_t limit,
                             bool& gave_up) {
  constexpr int W = ScanShape<T>::W;
  const int lane = lane_id();
  const T id = Op::template identity<T>();
  T run = id;
  int64_t newest = tile - 1;  // the window's lane 63
  for (uint32_t polls = 0;; ++polls) {
    if (lookback_stop(desc, polls, limit)) {
      // A predecessor never published: impossible unless tiles were
      // dispatched out of order, the scratch buffer was corrupted or it is
      // shared by overlapping calls. The tile stops (results are invalid).
      gave_up = true;
      return run;
    }
    const int64_t t = newest - (kWave - 1) + lane;
    const bool in_win = lane >= kWave - win;
    T v = id;
    // tiles before 0: an identity prefix; lanes outside the window: identity partials
    uint32_t state = in_win ? kStatePrefix : kStatePartial;
    if (t >= 0 && in_win) {
      uint64_t d[W];
#pragma unroll
      for (int i = 0; i < W; ++i) d[i] = ld_agent(desc + t * kDescWords + i);
      const uint32_t tag = (uint32_t)(d[0] >> 32);
      bool ok = (tag >> 2) == epoch30;
#pragma unroll
      for (int i = 1; i < W; ++i) ok &= (uint32_t)(d[i] >> 32) == tag;
      state = ok ? (tag & 3u) : 0u;
      Words<T> w;
#pragma unroll
      for (int i = 0; i < W; ++i) w.w[i] = (uint32_t)d[i];
      v = from_words<T>(w);
    }
    const uint64_t invalid = __builtin_amdgcn_ballot_w64(state == 0);
    const uint64_t prefix = __builtin_amdgcn_ballot_w64(state == kStatePrefix);
    if (prefix != 0) {
      const int m = 63 - __builtin_clzll(prefix);
      if ((invalid >> m) == 0) {
        const T tot = wave_reduce<Op>(lane >= m ? v : id);
        return Op::combine(tot, run);
      }
    } else if (invalid == 0) {
      const T tot = wave_reduce<Op>(v);
      run = Op::combine(tot, run);
      newest -= win;
      continue;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Lookback when every tile of the grid is resident at once, by P readers
// (one wave: P = 64; the whole workgroup: P = BLOCK): reader `idx` reads the
// descriptors of its contiguous chunk [idx*c, idx*c + c) of all `tile`
// predecessors (c <= CH) with every load in flight together and folds them
// in tile order (restarting at a PREFIX); a reader whose chunk still holds
// an unpublished descriptor re-reads it. Returns, for the calling wave, the
// ordered fold from its newest lane holding a PREFIX (from lane 0 if none
// does) in `out`, and whether any of its lanes holds one.
template <class T, class Op, int CH>
__device__ inline bool lookback_all_wave(const uint64_t* desc, int64_t tile, uint32_t epoch30, uint32_t limit,
                                         bool& gave_up, int64_t idx, int64_t P, T& out) {
  constexpr int W = ScanShape<T>::W;
  const int lane = lane_id();
  const T id = Op::template identity<T>();
  const int64_t c = (tile + P - 1) / P;
  const int64_t t0 = idx * c;
  const int cnt = (int)kmax<int64_t>(0, kmin<int64_t>(c, tile - t0));
  T val = id;
  bool has_prefix = false;
  bool done = cnt == 0;
  for (uint32_t polls = 0;; ++polls) {
    if (lookback_stop(desc, polls, limit)) {
      gave_up = true;
      break;
    }
    if (!done) {
      uint64_t d[CH][W];
#pragma unroll
      for (int k = 0; k < CH; ++k)
        if (k < cnt) {
#pragma unroll
          for (int i = 0; i < W; ++i) d[k][i] = ld_agent(desc + (t0 + k) * kDescWords + i);
        }
      bool ok = true;
      T run = id;
      bool pre = false;
#pragma unroll
      for (int k = 0; k < CH; ++k)
        if (k < cnt) {
          const uint32_t tag = (uint32_t)(d[k][0] >> 32);
          bool good = (tag >> 2) == epoch30 && (tag & 3u) != 0;
#pragma unroll
          for (int i = 1; i < W; ++i) good &= (uint32_t)(d[k][i] >> 32) == tag;
          ok &= good;
          Words<T> w;
#pragma unroll
          for (int i = 0; i < W; ++i) w.w[i] = (uint32_t)d[k][i];
          const T v = from_words<T>(w);
          if ((tag & 3u) == kStatePrefix) {
            run = v;
            pre = true;
          } else {
            run = Op::combine(run, v);
          }
        }
      if (ok) {
        val = run;
        has_prefix = pre;
        done = true;
      }
    }
    if (__builtin_amdgcn_ballot_w64(!done) == 0) break;
    __builtin_amdgcn_s_sleep(1);
  }
  const uint64_t pm = __builtin_amdgcn_ballot_w64(has_prefix);
  const int m = pm ? 63 - __builtin_clzll(pm) : 0;
  out = wave_reduce<Op>(lane >= m ? val : id);
  return pm != 0;
}

// One wave's lookback_all: the exclusive prefix of `tile`.
template <class T, class Op, int CH>
__device__ inline T lookback_all(const uint64_t* desc, int64_t tile, uint32_t epoch30, uint32_t limit,
                                 bool& gave_up) {
  T out;
  lookback_all_wave<T, Op, CH>(desc, tile, epoch30, limit, gave_up, lane_id(), kWave, out);
  return out;
}

// Byte-wise a + b (mod 256 in every byte) of four packed bytes.
__device__ inline uint32_t add_bytes(uint32_t a, uint32_t b) {
  return ((a & 0x7f7f7f7fu) + (b & 0x7f7f7f7fu)) ^ ((a ^ b) & 0x80808080u);
}
// The 16 bytes moved up by one position, a zero byte in front.
__device__ inline uint4 shift_in_byte(uint4 v) {
  return make_uint4(v.x << 8, __builtin_amdgcn_alignbyte(v.y, v.x, 3), __builtin_amdgcn_alignbyte(v.z, v.y, 3),
                    __builtin_amdgcn_alignbyte(v.w, v.z, 3));
}

// Tiles whose wave 0 parks its registers in LDS during the lookback: the
// kernel's VGPR count is the peak over the tile and lookback code, and
// parking lowers it where that buys a second workgroup per CU (8-byte
// types 85 -> 72, 1024-thread Float32 66 -> 58; Float32 at 768 already
// fits two and runs 1 % faster without).
template <class T, int BLOCK> constexpr bool kStashForLookback = sizeof(T) == 8 || (sizeof(T) == 4 && BLOCK == 1024);

// The post-map g on a stored value: sqrt or abs2 for floats, abs2
// (wrapping) for integers; kf_scan rejects anything else.
template <class T> __device__ inline T post_apply(int post, T v) {
  if constexpr (__is_same(T, f32x2) || is_quat<T>) {
    return v;
  } else if constexpr (__is_same(T, float)) {
    // v_sqrt_f32 (within 1 ulp) rather than the correctly rounded
    // expansion: the scanned values themselves carry reassociation error
    // far above 1 ulp, and the expansion's VALU work in the store phase
    // cost 12 % of a 2^28 scan
    return post == KF_POST_SQRT ? __builtin_amdgcn_sqrtf(v) : v * v;
  } else if constexpr (__is_same(T, double)) {
    return post == KF_POST_SQRT ? __builtin_sqrt(v) : v * v;
  } else {
    return MapAbs2::apply(v);
  }
}

template <class T, class Op> __device__ inline T exclusive_first() {
  if constexpr (__is_same(Op, OpAdd) && (__is_same(T, float) || __is_same(T, double)))
    return T(0);  // +0.0, as Julia / CUB produce for the first exclusive sum
  else
    return Op::template identity<T>();
}

// For sub-dword T, make the packed dwords of a vector the only live copy at
// this point; the compiler would otherwise keep all V*EPV unpacked values
// in registers between the phases of the scan (and spill).
template <class T, class VV> __device__ inline void pin_packed(VV& v) {
  if constexpr (sizeof(T) < 4) asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// Row prefixes of a wave's striped tile. Vector (j, lane) has in-lane total
// t[j]; the wave's order is j-major (vector j*64 + lane). Instead of one DPP
// wave scan per row, the V*64 totals go through the wave's LDS area `a`
// once: lane L takes the V consecutive totals L*V .. L*V+V-1, scans them in
// its registers, and one wave scan over the lane sums gives every lane's
// offset; the exclusive prefixes go back to `a` in the striped order, where
// vector (j, lane) finds its prefix at a[j*64 + lane]. Returns the wave's
// aggregate. LDS operations of one wave complete in issue order, so no
// barrier is needed between the writes and the reads of other lanes' slots.
template <class T, class Op, int V>
__device__ inline T wave_row_prefixes(const T (&t)[V], T* a, int lane) {
#pragma unroll
  for (int j = 0; j < V; ++j) a[j * kWave + lane] = t[j];
  __builtin_amdgcn_wave_barrier();
  T u[V];
  __builtin_memcpy(u, a + lane * V, sizeof u);
#pragma unroll
  for (int k = 1; k < V; ++k) u[k] = Op::combine(u[k - 1], u[k]);
  const T incl = wave_inclusive_scan<Op>(u[V - 1]);
  const T excl = wave_shift_right<Op>(incl);
  T e[V];
  e[0] = excl;
#pragma unroll
  for (int k = 1; k < V; ++k) e[k] = Op::combine(excl, u[k - 1]);
  __builtin_amdgcn_wave_barrier();
  __builtin_memcpy(a + lane * V, e, sizeof e);
  __builtin_amdgcn_wave_barrier();
  return read_lane(incl, kWave - 1);
}

// Where the LDS path above replaces the per-row scans: the affine pairs
// (two VALU operations per combine on two words), from 4 rows per lane.
// Measured on MI355X: affine 2^26 -1.5 %, 2^22 -3 % time; the additive
// types gain nothing (within 0.5 %) and UInt8 2^30 loses 1 %, since their
// per-row DPP scans are already one fused instruction per step.
constexpr int kRowsViaLds = 4;
template <class Op, int V> constexpr bool kLdsRowsFor = __is_same(Op, OpAffine) && V >= kRowsViaLds;
// Elements of 16 bytes or more (one element per lane unit: the
// quaternions) take a blocked layout instead of the striped one: lane l
// holds units l*V .. l*V + V-1 of its wave's chunk, scans them serially in
// registers, and one wave scan over the lane totals follows. Striped, every
// 64-element row needed its own 6-step wave scan (6 of the 16-product
// combines per element); blocked, about 2 to 3.5 (2^26 quaternions, HIP
// graphs: QuaternionF32 897 -> 608 us, Float64 1916 -> 1874 us). Full tiles
// reach that order through LDS (below); the partial tiles read and write
// their units in place, through the cache (temporal accesses, so that the
// lines a lane's V instructions share stay cached between them).
template <class T> constexpr bool kBlockedFor = ScanShape<T>::EPV == 1;

// Full tiles of the blocked layout move through LDS instead: the wave loads
// its chunk striped (unit j*64 + lane: every instruction one contiguous
// KiB, nontemporal) and transposes it to the blocked order, and the results
// go back to the striped order before the stores. A lane's units l*V ..
// l*V+V-1 are V*16 or V*32 bytes apart from its neighbours', so a blocked
// access instruction touches 64 cache lines where a striped one touches 8:
// a copy in the blocked pattern through the cache moves 3.9 TB/s on MI355X
// (1 GiB), in the striped pattern 5.7-6.6. The transpose runs in two halves
// (lanes 0-31, then 32-63) through a per-wave buffer of half the chunk, with
// one 16-byte pad per V units so that the blocked side's stride of V+1
// granules spreads over the banks.
template <class T, int V> struct BlockedLds {
  static constexpr int G = kVecBytes<T> / 16;                  // 16-byte granules per unit
  static constexpr int HALF = V / 2 * kWave;                     // units per half chunk
  static constexpr int GRANULES = HALF * G + HALF / V;           // with the pads
  __device__ static int at(int i) { return i * G + i / V; }     // granule of local unit i
};
template <class Vec> __device__ inline void lds_put(uint4* buf, int g, const Vec& v) {
  __builtin_memcpy(buf + g, &v, sizeof(Vec));
}
template <class Vec> __device__ inline void lds_get(const uint4* buf, int g, Vec& v) {
  __builtin_memcpy(&v, buf + g, sizeof(Vec));
}
// The striped side works in 16-byte granules: register granule i of a lane
// (granule i % G of unit i / G in r) is granule i*64 + lane of the wave's
// chunk, so that every load and store instruction covers one contiguous KiB
// also for the 32-byte units (QuaternionF64: loading whole units instead,
// each instruction read every other granule of 2 KiB: 2^24 at 768 x 8
// took 302.1 us against 229.3, 10^6 27.9 against 22.8).
// striped -> blocked (in place on r); buf: this wave's BlockedLds::GRANULES
template <class T, int V, class Vec>
__device__ inline void striped_to_blocked(Vec (&r)[V], uint4* buf, int lane) {
  using B = BlockedLds<T, V>;
  constexpr int G = B::G, HG = V * G / 2;  // register granules per half chunk
  uint4 rg[V * G];
  __builtin_memcpy(rg, r, sizeof rg);
  Vec b[V];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < HG; ++i) {
      const int q = i * kWave + lane;  // granule of the half chunk
      buf[B::at(q / G) + q % G] = rg[p * HG + i];
    }
    __builtin_amdgcn_wave_barrier();
    if ((lane >> 5) == p) {
#pragma unroll
      for (int k = 0; k < V; ++k) lds_get(buf, B::at((lane - 32 * p) * V + k), b[k]);
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < V; ++k) r[k] = b[k];
}
// blocked -> striped (in place on r)
template <class T, int V, class Vec>
__device__ inline void blocked_to_striped(Vec (&r)[V], uint4* buf, int lane) {
  using B = BlockedLds<T, V>;
  constexpr int G = B::G, HG = V * G / 2;
  uint4 sg[V * G];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    __builtin_amdgcn_wave_barrier();
    if ((lane >> 5) == p) {
#pragma unroll
      for (int k = 0; k < V; ++k) lds_put(buf, B::at((lane - 32 * p) * V + k), r[k]);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < HG; ++i) {
      const int q = i * kWave + lane;
      sg[p * HG + i] = buf[B::at(q / G) + q % G];
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_memcpy(r, sg, sizeof sg);
}
template <class T, int V> __device__ inline int unit_slot(int j, int lane) {
  return kBlockedFor<T> ? lane * V + j : j * kWave + lane;
}

template <class T, class Op, class Map, bool EXCL, int BLOCK, int VPL>
__global__ __launch_bounds__(BLOCK) void scan_kernel(
    const T* src, int64_t src_stride, T* dst, int64_t dst_stride, int64_t n,
    int64_t ntiles, uint64_t* scratch, int vec, int off, int win, int post, uint32_t limit, int64_t withhold,
    uint32_t* mbox) {
  // Tiles cover the virtual range [0, n + off): element i sits at virtual
  // position i + off, where `off` is dst's misalignment in elements, so
  // every interior tile stores whole 16-byte vectors at aligned addresses
  // (the source vectors are then aligned too when src is misaligned the
  // same way, and unaligned loads otherwise). Virtual positions before
  // `off` and after the end hold the identity and are never stored.
  // `limit` is the lookback's poll budget; `withhold` >= 0 makes that tile
  // publish nothing (a test hook that forces the give-up path). `mbox` is
  // the host-mapped give-up report word (report_giveup).
  using S = ScanShape<T, BLOCK, VPL>;
  constexpr int V = S::V, EPV = S::EPV;
  constexpr int kScanWaves = BLOCK / kWave;
  __shared__ T wave_agg[kScanWaves];
  __shared__ T wave_pre[kScanWaves];
  __shared__ T s_look_val[kLookBlockFor<T, BLOCK, VPL> ? kScanWaves : 1];
  __shared__ int s_look_pre[kLookBlockFor<T, BLOCK, VPL> ? kScanWaves : 1];
  __shared__ uint64_t s_ticket;
  __shared__ int s_stop;
  __shared__ int s_hdr_stop;  // the header's give-up flag (s_stop: this call's)
  constexpr bool kLdsRows = kLdsRowsFor<Op, V>;
  using Vec = VecT<T>;
  __shared__ Vec s_stash[kStashForLookback<T, BLOCK> ? V : 1][kWave];
  __shared__ T s_rowpre[kStashForLookback<T, BLOCK> && !kLdsRows ? V : 1][kWave];
  __shared__ __align__(16) T s_rows[kLdsRows ? kScanWaves : 1][kLdsRows ? V * kWave : 1];
  constexpr bool kTranspose = kBlockedFor<T> && V >= 2;
  __shared__ uint4 s_tr[kTranspose ? kScanWaves : 1][kTranspose ? BlockedLds<T, (V >= 2 ? V : 2)>::GRANULES : 1];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const T id = Op::template identity<T>();

#ifdef KF_TIMELINE
  const uint64_t tl_start = __builtin_amdgcn_s_memrealtime();
#endif
  // Thread 0 reads the header (epoch, give-up flag) without waiting for it:
  // the tile's loads and in-register scan do not depend on either, so the
  // round trip overlaps them and both reach the workgroup through LDS at
  // the barrier after the block scan (10^7 UInt8: the read had delayed
  // every tile's first load by one memory latency).
  uint64_t hdr_epoch = 0, hdr_stop = 0;
  if (tid == 0) {
    hdr_epoch = scratch[0];
    hdr_stop = ld_agent(scratch + 1);  // an earlier give-up: every call is a no-op until cleared
  }
  const int64_t tile = blockIdx.x;
  uint64_t* desc = scratch + kScanHeaderBytes / sizeof(uint64_t);
  first_gen_stagger(win, tile);

  const int64_t wbase = tile * S::TILE + (int64_t)wave * S::WAVE_ELEMS;  // this wave's virtual chunk
  const int64_t nv = n + off;
  const bool full = vec && (tile > 0 || off == 0) && (tile + 1) * S::TILE <= nv;
  const T* srcv = src - off;  // 16-byte aligned when vec
  T* dstv = dst - off;

  // ---- load, striped: lane holds vector j*64 + lane of the wave chunk ------
  // The tile stays packed in registers (4 dwords per vector whatever T is,
  // so 16 uint8 elements cost what 4 floats do); each vector is unpacked
  // only while it is being combined.
  Vec r[V];
  if (full) {
    const Vec* g = reinterpret_cast<const Vec*>(srcv + wbase);
    if constexpr (kTranspose) {
      // granule-striped: register granule i is granule i*64 + lane
      constexpr int G = kVecBytes<T> / 16;
      const uint4* gg = reinterpret_cast<const uint4*>(g);
      uint4 rg[V * G];
#pragma unroll
      for (int i = 0; i < V * G; ++i) rg[i] = ld_vec(gg + i * kWave + lane);
      __builtin_memcpy(r, rg, sizeof rg);
      striped_to_blocked<T, V>(r, s_tr[wave], lane);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j)
        r[j] = kBlockedFor<T> ? ld_unit_cached(g + unit_slot<T, V>(j, lane)) : ld_vec(g + unit_slot<T, V>(j, lane));
    }
    if constexpr (!__is_same(Map, MapIdentity)) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T x[EPV];
        __builtin_memcpy(x, &r[j], sizeof(Vec));
#pragma unroll
        for (int k = 0; k < EPV; ++k) x[k] = Map::apply(x[k]);
        __builtin_memcpy(&r[j], x, sizeof(Vec));
        pin_packed<T>(r[j]);
      }
    }
  } else {
    // partial tile (the last one, or the first of a misaligned view) or a
    // strided operand: vectors wholly inside [0, n) of a contiguous operand
    // still stream; the others go element by element
    // (all vector loads are issued before any is used, as in the full path)
    const Vec* g = reinterpret_cast<const Vec*>(srcv + wbase);
    bool inside[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t e0 = wbase + (int64_t)unit_slot<T, V>(j, lane) * EPV - off;  // real index of element 0
      inside[j] = vec && e0 >= 0 && e0 + EPV <= n;
      if (inside[j])
        r[j] = kBlockedFor<T> ? ld_unit_cached(g + unit_slot<T, V>(j, lane)) : ld_vec(g + unit_slot<T, V>(j, lane));
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t e0 = wbase + (int64_t)unit_slot<T, V>(j, lane) * EPV - off;
      T x[EPV];
      if (inside[j]) {
        __builtin_memcpy(x, &r[j], sizeof(Vec));
#pragma unroll
        for (int k = 0; k < EPV; ++k) x[k] = Map::apply(x[k]);
      } else {
#pragma unroll
        for (int k = 0; k < EPV; ++k) {
          const int64_t idx = e0 + k;
          x[k] = (idx >= 0 && idx < n) ? Map::apply(src[idx * src_stride]) : id;
        }
      }
      __builtin_memcpy(&r[j], x, sizeof(Vec));
      pin_packed<T>(r[j]);
    }
  }

  // ---- in-lane and wave scans; rowpre[j] = everything in the wave before
  // vector j's lane (earlier rows and earlier lanes of row j) --------------
  // (with kLdsRows the prefixes stay in s_rows until the store phase;
  // blocked: r[j] becomes the lane's inclusive scan and rowpre[0] the
  // lane's exclusive prefix in the wave)
  T carry = id;
  T rowpre[kBlockedFor<T> ? 1 : V];
  T tot[V];
  if constexpr (kBlockedFor<T>) {
    T run;
    __builtin_memcpy(&run, &r[0], sizeof(T));
#pragma unroll
    for (int j = 1; j < V; ++j) {
      T x;
      __builtin_memcpy(&x, &r[j], sizeof(T));
      run = Op::combine(run, x);
      __builtin_memcpy(&r[j], &run, sizeof(T));
    }
    const T incl = wave_inclusive_scan<Op>(run);
    rowpre[0] = wave_shift_right<Op>(incl);
    carry = read_lane(incl, kWave - 1);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      T x[EPV];
      __builtin_memcpy(x, &r[j], sizeof(Vec));
#pragma unroll
      for (int k = 1; k < EPV; ++k) x[k] = Op::combine(x[k - 1], x[k]);
      __builtin_memcpy(&r[j], x, sizeof(Vec));
      pin_packed<T>(r[j]);
      if constexpr (kLdsRows) {
        tot[j] = x[EPV - 1];
      } else {
        const T incl = wave_inclusive_scan<Op>(x[EPV - 1]);
        rowpre[j] = Op::combine(carry, wave_shift_right<Op>(incl));
        carry = Op::combine(carry, read_lane(incl, kWave - 1));
      }
    }
  }
  if constexpr (kLdsRows) carry = wave_row_prefixes<T, Op, V>(tot, s_rows[wave], lane);
  if (lane == 0) wave_agg[wave] = carry;
  if (tid == 0) {
    s_ticket = ((hdr_epoch >> 32) << 32) | (uint64_t)blockIdx.x;  // {epoch, tile}
    s_hdr_stop = hdr_stop != 0;
  }
  __syncthreads();
  if (s_hdr_stop) {
    // no store and no publication: reported, so that the skipped call
    // surfaces at the caller's next entry point instead of passing silently
    if (tid == 0 && tile == 0) report_giveup(mbox);
    return;
  }
  const uint64_t tk = s_ticket;
  const uint32_t epoch30 = (uint32_t)(tk >> 32) & 0x3fffffffu;
#ifdef KF_TIMELINE
  const uint64_t tl_scanned = __builtin_amdgcn_s_memrealtime();
#endif

  // ---- publish, look back, publish the inclusive prefix (wave 0) ----------
  // Lane w of wave 0 holds wave w's aggregate; a DPP scan over those lanes
  // gives the tile aggregate and every wave's exclusive prefix in the tile.
  // With win < 0 every wave of the workgroup reads a share of the
  // predecessors (lookback_all_wave) and wave 0 combines the waves' folds.
  const bool look_block = kLookBlockFor<T, BLOCK, VPL> && win < 0;
  T wexcl = id, agg = id, excl = id;
  bool gave_up = false;
  const bool pub = tile != withhold;
  if (wave == 0) {
    if constexpr (kStashForLookback<T, BLOCK>) {
      // park wave 0's tile in LDS so the lookback's registers do not add to
      // the tile's (the kernel's VGPR count is the peak over both)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        s_stash[j][lane] = r[j];
        if constexpr (!kLdsRows) s_rowpre[j][lane] = rowpre[j];
      }
      asm volatile("" ::: "memory");
    }
    const T wagg = lane < kScanWaves ? wave_agg[lane] : id;
    const T wincl = wave_inclusive_scan<Op>(wagg);
    wexcl = wave_shift_right<Op>(wincl);
    agg = read_lane(wincl, kScanWaves - 1);
    if (lane == 0 && pub) publish(desc, tile, (epoch30 << 2) | (tile == 0 ? kStatePrefix : kStatePartial), agg);
  }
  if constexpr (kLookBlockFor<T, BLOCK, VPL>) {
    if (look_block) {
      if (tile > 0) {
        T wv;
        const bool wp = lookback_all_wave<T, Op, kBlockChunk>(desc, tile, epoch30, limit, gave_up, tid, BLOCK, wv);
        if (lane == 0) {
          s_look_val[wave] = wv;
          s_look_pre[wave] = (wp ? 1 : 0) | (gave_up ? 2 : 0);
        }
      }
      __syncthreads();
      if (wave == 0 && tile > 0) {
        const int f = lane < kScanWaves ? s_look_pre[lane] : 0;
        gave_up = __builtin_amdgcn_ballot_w64((f & 2) != 0) != 0;
        const uint64_t pm = __builtin_amdgcn_ballot_w64((f & 1) != 0);
        const int m = pm ? 63 - __builtin_clzll(pm) : 0;
        excl = wave_reduce<Op>(lane >= m && lane < kScanWaves ? s_look_val[lane] : id);
      }
    }
  }
  if (wave == 0) {
    if (tile > 0 && !look_block) {
      if constexpr (kLookAllFor<T>)
        excl = win == 0 ? lookback_all<T, Op, kAllChunk>(desc, tile, epoch30, limit, gave_up)
                        : lookback<T, Op>(desc, tile, epoch30, window_of(win), limit, gave_up);
      else
        excl = lookback<T, Op>(desc, tile, epoch30, window_of(win), limit, gave_up);
    }
    if (tile > 0 && lane == 0 && pub && !gave_up)
      publish(desc, tile, (epoch30 << 2) | kStatePrefix, Op::combine(excl, agg));
    // next call's epoch, once every tile has read this one (the last tile's
    // completed lookback implies it); not after a give-up, which leaves the
    // buffer to the status query or a reset
    if (lane == 0 && tile == ntiles - 1 && !gave_up) st_agent(scratch, ((tk >> 32) + 1) << 32);
    if (lane == 0) s_stop = gave_up;
    if (lane == 0 && gave_up) report_giveup(mbox);
    if (lane < kScanWaves) wave_pre[lane] = lane == 0 ? excl : Op::combine(excl, wexcl);
    if constexpr (kStashForLookback<T, BLOCK>) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < V; ++j) {
        r[j] = s_stash[j][lane];
        if constexpr (!kLdsRows) rowpre[j] = s_rowpre[j][lane];
      }
    }
  }
  __syncthreads();
#ifdef KF_TIMELINE
  const uint64_t tl_prefix = __builtin_amdgcn_s_memrealtime();
#endif
  if (s_stop) return;  // this tile gave up: it stores nothing
  const T prefix = wave_pre[wave];
  if constexpr (kLdsRows) {
#pragma unroll
    for (int j = 0; j < V; ++j) rowpre[j] = s_rows[wave][j * kWave + lane];
  }

  // ---- apply and store ----------------------------------------------------
  if constexpr (kTranspose) {
    if (full) {
      // the lane's results in the blocked order, then back to striped
      // through LDS, then 16-byte nontemporal stores of whole KiB rows
      const T p = Op::combine(prefix, rowpre[0]);
      Vec ob[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T x, o;
        __builtin_memcpy(&x, &r[j], sizeof(T));
        if constexpr (EXCL) {
          if (j == 0) {
            o = (tile == 0 && tid == 0) ? exclusive_first<T, Op>() : p;  // element 0
          } else {
            T prev;
            __builtin_memcpy(&prev, &r[j - 1], sizeof(T));
            o = Op::combine(p, prev);
          }
        } else {
          o = Op::combine(p, x);
        }
        __builtin_memcpy(&ob[j], &o, sizeof(T));
      }
      blocked_to_striped<T, V>(ob, s_tr[wave], lane);
      constexpr int G = kVecBytes<T> / 16;
      uint4 og[V * G];
      __builtin_memcpy(og, ob, sizeof og);
      uint4* gd = reinterpret_cast<uint4*>(dstv + wbase);
#pragma unroll
      for (int i = 0; i < V * G; ++i) st_vec(gd + i * kWave + lane, og[i]);
    }
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (kTranspose && full) break;
    if constexpr (__is_same(T, uint8_t) && __is_same(Op, OpAdd)) {
      // UInt8 +: add the prefix byte to all 16 packed bytes at once (the
      // exclusive result is the inclusive one shifted by a byte; element 0
      // and virtual positions before `off` hold the identity 0)
      if (full && post == KF_POST_IDENTITY) {
        uint4 w = r[j];
        if constexpr (EXCL) w = shift_in_byte(w);
        const uint32_t b = 0x01010101u * (uint32_t)Op::combine(prefix, rowpre[j]);
        st_stream(reinterpret_cast<uint4*>(dstv + wbase) + j * kWave + lane,
                  make_uint4(add_bytes(w.x, b), add_bytes(w.y, b), add_bytes(w.z, b), add_bytes(w.w, b)));
        continue;
      }
    }
    T x[EPV], o[EPV];
    __builtin_memcpy(x, &r[j], sizeof(Vec));
    if constexpr (kBlockedFor<T>) {
      // r[j] holds the lane's inclusive scan up to unit j
      const T p = Op::combine(prefix, rowpre[0]);
      if constexpr (EXCL) {
        if (j == 0) {
          o[0] = (tile == 0 && tid == 0) ? exclusive_first<T, Op>() : p;  // element 0
        } else {
          T prev;
          __builtin_memcpy(&prev, &r[j - 1], sizeof(T));
          o[0] = Op::combine(p, prev);
        }
      } else {
        o[0] = Op::combine(p, x[0]);
      }
    } else {
      const T p = Op::combine(prefix, rowpre[j]);
      if constexpr (EXCL) {
        o[0] = p;
#pragma unroll
        for (int k = 1; k < EPV; ++k) o[k] = Op::combine(p, x[k - 1]);
        if (j == 0 && tile == 0 && tid == 0) o[off] = exclusive_first<T, Op>();  // element 0
      } else {
#pragma unroll
        for (int k = 0; k < EPV; ++k) o[k] = Op::combine(p, x[k]);
      }
    }
    if (post != KF_POST_IDENTITY) {  // the reference's g, applied at the store only
#pragma unroll
      for (int k = 0; k < EPV; ++k) o[k] = post_apply(post, o[k]);
    }
    const int64_t e0 = wbase + (int64_t)unit_slot<T, V>(j, lane) * EPV - off;  // real index of element 0
    if (full || (vec && e0 >= 0 && e0 + EPV <= n)) {
      Vec w;
      __builtin_memcpy(&w, o, sizeof(Vec));
      if constexpr (kBlockedFor<T>)
        st_unit_cached(reinterpret_cast<Vec*>(dstv + wbase) + unit_slot<T, V>(j, lane), w);
      else
        st_vec(reinterpret_cast<Vec*>(dstv + wbase) + unit_slot<T, V>(j, lane), w);
    } else {
#pragma unroll
      for (int k = 0; k < EPV; ++k) {
        const int64_t idx = e0 + k;
        if (idx >= 0 && idx < n) dst[idx * dst_stride] = o[k];
      }
    }
  }
#ifdef KF_TIMELINE
  __syncthreads();
  if (tid == 0 && g_scan_timeline) {
    uint64_t* w = g_scan_timeline + tile * kKfTimelineWords;
    w[0] = tl_start;
    w[1] = tl_scanned;
    w[2] = tl_prefix;
    w[3] = __builtin_amdgcn_s_memrealtime();
    w[4] = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // HW_REG_XCC_ID[3:0]
    w[5] = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID
  }
#endif
}

// Tile shape for n elements of T: a pure function of (T, n) so that the
// scratch query and the launch agree.
// Elements wider than 8 bytes carry 4-8 VGPRs per vector and per row
// prefix: they stop at 4 (16-byte) or 2 (32-byte) vectors per lane.
template <class T> constexpr int max_tier() { return sizeof(T) > 16 ? 1 : sizeof(T) > 8 ? 2 : kTiers - 1; }

template <class T> int scan_tier(int64_t n) {
  const int64_t bytes = n * (int64_t)sizeof(T);
  if (has_huge_tier<T>() && bytes >= kHugeBytes) return kTierHuge;
  if (has_wide_tier<T>() &&
      bytes >= (sizeof(T) == 1 ? kU8WideBytes : kWideBytes))
    return kTierWide;
  int t = max_tier<T>();
  while (t > kMinTier<T> && bytes < min_tiles<T>() * (int64_t)scan_block<T>(t) * kTierV[t] * kVecBytes<T>) --t;
  return t;
}

template <class T> int64_t tier_tile(int tier) {
  return (int64_t)scan_block<T>(tier) * tier_v<T>(tier) * ScanShape<T>::EPV;
}

template <class T> bool tier_exists(int tier) {
  if (tier >= 0 && tier < kTiers) return tier <= max_tier<T>();
  if (tier == kTierWide) return has_wide_tier<T>();
  if (tier == kTierHuge) return has_huge_tier<T>();
  return false;
}

// The tile shape for the reference's launch-shape keywords (workgroup =
// threads per workgroup, Nitem = elements per thread; <= 0: not given).
// Shapes are compiled ahead of time, so a request takes the shape nearest
// to it: the smallest sum of |log2(threads / workgroup)| and
// |log2(elements per lane / Nitem)|, a keyword not given standing for the
// size-based default shape's value; ties go to the default, then to the
// smaller tile. No keyword: the default.
template <class T> int shape_tier(int64_t n, int workgroup, int nitem) {
  const int def = scan_tier<T>(n);
  if (workgroup <= 0 && nitem <= 0) return def;
  const double want_threads = workgroup > 0 ? workgroup : scan_block<T>(def);
  const double want_items = nitem > 0 ? nitem : tier_v<T>(def) * ScanShape<T>::EPV;
  int best = -1;
  double best_d = 0;
  for (int t = 0; t <= kTierHuge; ++t) {
    if (!tier_exists<T>(t)) continue;
    const double d = fabs(log2(scan_block<T>(t) / want_threads)) +
                     fabs(log2(tier_v<T>(t) * ScanShape<T>::EPV / want_items));
    const bool tie = best >= 0 && fabs(d - best_d) < 1e-9;
    if (best < 0 || d < best_d - 1e-9 || (tie && t == def) ||
        (tie && best != def && tier_tile<T>(t) < tier_tile<T>(best))) {
      best = t;
      best_d = d;
    }
  }
  return best;
}

// Tiles for n elements starting `off` elements after a 16-byte boundary.
template <class T> int64_t scan_tiles(int64_t n, int off, int tier) {
  const int64_t tile = tier_tile<T>(tier);
  return (n + off + tile - 1) / tile;
}

template <class T> size_t scan_scratch(int64_t n, int tier) {
  constexpr int kMaxOff = 16 / (int)sizeof(T) - 1 > 0 ? 16 / (int)sizeof(T) - 1 : 0;
  return kScanHeaderBytes + (size_t)scan_tiles<T>(n, kMaxOff, tier) * kDescWords * sizeof(uint64_t);
}

// Workgroups of KERNEL the whole GPU holds at once (occupancy x CUs); the
// occupancy is computed once per kernel.
template <auto KERNEL> int64_t resident_tiles(int block) {
  static std::atomic<int> per_cu{0};
  int b = per_cu.load(std::memory_order_relaxed);
  if (b == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, KERNEL, block, 0) != hipSuccess || b <= 0) b = 1;
    per_cu.store(b, std::memory_order_relaxed);
  }
  return (int64_t)b * kf_device_cu_count();
}

// `mode` below carries the exclusive flag in bit 0 and the post-map g
// (kf_post) in the bits above.
#ifdef KF_TIMELINE
// Test hook (kf_debug_scan_giveup, instrumented library only): on this host
// thread, scans withhold the publication of one tile and give up after a
// short poll budget.
thread_local int64_t g_withhold = -1;
thread_local uint32_t g_spin_limit = kSpinLimit;
#else
constexpr int64_t g_withhold = -1;
constexpr uint32_t g_spin_limit = kSpinLimit;
#endif

template <class T, class Op, class Map, int TIER>
void launch_scan_tier(const void* src, int64_t ss, void* dst, int64_t ds, int64_t n, int mode, int64_t ntiles,
                      int vec, int off, void* scratch, hipStream_t stream) {
  constexpr int B = scan_block<T>(TIER), V = tier_v<T>(TIER);
  const int post = mode >> 1;
  if (mode & 1) {
    constexpr auto kernel = scan_kernel<T, Op, Map, true, B, V>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)ntiles), dim3(B), 0, stream, (const T*)src, ss, (T*)dst, ds, n,
                       ntiles, (uint64_t*)scratch, vec, off, look_window(ntiles, resident_tiles<kernel>(B), (int64_t)B * V * kVecBytes<T>, kLookAllFor<T>,
                                   kLookBlockFor<T, B, V>, B), post,
                       g_spin_limit, g_withhold, kf_mailbox(stream));
  } else {
    constexpr auto kernel = scan_kernel<T, Op, Map, false, B, V>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)ntiles), dim3(B), 0, stream, (const T*)src, ss, (T*)dst, ds, n,
                       ntiles, (uint64_t*)scratch, vec, off, look_window(ntiles, resident_tiles<kernel>(B), (int64_t)B * V * kVecBytes<T>, kLookAllFor<T>,
                                   kLookBlockFor<T, B, V>, B), post,
                       g_spin_limit, g_withhold, kf_mailbox(stream));
  }
}

template <class T, class Op, class Map>
int launch_scan(const void* src, int64_t ss, void* dst, int64_t ds, int64_t n, int excl, int tier,
                void* scratch, hipStream_t stream) {
  // Vector path when both operands are contiguous (views src[k:], dst[j:]
  // of aligned buffers included): `off` shifts the tiles to dst's alignment,
  // the loads of a differently misaligned src are unaligned vector loads.
  // (elements of 16 bytes or more need a 16-byte aligned dst for it)
  const int vec = ss == 1 && ds == 1 && ((uintptr_t)dst % 16 % sizeof(T) == 0);
  const int off = vec ? (int)(((uintptr_t)dst % 16) / sizeof(T)) : 0;
  const int64_t ntiles = scan_tiles<T>(n, off, tier);
  switch (tier) {
    case 0: launch_scan_tier<T, Op, Map, 0>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream); break;
    case 1: launch_scan_tier<T, Op, Map, 1>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream); break;
    case 2:
      if constexpr (max_tier<T>() >= 2)
        launch_scan_tier<T, Op, Map, 2>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream);
      break;
    case 3:
      if constexpr (max_tier<T>() >= 3)
        launch_scan_tier<T, Op, Map, 3>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream);
      break;
    case kTierWide:
      if constexpr (has_wide_tier<T>())
        launch_scan_tier<T, Op, Map, kTierWide>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream);
      break;
    default:
      if constexpr (has_huge_tier<T>())
        launch_scan_tier<T, Op, Map, kTierHuge>(src, ss, dst, ds, n, excl, ntiles, vec, off, scratch, stream);
  }
  return kf_check_launch("scan_kernel");
}

template <class T, class Op>
int scan_map(kf_map f, const void* src, int64_t ss, void* dst, int64_t ds, int64_t n, int excl, int tier,
             void* scratch, hipStream_t stream) {
  if constexpr (__is_same(T, f32x2) || is_quat<T>) {
    return launch_scan<T, Op, MapIdentity>(src, ss, dst, ds, n, excl, tier, scratch, stream);
  } else {
    if (f == KF_MAP_ABS2) return launch_scan<T, Op, MapAbs2>(src, ss, dst, ds, n, excl, tier, scratch, stream);
    return launch_scan<T, Op, MapIdentity>(src, ss, dst, ds, n, excl, tier, scratch, stream);
  }
}

template <class T>
int scan_op(kf_op op, kf_map f, const void* src, int64_t ss, void* dst, int64_t ds, int64_t n,
            int excl, int workgroup, int nitem, void* scratch, hipStream_t stream) {
  const int tier = shape_tier<T>(n, workgroup, nitem);
  if constexpr (__is_same(T, f32x2)) {
    return scan_map<T, OpAffine>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
  } else if constexpr (is_quat<T>) {
    return scan_map<T, OpMul>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
  } else {
    switch (op) {
      case KF_OP_ADD: return scan_map<T, OpAdd>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
      case KF_OP_MAX: return scan_map<T, OpMax>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
      case KF_OP_MUL: return scan_map<T, OpMul>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
      default: return scan_map<T, OpMin>(f, src, ss, dst, ds, n, excl, tier, scratch, stream);
    }
  }
}

// Dispatch of a per-element-type function object over kf_dtype.
template <class Fn> auto by_dtype(kf_dtype dt, Fn&& fn) -> decltype(fn((float*)nullptr)) {
  switch (dt) {
    case KF_F32: return fn((float*)nullptr);
    case KF_F64: return fn((double*)nullptr);
    case KF_I32: return fn((int32_t*)nullptr);
    case KF_I64: return fn((int64_t*)nullptr);
    case KF_U8: return fn((uint8_t*)nullptr);
    case KF_F32X2: return fn((f32x2*)nullptr);
    case KF_Q32: return fn((q32*)nullptr);
    case KF_Q64: return fn((q64*)nullptr);
  }
  return decltype(fn((float*)nullptr))();
}

}  // namespace kf

using namespace kf;

namespace kf {
// After a give-up (nothing in flight: the status query synchronised the
// stream): clear the flag and move the epoch two past the current one, so
// that no descriptor published by the failed call (tagged with its epoch or,
// from tiles that started after the last tile advanced it, the next one)
// can read as current.
__global__ void reepoch_kernel(uint64_t* hdr) {
  const uint64_t e = (hdr[0] >> 32) + 2;
  hdr[0] = (e & 0x3fffffffull) << 32;
  hdr[1] = 0;
}
}  // namespace kf

extern "C" int kf_scan_scratch_status(void* scratch, void* stream, int* gave_up) {
  if (!scratch || !gave_up) return kf_set_error(KF_EINVAL, "kf_scan_scratch_status: null pointer");
  hipStream_t s = (hipStream_t)stream;
  uint64_t* flag = (uint64_t*)scratch + 1;  // header word 1
  uint64_t w = 0;
  if (hipMemcpyAsync(&w, flag, sizeof w, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return kf_check_launch("kf_scan_scratch_status");
  *gave_up = w != 0;
  if (w != 0) hipLaunchKernelGGL(reepoch_kernel, dim3(1), dim3(1), 0, s, (uint64_t*)scratch);
  return kf_check_launch("reepoch_kernel");
}

#ifdef KF_TIMELINE
extern "C" int kf_debug_scan_giveup(int64_t tile, uint32_t spin_limit) {
  if (tile < 0) {
    g_withhold = -1;
    g_spin_limit = kSpinLimit;
    return KF_OK;
  }
  if (spin_limit == 0) return kf_set_error(KF_EINVAL, "kf_debug_scan_giveup: spin_limit must be > 0");
  g_withhold = tile;
  g_spin_limit = spin_limit;
  return KF_OK;
}
#endif

extern "C" size_t kf_scan_shaped_scratch_bytes(kf_dtype dt, kf_op op, int64_t n, int workgroup, int nitem) {
  (void)op;
  if (n < 0) n = 0;
  return by_dtype(dt, [&](auto* p) -> size_t {
    using T = std::remove_pointer_t<decltype(p)>;
    return scan_scratch<T>(n, shape_tier<T>(n, workgroup, nitem));
  });
}

extern "C" size_t kf_scan_scratch_bytes(kf_dtype dt, kf_op op, int64_t n) {
  return kf_scan_shaped_scratch_bytes(dt, op, n, 0, 0);
}

extern "C" int kf_scan_shape(kf_dtype dt, int64_t n, int workgroup, int nitem, int* threads, int* items) {
  if (!threads || !items) return kf_set_error(KF_EINVAL, "kf_scan_shape: null output pointer");
  if (kf_dtype_size(dt) == 0) return kf_set_error(KF_EINVAL, "kf_scan_shape: bad dtype %d", (int)dt);
  if (n < 0) n = 0;
  by_dtype(dt, [&](auto* p) -> int {
    using T = std::remove_pointer_t<decltype(p)>;
    const int t = shape_tier<T>(n, workgroup, nitem);
    *threads = scan_block<T>(t);
    *items = tier_v<T>(t) * ScanShape<T>::EPV;
    return 0;
  });
  return KF_OK;
}

extern "C" int kf_scan_shaped(kf_op op, kf_map f, kf_post g, kf_dtype dt, int exclusive, const void* src,
                              int64_t src_stride, void* dst, int64_t dst_stride, int64_t n, int workgroup,
                              int nitem, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = kf_validate_op(op, f, dt, /*allow_affine=*/1);
  if (rc) return rc;
  if ((rc = kf_take_giveup("kf_scan"))) return rc;
  if (g != KF_POST_IDENTITY && g != KF_POST_SQRT && g != KF_POST_ABS2)
    return kf_set_error(KF_EINVAL, "kf_scan: unknown post-map g = %d", (int)g);
  if (g != KF_POST_IDENTITY && (dt == KF_F32X2 || dt == KF_Q32 || dt == KF_Q64))
    return kf_set_error(KF_EINVAL, "kf_scan: the affine and quaternion scans take no post-map");
  if (g == KF_POST_SQRT && dt != KF_F32 && dt != KF_F64)
    return kf_set_error(KF_EINVAL, "kf_scan: sqrt post-map needs a floating-point type");
  if (n < 0) return kf_set_error(KF_EINVAL, "kf_scan: n = %lld < 0", (long long)n);
  if (n == 0) return KF_OK;
  if (!src || !dst) return kf_set_error(KF_EINVAL, "kf_scan: null src or dst");
  if (src_stride < 1 || dst_stride < 1)
    return kf_set_error(KF_EINVAL, "kf_scan: strides must be >= 1 (got %lld, %lld)",
                        (long long)src_stride, (long long)dst_stride);
  const size_t es = kf_dtype_size(dt);
  const size_t align = dt == KF_F32X2 || dt == KF_Q32 ? 4 : dt == KF_Q64 ? 8 : es;
  if ((uintptr_t)src % align || (uintptr_t)dst % align)
    return kf_set_error(KF_EINVAL, "kf_scan: src/dst not aligned to the element type");
  // Overlap other than exact in-place aliasing would make tiles read data
  // that other tiles already overwrote.
  if (src != dst || src_stride != dst_stride) {
    const uintptr_t s0 = (uintptr_t)src, s1 = s0 + (uintptr_t)((n - 1) * src_stride + 1) * es;
    const uintptr_t d0 = (uintptr_t)dst, d1 = d0 + (uintptr_t)((n - 1) * dst_stride + 1) * es;
    if (s0 < d1 && d0 < s1)
      return kf_set_error(KF_EINVAL, "kf_scan: src and dst overlap without being identical");
  }
  const size_t need = kf_scan_shaped_scratch_bytes(dt, op, n, workgroup, nitem);
  if (!scratch || scratch_bytes < need)
    return kf_set_error(KF_ENOSCRATCH, "kf_scan: scratch of %zu bytes needed, %zu given", need,
                        scratch ? scratch_bytes : (size_t)0);
  if ((uintptr_t)scratch % 256)
    return kf_set_error(KF_EINVAL, "kf_scan: scratch must be 256-byte aligned");
  // tiles of this dtype (an upper bound: the scratch query allows for the
  // largest misalignment shift) times threads per tile must fit the grid
  const int64_t tiles = (int64_t)((need - kScanHeaderBytes) / (kDescWords * sizeof(uint64_t)));
  if (tiles * kScanBlock > (int64_t)0xffffffffLL)
    return kf_set_error(KF_EINVAL, "kf_scan: n = %lld exceeds the grid limit", (long long)n);
  hipStream_t s = (hipStream_t)stream;
  const int mode = (exclusive ? 1 : 0) | ((int)g << 1);
  return by_dtype(dt, [&](auto* p) -> int {
    using T = std::remove_pointer_t<decltype(p)>;
    return scan_op<T>(op, f, src, src_stride, dst, dst_stride, n, mode, workgroup, nitem, scratch, s);
  });
}

extern "C" int kf_scan(kf_op op, kf_map f, kf_post g, kf_dtype dt, int exclusive, const void* src,
                       int64_t src_stride, void* dst, int64_t dst_stride, int64_t n, void* scratch,
                       size_t scratch_bytes, void* stream) {
  return kf_scan_shaped(op, f, g, dt, exclusive, src, src_stride, dst, dst_stride, n, 0, 0, scratch,
                        scratch_bytes, stream);
}

#ifdef KF_TIMELINE
// Points the instrumented scan kernels at a device buffer of
// kKfTimelineWords words per tile (null: stop recording). Exported by
// libkfhip_timeline.so only.
extern "C" int kf_debug_scan_timeline(void* buf) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_scan_timeline), &buf, sizeof(buf)) != hipSuccess)
    return kf_check_launch("kf_debug_scan_timeline");
  return KF_OK;
}
#endif
