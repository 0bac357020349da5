// Narrow-output FP32 GEMMs on gfx950 matrix cores: 16-row strips spanning all
// N <= 128 output columns, K <= 256 (the router GEMM and the expert GEMM of
// the fused chain at the shapes of the reference chain benchmarks).
//
// Work unit: a strip = 16 rows of one segment (expert) x every output column.
// One persistent workgroup per CU owns a contiguous range of strips; wave w
// computes columns [16 w, 16 w + 16) of each strip (BN / 16 waves).
//   B (the segment's [K, N] weights) stays in registers for as long as the
//     workgroup stays on that segment: wave w holds its own 16 columns for the
//     whole K in MFMA operand order (lane (li, g) holds B[16c + 4g + s][16w + li],
//     64 floats), loaded straight from global memory (one load instruction
//     reads 64 contiguous bytes of four k rows). B needs no LDS stage, no
//     transposing stores and no barrier, and the first strip's MFMAs wait for
//     each k chunk of B as it arrives rather than for all of it. The router
//     (K = 256, four waves) instead keeps B in LDS, each wave filling its own
//     columns with 16 direct loads.
//   A rows (16 x K) are loaded by the whole workgroup with row-contiguous
//     float4 accesses into registers, stored to one of two [16][K + 4] LDS
//     stages (strips alternate, one barrier per strip), and the next strip's
//     rows are loaded while the current strip's MFMAs run.
// Accumulation order per output element: k chunks of 16 ascending, inside a
// chunk MFMA step s sums k = 16c + 4g + s over g = 0..3, exactly as the tiled
// kernel in gemm.hip does, so both produce bit-identical results.
//
// Modes:
//   kStripDense      c = a * w (one segment of M rows);
//   kStripRouterGate dense + every row's top-2 gate (ids, selected-softmax
//                    weights) in the epilogue + zeroing of the row's y slice;
//   kStripGrouped    segments from offsets (read on the device);
//   kStripChain      the chain's route preparation and expert GEMM in one
//                    launch: every workgroup holds all route ids in
//                    registers (a quarter per wave), counts them into offsets,
//                    compacts the routes of its own strips in stable (route
//                    index) order with wave ballots, writes their
//                    route_pos / sorted_route entries, gathers the token rows
//                    of x (written to x_permuted when given), stores
//                    y_permuted and, for top-2 chains, adds w * y_permuted
//                    into the zeroed y (fl(0 + a) + b is the same in either
//                    order, so that combine is deterministic and equals the
//                    rank-order unpermute). Any top_k: route = top_k * token + rank.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstddef>
#include <cstdint>

#include "gate.h"
#include "launchers.h"
#include "wave.h"

namespace rr::kern {
namespace {

// Phase stamps of the chain launch (instrumentation build only: strip.hip
// compiled with -DRR_PHASE_STAMPS into libraggedroute_amd_stamps.so; the
// product library has none of this). Lane 0 of every wave writes the shader
// clock (s_memtime) at each phase boundary of the chain-mode kernel into
// g_phase_stamps[(block * 8 + wave) * kStampSlots + i], with the 100 MHz
// clock (s_memrealtime) at the start and end of the wave so that the shader
// clock's rate can be read off each wave. Slots: 0 start; 1 / 2 around the
// barrier after the id loads and LDS clears; 3 / 4 around the barrier after
// the histogram; 5 before the strip assignment, 6 after it; 7 strip table and
// the early part of B issued; 8 / 9 around the barrier after the rank passes;
// 10 route map and the rest of B issued; per strip k < 6: 11 + 4k top,
// 12 + 4k A rows stored, 13 + 4k past the barrier, 14 + 4k MFMAs issued; 36
// last epilogue issued; 37 every memory operation done; 38 / 39 the 100 MHz
// clock at start / end; 40 strips of the range; 41 half strips of the range.
#ifdef RR_PHASE_STAMPS
constexpr int kStampSlots = 48;
constexpr int kStampBlocks = 1024;
__device__ unsigned long long g_phase_stamps[kStampBlocks * 8 * kStampSlots];
#define RR_STAMP_AT(i, value)                                                             \
  do {                                                                                    \
    if constexpr (MODE == kStripChain) {                                                  \
      const unsigned long long v_ = (value);                                              \
      if (lane == 0 && b < kStampBlocks) g_phase_stamps[(b * 8 + wave) * kStampSlots + (i)] = v_; \
    }                                                                                     \
  } while (0)
#define RR_STAMP(i) RR_STAMP_AT(i, __builtin_amdgcn_s_memtime())
#else
#define RR_STAMP_AT(i, value) \
  do {                        \
  } while (0)
#define RR_STAMP(i) RR_STAMP_AT(i, 0)
#endif

using rr::dev::lane_id;
using rr::dev::lanemask_lt;

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;        // rows per strip = one MFMA tile
constexpr int kMaxChunks = 16;   // K <= 256 in chunks of 16
constexpr int kXcds = 8;         // MI355X: workgroups round-robin over 8 XCDs
constexpr int kMaxRoutes = 16384; // chain: route ids held in registers
constexpr int kMaxSegs = 8;       // chain: segments one workgroup's strips may span
constexpr int kMaxBlocks = 4;     // segments <= 256, 64 per lane column

enum StripMode : int { kStripDense = 0, kStripRouterGate = 1, kStripGrouped = 2, kStripChain = 3 };

struct StripParams {
  const float* A;  // dense / grouped: [rows, K]; chain: x [T, K] gathered by token
  const float* W;  // [segments, K, N]
  float* C;        // dense: [M, N]; grouped / chain: y_permuted [R, N]
  int M;           // dense: rows; chain: routes R = 2T
  int K;
  int N;
  int segments;    // 1 (dense) or experts
  int max_strips;  // chain: LDS capacity of the per-workgroup strip table
  const int32_t* offsets;  // grouped: [segments + 1]
  // router gate
  int32_t* gate_ids;
  float* gate_weights;
  float* y_zero;
  int y_cols;
  // chain
  int top_k;    // routes per token (route = top_k * token + rank)
  int combine;  // 1: y[token] += w * y_permuted row (top-2, y zeroed before)
  const int32_t* ids;
  const float* route_weights;
  int32_t* counts;
  int32_t* offsets_out;
  int32_t* cursors;
  int32_t* route_pos;
  int32_t* sorted_route;  // optional
  float* x_permuted;  // optional
  float* y;           // combine only
};

// Always-issued 16-byte load from an address the caller clamps in bounds; the
// caller replaces invalid values by zeros where it consumes them. A load under
// a condition becomes a branch per load and a wait at every join; a select
// right after the load waits for the data there. Prefetches keep the raw
// value and select at the LDS store, after the work they overlap.
__device__ __forceinline__ v4f load_raw(const float* ptr) {
  return *reinterpret_cast<const v4f*>(ptr);
}

__device__ __forceinline__ v4f zero_unless(bool valid, const v4f& v) {
  return valid ? v : v4f{0.0F, 0.0F, 0.0F, 0.0F};
}

// s_waitcnt vmcnt(n) for n known after unrolling (the builtin takes a constant)
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
#define RR_VM(i) case i: __builtin_amdgcn_s_waitcnt(0x0F70 | i); break;
    RR_VM(0) RR_VM(1) RR_VM(2) RR_VM(3) RR_VM(4) RR_VM(5) RR_VM(6) RR_VM(7)
    RR_VM(8) RR_VM(9) RR_VM(10) RR_VM(11) RR_VM(12) RR_VM(13) RR_VM(14) RR_VM(15)
#undef RR_VM
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}

// Per-lane segment table: lane l holds segment e = 64 j + l (segments <= 256)
// with rows [off[j], off[j] + cnt[j]) and strips [pre[j], pre[j] + strips).
// Lookups of a uniform segment are readlanes, the strip -> segment search is a
// ballot: no LDS round trips in the scheduling arithmetic.
struct SegTable {
  int32_t cnt[kMaxBlocks];
  int32_t off[kMaxBlocks];
  int32_t pre[kMaxBlocks];
  int32_t total_strips;
};

__device__ __forceinline__ int32_t strips_of(int32_t rows) { return (rows + kRows - 1) / kRows; }

// cnt[] set (zero past the last segment) -> off[], pre[], total_strips.
// Every lane of the wave takes part.
__device__ __forceinline__ void seg_scan(SegTable& t, int nblk) {
  int32_t carry_rows = 0, carry_strips = 0;
#pragma unroll
  for (int j = 0; j < kMaxBlocks; ++j) {
    if (j < nblk) {
      const int32_t st = strips_of(t.cnt[j]);
      const int32_t ri = rr::dev::wave_inclusive_scan(t.cnt[j]);
      const int32_t si = rr::dev::wave_inclusive_scan(st);
      t.off[j] = carry_rows + ri - t.cnt[j];
      t.pre[j] = carry_strips + si - st;
      carry_rows += __builtin_amdgcn_readlane(ri, 63);
      carry_strips += __builtin_amdgcn_readlane(si, 63);
    }
  }
  t.total_strips = carry_strips;
}

// Value of a per-lane table column for the uniform segment e (< 64 nblk).
__device__ __forceinline__ int32_t seg_field(const int32_t (&col)[kMaxBlocks], int nblk, int e) {
  int32_t v = 0;
#pragma unroll
  for (int j = 0; j < kMaxBlocks; ++j) {
    if (j < nblk && j == (e >> 6)) v = __builtin_amdgcn_readlane(col[j], e & 63);
  }
  return v;
}

// Segment of strip s: the last segment whose first strip is <= s (it is never
// empty, since an empty segment shares its first strip with the next one).
// Every lane of the wave must be active (ballot).
__device__ __forceinline__ int seg_find(const SegTable& t, int nblk, int segments, int s) {
  const int lane = lane_id();
#pragma unroll
  for (int j = kMaxBlocks - 1; j >= 0; --j) {
    if (j < nblk) {
      const uint64_t m = __ballot(64 * j + lane < segments && t.pre[j] <= s);
      if (m != 0) return 64 * j + 63 - __builtin_clzll(m);
    }
  }
  return 0;
}

// Sum over the wave of a per-lane value (every lane active).
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
  return __builtin_amdgcn_readlane(rr::dev::wave_inclusive_scan(v), 63);
}

struct StripRange {
  int s0, s1;
  // Half strips [h0, h1) of the range (half strip 2 s: the left half of strip
  // s's columns, 2 s + 1: the right half); strips s0 and s1 - 1 may be shared
  // with the neighbouring workers, which own their other halves.
  int h0, h1;
  // Segment-aligned ranges: all strips lie in segment e, whose strips start
  // at pre, rows at off, cnt rows (e = -1: the range may span segments).
  int e, pre, off, cnt;
};

// ceil(x / m) in 32-bit unsigned arithmetic (x >= 0, m >= 1).
__device__ __forceinline__ int32_t ceil_div32(int32_t x, int32_t m) {
  return static_cast<int32_t>((static_cast<uint32_t>(x) + static_cast<uint32_t>(m) - 1u) /
                              static_cast<uint32_t>(m));
}

// Even contiguous split of [0, total) over grid workers: sizes q or q + 1
// (no product of worker and total, so no overflow for any int32 total).
__device__ __forceinline__ StripRange even_range(int total, int grid, int worker) {
  const int q = total / grid;
  const int rem = total - q * grid;
  StripRange r;
  r.s0 = worker * q + (worker < rem ? worker : rem);
  r.s1 = r.s0 + q + (worker < rem ? 1 : 0);
  r.h0 = 2 * r.s0;
  r.h1 = 2 * r.s1;
  r.e = -1;
  r.pre = r.off = r.cnt = 0;
  return r;
}

// Strips [s0, s1) of one worker. Preferred: segment-aligned ranges counted in
// half strips (the left or right half of a strip's columns, computed by half
// of the waves), m halves per worker with w_e = ceil(2 strips_e / m) workers
// per segment, each taking an even share (at most m) of the segment's halves,
// so a worker loads one segment's B once. m is the smallest of
// m_even = ceil(2 total / grid) and m_even + 1 for which those workers fit
// the grid; otherwise (many small segments), or when a worker's strips would
// exceed cap, the even contiguous split of whole strips is used. (With 2.1
// strips per worker on average, whole strips put 3 on some workers; halves
// put at most 2 strips and one half strip, which runs half the MFMA work.)
// U: units per strip, 2 (half strips) when a strip has two waves per SIMD
// (eight waves: a half strip keeps every SIMD busy with one wave), else 1.
template <int U>
__device__ __forceinline__ StripRange assign_strips(const SegTable& t, int nblk, int segments,
                                                    int total, int grid, int worker, int cap) {
  static_assert(U == 1 || U == 2, "whole or half strips");
  const int lane = lane_id();
  const int m0 = total > 0 ? ceil_div32(U * total, grid) : U;
  // units (strips or half strips) of each lane's segments, computed once
  int32_t units[kMaxBlocks];
#pragma unroll
  for (int j = 0; j < kMaxBlocks; ++j) units[j] = j < nblk ? U * strips_of(t.cnt[j]) : 0;
  // m halves touch at most m / 2 + 1 strips (+1 when the range starts with a right half)
  auto fits_cap = [&](int m) { return (U == 2 ? m / 2 + 1 : m) <= cap; };
  // workers of segment e: [wpre_e, wpre_e + ceil(units_e / m)); the scans'
  // totals say whether m fits the grid (m0 first, m0 + 1 only when m0 fails)
  int32_t wpre[kMaxBlocks];
  auto workers_for = [&](int m) {
    int32_t carry = 0;
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
      if (j < nblk) {
        const int32_t wk = ceil_div32(units[j], m);
        const int32_t incl = rr::dev::wave_inclusive_scan(wk);
        wpre[j] = carry + incl - wk;
        carry += __builtin_amdgcn_readlane(incl, 63);
      } else {
        wpre[j] = INT_MAX;
      }
    }
    return carry;
  };
  int m = m0;
  int carry = fits_cap(m0) ? workers_for(m0) : INT_MAX;
  if (carry > grid) {
    m = m0 + 1;
    carry = fits_cap(m) ? workers_for(m) : INT_MAX;
    if (carry > grid) return even_range(total, grid, worker);
  }
  StripRange r;
  r.s0 = r.s1 = r.h0 = r.h1 = 0;
  r.e = -1;
  r.pre = r.off = r.cnt = 0;
  if (worker < carry) {
    int e = 0;
#pragma unroll
    for (int j = kMaxBlocks - 1; j >= 0; --j) {
      const uint64_t mask = __ballot(64 * j + lane < segments && wpre[j] <= worker);
      if (mask != 0) {
        e = 64 * j + 63 - __builtin_clzll(mask);
        break;
      }
    }
    const int first = seg_field(wpre, nblk, e);
    const int pre_e = seg_field(t.pre, nblk, e);
    const int cnt_e = seg_field(t.cnt, nblk, e);
    const int units_e = U * strips_of(cnt_e);
    const int workers = ceil_div32(units_e, m);  // >= 1: worker lies in this segment
    const int j = worker - first;
    // even share: units [j H / w, (j + 1) H / w); j < w <= grid, so for
    // grid <= 2^8 the products fit 32 bits below H = 2^24 (every chain shape; 64-bit
    // arithmetic for larger grouped GEMMs)
    int lo, hi;
    if (units_e < (1 << 24) && grid <= 256) {
      const uint32_t h = static_cast<uint32_t>(units_e), w = static_cast<uint32_t>(workers);
      lo = static_cast<int>(static_cast<uint32_t>(j) * h / w);
      hi = static_cast<int>(static_cast<uint32_t>(j + 1) * h / w);
    } else {
      lo = static_cast<int>(static_cast<long long>(j) * units_e / workers);
      hi = static_cast<int>(static_cast<long long>(j + 1) * units_e / workers);
    }
    lo *= 2 / U;
    hi *= 2 / U;
    r.h0 = 2 * pre_e + lo;
    r.h1 = 2 * pre_e + hi;
    r.s0 = pre_e + lo / 2;
    r.s1 = pre_e + (hi + 1) / 2;
    r.e = e;
    r.pre = pre_e;
    r.off = seg_field(t.off, nblk, e);
    r.cnt = cnt_e;
  }
  return r;
}

struct StripInfo {
  int e;        // segment
  int row0;     // first row of the strip (segment order)
  int row_end;  // end of the segment's rows
  int rank0;    // rank of row0 inside the segment
};

__device__ __forceinline__ StripInfo strip_info(const SegTable& t, int nblk, int segments, int s) {
  StripInfo si;
  si.e = seg_find(t, nblk, segments, s);
  const int off = seg_field(t.off, nblk, si.e);
  si.rank0 = (s - seg_field(t.pre, nblk, si.e)) * kRows;
  si.row0 = off + si.rank0;
  si.row_end = off + seg_field(t.cnt, nblk, si.e);
  return si;
}

// Waves per workgroup: one per 16-column tile (BN / 16), each holding its
// tile's B in registers. (Four waves of two tiles each, tried at BN = 128
// when B sat in LDS, measured 26.6 us for the headline chain's expert launch
// against 22.6 us for eight waves of one tile: two waves per SIMD hide the
// LDS and memory latencies that one wave exposes.)
constexpr int kWaves128 = 8;
constexpr int strip_waves(int bn, int mode) {
  return mode == kStripRouterGate ? bn / 16 : (bn == 128 ? kWaves128 : 4);
}

// NB: segment blocks of 64 the launch may hold (1: segments <= 64, the
// scheduling tables fold to one register column; else kMaxBlocks).
template <int BN, int WAVES, int MODE, int CHUNKS, int NB>
__global__ __launch_bounds__(WAVES * 64, 1) void rr_strip_gemm_kernel(StripParams p) {
  constexpr int kWaves = WAVES;
  constexpr int kTiles = BN / 16 / WAVES;              // 16-column MFMA tiles per wave
  static_assert(kTiles * 16 * WAVES == BN && kTiles == 1, "one 16-column tile per wave (B in its registers)");
  static_assert(MODE != kStripRouterGate || kTiles == 1, "the gate merge takes one tile per wave");
  constexpr int kThreads = kWaves * 64;
  constexpr int kIdChunks = kMaxRoutes / 256 / kWaves; // route-id chunks per wave
  constexpr int kRowThreads = kThreads / kRows;        // A staging: threads per row
  constexpr int kALoads = 64 / kRowThreads;            // float4 per thread (K <= 256)
  static_assert(BN == 64 || BN == 128, "BN is 64 or 128");
  constexpr bool kSingle = MODE == kStripDense || MODE == kStripRouterGate;  // one segment
  extern __shared__ __align__(16) float lds[];

  const int K = p.K;
  const int N = p.N;
  const int E = p.segments;
  static_assert(NB == 1 || NB == kMaxBlocks, "one block or all");
  const int nblk = NB == 1 ? 1 : (E + 63) >> 6;
  const int chunks = CHUNKS > 0 ? CHUNKS : (K + 15) >> 4;
  const int kLd = chunks * 16 + 4;
  float* As2 = lds;               // [2][16][kLd]: A rows of strip s in buffer s & 1
  constexpr int kLgLd = BN + 4;       // router: padded row of the logit tile
  float* s_lg = As2 + 2 * kRows * kLd;  // router: [16][kLgLd] logits of the strip
  // chain: [waves][kMaxSegs][4] segment lists (16-byte aligned)
  int32_t* s_seglist = reinterpret_cast<int32_t*>(s_lg + (MODE == kStripRouterGate ? kRows * kLgLd : 0));
  // Router with K = 256 and four waves: B lives in LDS, each wave's 16 columns
  // in 16 blocks of 1 KiB (one per k chunk) filled by the wave's own direct
  // loads (global_load_lds_dwordx4, lane L -> bytes [16 L, 16 L + 16) of the
  // block). Lane L fetches row 4 ((L >> 2) & 3) + (L >> 4) of the chunk and
  // columns 4 (L & 3) .. + 3, so the MFMA operand of lane (li, g) at step s,
  // B[16 c + 4 g + s][16 w + li], sits at float 64 s + 16 g + li of block c:
  // the 64 lanes of a read hit 64 distinct banks, and steps s, s + 1 pair into
  // one ds_read2st64_b32. No cross-wave dependency: no barrier for B.
  constexpr bool kBLds = MODE == kStripRouterGate && CHUNKS == kMaxChunks && WAVES == 4;
  float* s_bl = s_lg + kRows * kLgLd;  // router (kBLds): [waves][16][256]
  int32_t* s_slot = s_seglist + (MODE == kStripChain ? kWaves * kMaxSegs * 4 : 0);  // chain: [max_strips * 16]
  float* s_w = reinterpret_cast<float*>(s_slot + (MODE == kStripChain ? p.max_strips * kRows : 0));
  // chain: [max_strips * 16] token of each slot's route (-1: none), [max_strips][4] strip info
  int32_t* s_tok = reinterpret_cast<int32_t*>(s_w + (MODE == kStripChain ? p.max_strips * kRows : 0));
  int32_t* s_info = s_tok + (MODE == kStripChain ? p.max_strips * kRows : 0);
  // chain: [waves][64 nblk] route-id histogram of each wave's chunks
  int32_t* s_cntw = s_info + (MODE == kStripChain ? p.max_strips * 4 : 0);

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int g = (lane >> 4) & 3;  // (the mask tells the compiler g < 4)
  const int li = lane & 15;
  const int grid = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  // Consecutive workers on one XCD: the workgroups of one segment share its
  // weights through the same L2.
  const int worker = (grid % kXcds == 0) ? (b % kXcds) * (grid / kXcds) + b / kXcds : b;
  RR_STAMP_AT(38, __builtin_amdgcn_s_memrealtime());
  RR_STAMP(0);

  // ---- B of a segment: this wave's 16 columns, whole K, in registers ----
  // bq[c][s] = B[16c + 4g + s][16 wave + li]: sixteen lanes read 64
  // contiguous bytes of one k row, a load instruction four rows. Columns past
  // N read column N - 1 (their outputs are never stored); rows past K are
  // zero (lanes masked off the load keep the zero: no wait for the data).
  float bq[kBLds ? 1 : kMaxChunks][4];
  // chain at K = 256: the B of a later segment of the range, loaded ahead
  // (at K = 128 a segment's B arrives soon enough and the early loads cost:
  // post-route chains at the release shapes +0.1-0.4 us)
  constexpr bool kPfB = MODE == kStripChain && CHUNKS == kMaxChunks && !kBLds;
  float bq2[kPfB ? kMaxChunks : 1][4];
  int pf_e = -1;  // segment held in bq2 (-1: none)
  auto load_b2 = [&](int e) {
    if constexpr (kPfB) {
      const int n = 16 * wave + li;
      const int nc = n < N ? n : N - 1;
      const float* Wl = p.W + static_cast<std::size_t>(e) * K * N + 4 * g * N + nc;
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bq2[c][r] = Wl[(16 * c + r) * N];
      }
    } else {
      (void)e;
    }
  };
  auto load_b = [&](int e, int c_lo = 0, int c_hi = kMaxChunks) {
    if constexpr (kBLds) {
      (void)e; (void)c_lo; (void)c_hi;
      const int r = 4 * ((lane >> 2) & 3) + (lane >> 4);
      const int n = 16 * wave + 4 * (lane & 3);
      const float* src = p.W + r * N + (n < N ? n : N - 4);  // (N % 4 == 0)
      float* dst = s_bl + wave * (kMaxChunks * 256);
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        __builtin_amdgcn_global_load_lds(src + 16 * c * N, dst + 256 * c, 16, 0, 0);
      }
      return;
    }
    const float* W = p.W + static_cast<std::size_t>(e) * K * N;
    const int n = 16 * wave + li;
    const int nc = n < N ? n : N - 1;
    // K = 16 CHUNKS exactly: the lane's column at row 4g, each load adding a
    // wave-uniform row offset (one pointer per lane; with per-load lane
    // offsets the compiler keeps 64 addresses live and the chain launch
    // sits at the 256-register limit)
    const float* Wl = W + 4 * g * N + nc;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (c < chunks && c >= c_lo && c < c_hi) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if constexpr (CHUNKS > 0) {
            bq[c][s] = Wl[(16 * c + s) * N];
          } else {
            const int k = 16 * c + 4 * g + s;  // (k * N < 2^31: K <= 256, N <= 128)
            float v = 0.0F;
            if (k < K) v = W[k * N + nc];
            bq[c][s] = v;
          }
        }
      }
    }
  };

  // ---------------------------------------------------------------- segments
  SegTable tab;
  // Chain: wave w keeps route-id chunks [c_begin, c_end) of 256 routes in
  // registers (lane l holds routes 256c + 4l .. + 3); they feed the histogram
  // here and the route compaction below.
  int4 idv[kIdChunks];
  int c_begin = 0, c_end = 0;
  if constexpr (MODE == kStripChain) {
    const int R = p.M;
    const int nchunks = (R + 255) >> 8;
    c_begin = wave * nchunks / kWaves;
    c_end = (wave + 1) * nchunks / kWaves;
    // Every chunk load is issued before any is used (a select or a branch
    // between them would wait for each in turn): clamped in-bounds addresses,
    // validity applied afterwards, the ragged tail (R % 4 != 0) read last.
    // No vector read at all when R < 4: it would pass the end of ids.
    if (R >= 4) {
#pragma unroll
      for (int u = 0; u < kIdChunks; ++u) {
        const int r = (c_begin + u) * 256 + 4 * lane;
        idv[u] = *reinterpret_cast<const int4*>(p.ids + (r + 3 < R ? r : R - 4));
      }
    }
    // (LDS clears while the id loads are in flight)
    for (int i = tid; i < kWaves * 64 * nblk; i += kThreads) s_cntw[i] = 0;
    // Empty route slots of every strip this workgroup may own: cleared here,
    // barriers before the rank passes, whose waves fill slots that another
    // wave's thread would otherwise clear (a clear racing a fill loses the route).
    for (int i = tid; i < p.max_strips * kRows; i += kThreads) s_slot[i] = -1;
#pragma unroll
    for (int u = 0; u < kIdChunks; ++u) {
      const int r = (c_begin + u) * 256 + 4 * lane;
      const bool full = R >= 4 && c_begin + u < c_end && r + 3 < R;
      idv[u] = full ? idv[u] : make_int4(-1, -1, -1, -1);
    }
#pragma unroll
    for (int u = 0; u < kIdChunks; ++u) {
      const int r = (c_begin + u) * 256 + 4 * lane;
      if (c_begin + u < c_end && r < R && r + 3 >= R) {  // the ragged tail
        idv[u].x = p.ids[r];
        if (r + 1 < R) idv[u].y = p.ids[r + 1];
        if (r + 2 < R) idv[u].z = p.ids[r + 2];
      }
    }
    // Dominant experts: skewed routing (single-hot, heavy Zipf) puts most of
    // a wave's ids on one or two experts, and their LDS atomics would
    // serialise every instruction's lanes on one address. The wave's first
    // two ids (its first token's experts) are the candidates; one holding at
    // least a quarter of the first chunk's 256 ids is counted with a ballot
    // per id slot (popcounts summed in scalar registers) and skips the
    // atomics. (Eight independent ballots, no branches: probing more ids
    // cost the uniform headline chain 0.6 us.)
    int hot0 = -1, hot1 = -1;
    {
      const int c0 = __builtin_amdgcn_readfirstlane(idv[0].x);
      const int c1 = __builtin_amdgcn_readfirstlane(idv[0].y);
      const int n0 = __popcll(__ballot(idv[0].x == c0)) + __popcll(__ballot(idv[0].y == c0)) +
                     __popcll(__ballot(idv[0].z == c0)) + __popcll(__ballot(idv[0].w == c0));
      const int n1 = __popcll(__ballot(idv[0].x == c1)) + __popcll(__ballot(idv[0].y == c1)) +
                     __popcll(__ballot(idv[0].z == c1)) + __popcll(__ballot(idv[0].w == c1));
      const bool ok0 = c_begin < c_end && static_cast<unsigned>(c0) < static_cast<unsigned>(E) && n0 >= 64;
      const bool ok1 = c_begin < c_end && static_cast<unsigned>(c1) < static_cast<unsigned>(E) && n1 >= 64 &&
                       c1 != c0;
      hot0 = ok0 ? c0 : (ok1 ? c1 : -1);
      hot1 = ok0 && ok1 ? c1 : -1;
    }
    RR_STAMP(1);
    __syncthreads();  // counts zeroed
    RR_STAMP(2);
    int32_t* my_row = s_cntw + wave * 64 * nblk;  // this wave's own row
    auto unplaced = [&](int r) {
      // a route whose id lies outside [0, E) is never placed: its map entry
      // says so (workgroup 0 alone holds the write)
      if (b == 0 && r < R) p.route_pos[r] = -1;
    };
    if (hot0 >= 0) {
      int32_t n0 = 0, n1 = 0;
#pragma unroll
      for (int u = 0; u < kIdChunks; ++u) {
        if (c_begin + u < c_end) {
          const int vals[4] = {idv[u].x, idv[u].y, idv[u].z, idv[u].w};
          const int r = (c_begin + u) * 256 + 4 * lane;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const bool h0 = vals[k] == hot0;
            const bool h1 = hot1 >= 0 && vals[k] == hot1;
            n0 += __popcll(__ballot(h0));
            n1 += __popcll(__ballot(h1));
            if (static_cast<unsigned>(vals[k]) < static_cast<unsigned>(E)) {
              if (!h0 && !h1) atomicAdd(my_row + vals[k], 1);
            } else {
              unplaced(r + k);
            }
          }
        }
      }
      if (lane == 0) {
        atomicAdd(my_row + hot0, n0);
        if (hot1 >= 0) atomicAdd(my_row + hot1, n1);
      }
    } else {
#pragma unroll
      for (int u = 0; u < kIdChunks; ++u) {
        if (c_begin + u < c_end) {
          const int vals[4] = {idv[u].x, idv[u].y, idv[u].z, idv[u].w};
          const int r = (c_begin + u) * 256 + 4 * lane;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (static_cast<unsigned>(vals[k]) < static_cast<unsigned>(E)) {
              atomicAdd(my_row + vals[k], 1);
            } else {
              unplaced(r + k);
            }
          }
        }
      }
    }
    RR_STAMP(3);
    __syncthreads();
    RR_STAMP(4);
    // every wave sums the waves' rows itself (no combined row, no second barrier)
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
      int32_t total = 0;
      if (j < nblk) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total += s_cntw[w * 64 * nblk + 64 * j + lane];
      }
      tab.cnt[j] = total;
    }
  } else if constexpr (MODE == kStripGrouped) {
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
      const int e = 64 * j + lane;
      const int ec = e < E ? e : E - 1;
      const int32_t lo = p.offsets[ec];
      const int32_t hi = p.offsets[ec + 1];
      tab.cnt[j] = (j < nblk && e < E) ? hi - lo : 0;
    }
  }
  if constexpr (kSingle) {
    tab.total_strips = strips_of(p.M);  // one segment: rows [0, M)
  } else {
    seg_scan(tab, nblk);
  }
  if constexpr (MODE == kStripGrouped) {
    // rows keep the caller's offsets (the same as the prefix of the counts for
    // well-formed offsets; the caller's base is honoured)
#pragma unroll
    for (int j = 0; j < kMaxBlocks; ++j) {
      const int e = 64 * j + lane;
      tab.off[j] = (j < nblk && e < E) ? p.offsets[e] : 0;
    }
  }
  if constexpr (MODE == kStripChain) {
    if (b == 0 && wave == 0) {
#pragma unroll
      for (int j = 0; j < kMaxBlocks; ++j) {
        const int e = 64 * j + lane;
        if (j < nblk && e < E) {
          p.counts[e] = tab.cnt[j];
          p.cursors[e] = tab.cnt[j];
          p.offsets_out[e] = tab.off[j];
        }
      }
      if (lane == 0) p.offsets_out[E] = seg_field(tab.off, nblk, E - 1) + seg_field(tab.cnt, nblk, E - 1);
    }
  }

  RR_STAMP(5);
  const int total = tab.total_strips;
  StripRange range;
  if constexpr (kSingle) {
    range = even_range(total, grid, worker);
  } else {
    range = assign_strips<kWaves == 8 ? 2 : 1>(tab, nblk, E, total, grid, worker,
                                               MODE == kStripChain ? p.max_strips : INT_MAX);
  }
  RR_STAMP(6);
  const int s0 = range.s0;
  const int s1 = range.s1;
  // Half strips: waves [0, kWaves / 2) compute the left half of a strip's
  // columns, the others the right half. A wave runs strip s when its half is
  // in [h0, h1); the worker with the left half writes the strip's route map
  // and x_permuted rows (a shared strip's other worker only reads them).
  const int side = wave >= kWaves / 2 ? 1 : 0;
  auto runs = [&](int s) { return 2 * s + side >= range.h0 && 2 * s + side < range.h1; };
  auto owns_map = [&](int s) { return 2 * s >= range.h0; };
  auto info = [&](int s) -> StripInfo {
    if constexpr (kSingle) {
      return StripInfo{0, s * kRows, p.M, s * kRows};
    } else {
      if (range.e >= 0) {  // segment-aligned range: arithmetic, no lookup
        const int rank0 = (s - range.pre) * kRows;
        return StripInfo{range.e, range.off + rank0, range.off + range.cnt, rank0};
      }
      return strip_info(tab, nblk, E, s);
    }
  };
  StripInfo cur{};
  if (s0 < s1) cur = info(s0);
  constexpr int kEarlyB = 12;  // chain: k chunks of B issued before the ranks
  if constexpr (MODE == kStripChain) {
    // k chunks 0..11 of B (48 loads per lane) as soon as the first segment is
    // known: they arrive while the ranks are computed. All of B here would
    // reach the wave's limit of outstanding loads (63) and stall the rank
    // passes at issue (measured at the headline shape: expert launch 19.6 us
    // with all of B here, 18.5 us with half, 18.7 us with none; with one
    // pointer per lane for B, chunks 0..11 15.87 us against 16.13 us for
    // 0..7, 16.12 for 0..9 and 15.98 for 0..13).
    if (s0 < s1) load_b(cur.e, 0, kEarlyB);
  }
  if constexpr (MODE == kStripChain) {
    // Every strip's info, once and in parallel (wave w: strips s0 + w,
    // s0 + w + waves, ...), for the strip loop to read back from LDS (read
    // after the barrier that ends the rank passes).
#pragma unroll 1
    for (int k = wave; k < s1 - s0; k += kWaves) {
      const StripInfo si = info(s0 + k);
      if (lane == 0) *reinterpret_cast<int4*>(s_info + 4 * k) = make_int4(si.e, si.row0, si.row_end, si.rank0);
    }
  }
  auto next_info = [&](int s) -> StripInfo {
    if constexpr (MODE == kStripChain) {
      const int4 v = *reinterpret_cast<const int4*>(s_info + 4 * (s - s0));
      return StripInfo{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                       __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
    } else {
      return info(s);
    }
  };

  RR_STAMP(7);
  // ------------------------------------------- chain: routes of my strips
  float w_pending = 0.0F;
  if constexpr (MODE == kStripChain) {
    // My segments: segment e covers my strips [s, last), i.e. its stable
    // ranks [lo, hi), stored from slot base + rank. The walk (ballot lookups
    // and readlanes, uniform control flow only) runs once per wave into the
    // wave's own LDS rows; the passes read them back (LDS operations of one
    // wave complete in order, so no barrier is needed).
    int32_t* s_segs = s_seglist + wave * kMaxSegs * 4;  // [kMaxSegs][e, lo, hi, base]
    int nseg = 0;
    if (range.e >= 0) {
      // segment-aligned range: one segment, no walk
      if (s0 < s1) {
        const int hi = (s1 - range.pre) * kRows;
        if (lane == 0) {
          *reinterpret_cast<int4*>(s_segs) = make_int4(range.e, (s0 - range.pre) * kRows,
                                                       hi < range.cnt ? hi : range.cnt,
                                                       (range.pre - s0) * kRows);
        }
        nseg = 1;
      }
    } else {
#pragma unroll 1
      for (int s = s0; s < s1 && nseg < kMaxSegs; ++nseg) {
        const int e = seg_find(tab, nblk, E, s);
        const int pre_e = seg_field(tab.pre, nblk, e);
        const int rows_e = seg_field(tab.cnt, nblk, e);
        const int end_e = pre_e + strips_of(rows_e);
        const int last = s1 < end_e ? s1 : end_e;
        const int hi = (last - pre_e) * kRows;
        if (lane == 0) {
          *reinterpret_cast<int4*>(s_segs + nseg * 4) =
              make_int4(e, (s - pre_e) * kRows, hi < rows_e ? hi : rows_e, (pre_e - s0) * kRows);
        }
        s = last > s ? last : s1;  // always advances
      }
    }
    struct Seg {
      int e, lo, hi, base;
    };
    auto seg_read = [&](int i) -> Seg {
      const int4 v = *reinterpret_cast<const int4*>(s_segs + i * 4);
      return Seg{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                 __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
    };
    // Stable ranks (route order = wave, chunk, lane, component): a segment's
    // routes in the chunks of the waves before mine are the sum of those
    // waves' histogram rows (q0). Inside my wave, each lane compares its four
    // ids of every chunk with the segment (a 4-bit match mask per chunk) and
    // one DPP scan of the per-lane match counts (two chunks per 32-bit word,
    // 16-bit fields: at most 256 matches per chunk) gives every lane its
    // rank base in each chunk. Only lanes with a match then loop over their
    // set bits and keep the ranks that fall in my strips. (One scan per two
    // chunks replaces four ballots and two mbcnts per chunk.)
    constexpr int kPairs = (kIdChunks + 1) / 2;
#pragma unroll 1
    for (int i = 0; i < nseg; ++i) {
      const Seg sg = seg_read(i);
      // (one LDS read per lane and a wave sum: a loop of dependent reads
      // costs one LDS round trip per earlier wave)
      const int32_t earlier = s_cntw[(lane < kWaves ? lane : 0) * 64 * nblk + sg.e];
      const int32_t q0 = wave_sum(lane < wave ? earlier : 0);
      const int32_t mine = __builtin_amdgcn_readlane(earlier, wave);
      if (q0 >= sg.hi || q0 + mine <= sg.lo) continue;  // no rank of this wave lies in my strips
      static_assert(kIdChunks <= 16, "4 match bits per chunk in 64 bits");
      uint64_t mk = 0;  // bit 4u + k: component k of chunk u matches
      uint32_t packed[kPairs];
#pragma unroll
      for (int j = 0; j < kPairs; ++j) packed[j] = 0;
#pragma unroll
      for (int u = 0; u < kIdChunks; ++u) {
        const uint32_t m = (idv[u].x == sg.e ? 1u : 0u) | (idv[u].y == sg.e ? 2u : 0u) |
                           (idv[u].z == sg.e ? 4u : 0u) | (idv[u].w == sg.e ? 8u : 0u);
        mk |= static_cast<uint64_t>(m) << (4 * u);
        packed[u >> 1] += static_cast<uint32_t>(__builtin_popcount(m)) << (16 * (u & 1));
      }
      int32_t base[kIdChunks];
      int32_t run = q0;
#pragma unroll
      for (int j = 0; j < kPairs; ++j) {
        if (c_begin + 2 * j < c_end) {
          const uint32_t incl = static_cast<uint32_t>(rr::dev::wave_inclusive_scan(static_cast<int32_t>(packed[j])));
          const uint32_t tot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(incl), 63));
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int u = 2 * j + h;
            if (u < kIdChunks) {
              const int32_t inc = static_cast<int32_t>((incl >> (16 * h)) & 0xFFFFu);
              const int32_t cnt = static_cast<int32_t>((packed[j] >> (16 * h)) & 0xFFFFu);
              base[u] = run + inc - cnt;
              run += static_cast<int32_t>((tot >> (16 * h)) & 0xFFFFu);
            }
          }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if (2 * j + h < kIdChunks) base[2 * j + h] = run;
          }
        }
      }
      // lanes with matches: one trip per match (divergent; usually none or one)
      uint64_t left = mk;
      while (left != 0) {
        const int bit = __builtin_ctzll(left);
        left &= left - 1;
        const int u = bit >> 2;
        const int k = bit & 3;
        int32_t b0 = base[0];
#pragma unroll
        for (int uu = 1; uu < kIdChunks; ++uu) b0 = u == uu ? base[uu] : b0;
        const uint32_t m = static_cast<uint32_t>(mk >> (4 * u)) & 15u;
        const int rank = b0 + __builtin_popcount(m & ((1u << k) - 1u));
        if (rank >= sg.lo && rank < sg.hi) s_slot[sg.base + rank] = (c_begin + u) * 256 + 4 * lane + k;
      }
    }
    RR_STAMP(8);
    __syncthreads();
    RR_STAMP(9);
  }

  // ------------------------------------------------------------ strip loop
  // A staging: thread t loads row t / kRowThreads, float4 columns
  // (t % kRowThreads) + kRowThreads u (row-contiguous across the threads).
  const int a_row = tid / kRowThreads;
  const int a_col = tid % kRowThreads;
  // token of a route (route = top_k * token + rank, route >= 0): a shift for
  // the top-2 chains instead of an integer division
  auto token_of = [&](int32_t route) -> int32_t {
    return p.top_k == 2 ? (route >> 1) : route / p.top_k;
  };
  auto a_source = [&](int s, const StripInfo& si) -> int {
    if constexpr (MODE == kStripChain) {
      (void)si;
      if (s == s0) {  // before the loop: s_tok is written after the last barrier
        const int32_t route = s_slot[a_row];
        return route >= 0 ? token_of(route) : -1;
      }
      return s_tok[(s - s0) * kRows + a_row];
    } else {
      (void)s;
      const int row = si.row0 + a_row;
      return row < si.row_end ? row : -1;
    }
  };
  v4f a_regs[kALoads];
  auto load_a = [&](int src) {
    const float* row = p.A + static_cast<std::size_t>(src < 0 ? 0 : src) * K;
#pragma unroll
    for (int u = 0; u < kALoads; ++u) {
      const int k = 4 * (a_col + kRowThreads * u);
      a_regs[u] = load_raw(row + (k < K ? k : K - 4));  // zeroed at the LDS store
    }
  };

  // chain: route and weight of the deferred strip's rows 4g + r, read from LDS
  // when the strip is deferred (not between the next strip's MFMAs)
  int32_t ep_route[4] = {-1, -1, -1, -1};
  float ep_w[4] = {0.0F, 0.0F, 0.0F, 0.0F};
  // ---- epilogue of one output row group: acc[t][r] is row 4g + r, column
  // col0 + 16 t ----
  const int col0 = 16 * kTiles * wave + li;
  auto epilogue_row = [&](int r, const v4f (&a)[kTiles], const StripInfo& st) {
    const int rl = 4 * g + r;
    if constexpr (MODE == kStripChain) {
      const int32_t route = ep_route[r];
      if (route >= 0) {
        float* crow = p.C + static_cast<std::size_t>(st.row0 + rl) * N;
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
          const int col = col0 + 16 * t;
          if (col < N) {
            // a combined chain never reads y_permuted again: nontemporal
            // stores leave no dirty lines for the end-of-launch write-back
            if (p.combine) {
              __builtin_nontemporal_store(a[t][r], crow + col);
            } else {
              crow[col] = a[t][r];
            }
          }
        }
        if (p.combine) {
          // Both routes of a token add into the zeroed output: fl(0 + a) + b
          // is the same in either order, so the combine is deterministic.
          const float w = ep_w[r];
          float* yrow = p.y + static_cast<std::size_t>(route >> 1) * N;
#pragma unroll
          for (int t = 0; t < kTiles; ++t) {
            const int col = col0 + 16 * t;
            if (col < N) unsafeAtomicAdd(yrow + col, __fmul_rn(w, a[t][r]));
          }
        }
      }
    } else {
      const int row = st.row0 + rl;
      if (row < st.row_end) {
        float* crow = p.C + static_cast<std::size_t>(row) * N;
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
          const int col = col0 + 16 * t;
          if (col < N) {
            if constexpr (MODE == kStripRouterGate) {
              __builtin_nontemporal_store(a[t][r], crow + col);  // (the gate reads LDS)
            } else {
              crow[col] = a[t][r];
            }
          }
        }
      }
    }
  };
  // Deferred epilogues (all modes but the router, whose gate merge needs the
  // whole strip at once).
  constexpr bool kDeferred = MODE != kStripRouterGate;
  v4f acc_prev[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc_prev[t] = v4f{0.0F, 0.0F, 0.0F, 0.0F};
  StripInfo prev{};
  bool pending = false;

  // Issue order (chain): k chunks 0..11 of B (above), the first strip's A
  // rows, the route map's weight loads and stores, then the rest of B.
  // Memory operations complete in order, so the A stage waits for the first
  // chunks of B, A and the weights, and the first strip's MFMAs wait for the
  // rest of B one k chunk at a time. Other modes: A rows, then all of B.
  int src = -1;
  if (s0 < s1) {
    src = a_source(s0, cur);
    load_a(src);
  }
  if constexpr (MODE == kStripChain) {
    // Route map entries of my rows; the route weights are loaded now and
    // stored to LDS with the first strip's A rows.
    const bool mine = tid < (s1 - s0) * kRows;  // <= (kMaxSegs + 1) * 16 <= kThreads
    const int32_t route = mine ? s_slot[tid] : -1;
    if (route >= 0 && p.combine) w_pending = p.route_weights[route];
    if (mine) {
      // slot tid holds row (tid % 16) of strip s0 + tid / 16 (strip info tabulated above)
      const int row = s_info[4 * (tid / kRows) + 1] + tid % kRows;
      s_tok[tid] = route >= 0 ? token_of(route) : -1;
      if (route >= 0 && owns_map(s0 + tid / kRows)) {
        p.route_pos[route] = row;
        if (p.sorted_route != nullptr) p.sorted_route[row] = route;
      }
    }
    if (s0 < s1) load_b(cur.e, kEarlyB, kMaxChunks);  // the rest of B
  } else {
    if (s0 < s1) load_b(cur.e);
  }
  RR_STAMP(10);
  for (int s = s0; s < s1; ++s) {
    const StripInfo si = cur;
    if (s - s0 < 6) RR_STAMP(11 + 4 * (s - s0));
    // No barrier before the A store: buffer s & 1 was last read by strip
    // s - 2's MFMAs, which every wave finished before the barrier below in
    // strip s - 1 (and the router's logit tile is rewritten only after that
    // barrier too).
    float* As = As2 + (s & 1) * kRows * kLd;
    // ---- this strip's A rows -> LDS (zeros past K up to the chunk edge) ----
#pragma unroll
    for (int u = 0; u < kALoads; ++u) {
      const int k = 4 * (a_col + kRowThreads * u);
      if (k < chunks * 16) {
        *reinterpret_cast<v4f*>(As + a_row * kLd + k) = zero_unless(src >= 0 && k < K, a_regs[u]);
      }
    }
    if constexpr (MODE == kStripChain) {
      if (src >= 0 && p.x_permuted != nullptr && owns_map(s)) {  // gathered rows -> x_permuted
        float* out = p.x_permuted + static_cast<std::size_t>(si.row0 + a_row) * K;
#pragma unroll
        for (int u = 0; u < kALoads; ++u) {
          const int k = 4 * (a_col + kRowThreads * u);
          if (k < K) __builtin_nontemporal_store(a_regs[u], reinterpret_cast<v4f*>(out + k));
        }
      }
      if (s == s0 && tid < (s1 - s0) * kRows) s_w[tid] = w_pending;
    }
    if (s - s0 < 6) RR_STAMP(12 + 4 * (s - s0));
    __syncthreads();
    if (s - s0 < 6) RR_STAMP(13 + 4 * (s - s0));
    // ---- prefetch the next strip's A rows (B of a new segment follows the
    // MFMAs, which still read this segment's B) ----
    if (s + 1 < s1) {
      cur = next_info(s + 1);
      src = a_source(s + 1, cur);
      load_a(src);
    }

    // ---- MFMA: acc[t] = rows x columns [col0 + 16 t - li, + 16) ----
    // The previous strip's epilogue (kept in acc_prev) is issued between these
    // MFMAs, one row per four k chunks, so its stores leave in the shadow of
    // the matrix pipe instead of after it. With two tiles the chains
    // alternate, each keeping its own k order.
    v4f acc[kTiles];
    acc[0] = v4f{0.0F, 0.0F, 0.0F, 0.0F};
    const bool active = runs(s);  // (wave-uniform)
    if (active) {
      const float* aw = As + li * kLd + 4 * g;
      // Software pipelined: chunk c + 1's A operands are read from LDS before
      // chunk c's MFMAs issue, so their latency hides behind that chunk's
      // dependent MFMA chain (k order unchanged). B comes from registers.
      v4f af_next = *reinterpret_cast<const v4f*>(aw);
      if constexpr (kBLds) {
        // B chunk c from LDS once the wave's direct load of block c is done:
        // vmcnt(15 - c) (later memory operations only make the wait longer).
        // (The compiler already waits for every direct load before the A
        // stage's LDS store, which it cannot prove disjoint from them; issuing
        // B this way still beats 64 register loads per lane, which pass the
        // 63 a wave may have outstanding: router launch 5.05 -> 4.77 us.)
        auto run = [&](const float* __restrict__ bl) {
          v4f bf_next;
          __builtin_amdgcn_s_waitcnt(0x0F70 | 15);
          bf_next[0] = bl[li + 16 * g];
          bf_next[1] = bl[li + 16 * g + 64];
          bf_next[2] = bl[li + 16 * g + 128];
          bf_next[3] = bl[li + 16 * g + 192];
#pragma unroll
          for (int c = 0; c < kMaxChunks; ++c) {
            const v4f af = af_next;
            const v4f bf = bf_next;
            if (c + 1 < kMaxChunks) {
              af_next = *reinterpret_cast<const v4f*>(aw + 16 * (c + 1));
              wait_vmcnt(14 - c);
              const float* bc = bl + 256 * (c + 1) + li + 16 * g;
              bf_next[0] = bc[0];
              bf_next[1] = bc[64];
              bf_next[2] = bc[128];
              bf_next[3] = bc[192];
            }
            __builtin_amdgcn_sched_barrier(0);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf[0], acc[0], 0, 0, 0);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf[1], acc[0], 0, 0, 0);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf[2], acc[0], 0, 0, 0);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf[3], acc[0], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
        };
        run(s_bl + wave * (kMaxChunks * 256));
      } else {
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        if (c < chunks) {
          const v4f af = af_next;
          if (c + 1 < chunks) af_next = *reinterpret_cast<const v4f*>(aw + 16 * (c + 1));
          // (the scheduler would otherwise sink that read to its use)
          __builtin_amdgcn_sched_barrier(0);
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bq[c][0], acc[0], 0, 0, 0);
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bq[c][1], acc[0], 0, 0, 0);
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bq[c][2], acc[0], 0, 0, 0);
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bq[c][3], acc[0], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (kDeferred) {
          if (c < 4 && pending) epilogue_row(c, acc_prev, prev);
        }
      }
      }
    } else if constexpr (kDeferred) {
      // the other half's strip: only the previous strip's epilogue
      if (pending) {
#pragma unroll
        for (int r = 0; r < 4; ++r) epilogue_row(r, acc_prev, prev);
      }
    }
    if (s - s0 < 6) RR_STAMP(14 + 4 * (s - s0));
    if (s + 1 < s1 && cur.e != si.e) {  // the next strip's segment
      if (kPfB && pf_e == cur.e) {
#pragma unroll
        for (int c = 0; c < kMaxChunks; ++c) {
#pragma unroll
          for (int r = 0; r < 4; ++r) bq[c][r] = bq2[c][r];
        }
        pf_e = -1;
      } else {
        load_b(cur.e);
      }
    } else if constexpr (kPfB) {
      // A range whose last segment starts after its second strip: that
      // segment's B is loaded now, behind the first strip's MFMAs, into a
      // second register set (instead of after the MFMAs of the strip before
      // the switch, where the next strip's MFMAs would wait for it)
      if (s == s0 && s1 - s0 >= 3) {
        const int e_last = __builtin_amdgcn_readfirstlane(s_info[4 * (s1 - 1 - s0)]);
        if (e_last != si.e) {
          load_b2(e_last);
          pf_e = e_last;
        }
      }
    }
    if constexpr (kDeferred) {
      // (rows 0..3 of the previous strip went out at c = 3, 7, 11, 15: the
      // calls sit outside the c < chunks test, so short K emits them too)
#pragma unroll
      for (int t = 0; t < kTiles; ++t) acc_prev[t] = acc[t];
      prev = si;
      prev.rank0 = (s - s0) * kRows;  // slot of the strip's first row (chain)
      if constexpr (MODE == kStripChain) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ep_route[r] = s_slot[prev.rank0 + 4 * g + r];
          ep_w[r] = s_w[prev.rank0 + 4 * g + r];
        }
      }
      pending = active;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) epilogue_row(r, acc, si);
    }
    if constexpr (MODE == kStripRouterGate) {
      // Top-2 of each row over its N logits: the strip's 16 x BN logits go
      // through LDS, then the kThreads / 16 lanes of a row each take four
      // adjacent columns (one ds_read_b128) and merge with register moves.
      // Keys carry the expert id, so the merge order does not change the pick.
      constexpr int kRowLanes = kThreads / kRows;  // 16 (BN = 64) or 32 (BN = 128)
      static_assert(kRowLanes * 4 == BN, "four columns per lane");
#pragma unroll
      for (int r = 0; r < 4; ++r) s_lg[(4 * g + r) * kLgLd + col0] = acc[0][r];
      __syncthreads();
      const int rows = si.row_end - si.row0 < kRows ? si.row_end - si.row0 : kRows;
      const int my_row = tid / kRowLanes;
      const int c0 = 4 * (tid % kRowLanes);
      const v4f lg = *reinterpret_cast<const v4f*>(s_lg + my_row * kLgLd + c0);
      uint64_t k1 = 0, k2 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (c0 + j < N) rr::dev::insert_key(rr::dev::gate_key(lg[j], c0 + j), k1, k2);
      }
      rr::dev::merge_top2_row16(k1, k2);
      if constexpr (kRowLanes == 32) {  // the row's other 16 lanes
        rr::dev::merge_pair(k1, k2, rr::dev::shfl_xor_u64(k1, 16), rr::dev::shfl_xor_u64(k2, 16));
      }
      if (tid % kRowLanes == 0 && my_row < rows) {
        float w1, w2;
        rr::dev::gate_weights(k1, k2, &w1, &w2);
        const std::size_t row = static_cast<std::size_t>(si.row0 + my_row);
        p.gate_ids[2 * row] = rr::dev::key_expert(k1);
        p.gate_ids[2 * row + 1] = rr::dev::key_expert(k2);
        p.gate_weights[2 * row] = w1;
        p.gate_weights[2 * row + 1] = w2;
      }
      if (p.y_zero != nullptr) {
        float* base = p.y_zero + static_cast<std::size_t>(si.row0) * p.y_cols;
        const int n = rows * p.y_cols;
        if ((p.y_cols & 3) == 0 && (reinterpret_cast<std::uintptr_t>(p.y_zero) & 15u) == 0) {
          for (int i = tid; i < n / 4; i += kThreads) {
            reinterpret_cast<v4f*>(base)[i] = v4f{0.0F, 0.0F, 0.0F, 0.0F};
          }
        } else {
          for (int i = tid; i < n; i += kThreads) base[i] = 0.0F;
        }
      }
    }
  }
  if constexpr (kDeferred) {
    if (pending) {
#pragma unroll
      for (int r = 0; r < 4; ++r) epilogue_row(r, acc_prev, prev);
    }
  }
#ifdef RR_PHASE_STAMPS
  if constexpr (MODE == kStripChain) {
    RR_STAMP(36);
    __builtin_amdgcn_s_waitcnt(0);
    RR_STAMP(37);
    RR_STAMP_AT(39, __builtin_amdgcn_s_memrealtime());
    RR_STAMP_AT(40, static_cast<unsigned long long>(s1 - s0));
    RR_STAMP_AT(41, static_cast<unsigned long long>(range.h1 - range.h0));
  }
#endif
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices] = {};

int cu_count() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 256;
  if (device >= 0 && device < kMaxDevices) {
    const int cached = g_cus[device].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0) {
    cus = 256;
  }
  if (device >= 0 && device < kMaxDevices) g_cus[device].store(cus, std::memory_order_relaxed);
  return cus;
}

constexpr std::size_t kLdsLimit = 160 * 1024;  // gfx950 LDS per workgroup

template <class Kernel>
hipError_t allow_lds(Kernel kernel) {
  static const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(kLdsLimit));
  return status;
}

int bn_for(int n) { return n <= 64 ? 64 : 128; }

// Dynamic LDS bytes of one launch.
std::size_t strip_lds(int bn, int mode, int K, int segments, int max_strips) {
  const int chunks = (K + 15) >> 4;
  const std::size_t stage = 2 * static_cast<std::size_t>(kRows) * (chunks * 16 + 4);  // A rows, two buffers (B: registers)
  std::size_t bytes = stage * sizeof(float);
  const int waves = strip_waves(bn, mode);
  if (mode == kStripRouterGate) bytes += static_cast<std::size_t>(kRows) * (bn + 4) * sizeof(float);
  if (mode == kStripRouterGate && K == 256 && waves == 4) {
    bytes += static_cast<std::size_t>(waves) * kMaxChunks * 256 * sizeof(float);  // B in LDS
  }
  if (mode == kStripChain) {
    bytes += static_cast<std::size_t>(waves) * kMaxSegs * 4 * sizeof(int32_t);  // segment lists
    bytes += 3 * static_cast<std::size_t>(max_strips) * kRows * sizeof(int32_t);  // slots, weights, tokens
    bytes += static_cast<std::size_t>(max_strips) * 4 * sizeof(int32_t);          // strip info
    bytes += static_cast<std::size_t>(waves) * 64 * ((segments + 63) / 64) * sizeof(int32_t);  // per-wave histograms
  }
  return bytes;
}

template <int BN, int MODE, int CHUNKS, int NB>
hipError_t launch_strip_4(const StripParams& p, int grid, std::size_t lds, hipStream_t stream) {
  constexpr int kWaves = strip_waves(BN, MODE);
  const hipError_t attr = allow_lds(rr_strip_gemm_kernel<BN, kWaves, MODE, CHUNKS, NB>);
  if (attr != hipSuccess) return attr;
  rr_strip_gemm_kernel<BN, kWaves, MODE, CHUNKS, NB><<<grid, kWaves * 64, lds, stream>>>(p);
  return hipGetLastError();
}

template <int BN, int MODE, int CHUNKS>
hipError_t launch_strip_3(const StripParams& p, int grid, std::size_t lds, hipStream_t stream) {
  if constexpr (MODE == kStripGrouped || MODE == kStripChain) {
    if (p.segments > 64) return launch_strip_4<BN, MODE, CHUNKS, kMaxBlocks>(p, grid, lds, stream);
  }
  return launch_strip_4<BN, MODE, CHUNKS, 1>(p, grid, lds, stream);
}

template <int BN, int MODE>
hipError_t launch_strip_2(const StripParams& p, int grid, std::size_t lds, hipStream_t stream) {
  if (p.K == 256) return launch_strip_3<BN, MODE, 16>(p, grid, lds, stream);
  if (p.K == 128) return launch_strip_3<BN, MODE, 8>(p, grid, lds, stream);
  return launch_strip_3<BN, MODE, 0>(p, grid, lds, stream);
}

template <int MODE>
hipError_t launch_strip(const StripParams& p, int grid, hipStream_t stream) {
  const int bn = bn_for(p.N);
  const std::size_t lds = strip_lds(bn, MODE, p.K, p.segments, p.max_strips);
  if (lds > kLdsLimit) return hipErrorInvalidValue;
  if (grid < 1) grid = 1;
  return bn == 64 ? launch_strip_2<64, MODE>(p, grid, lds, stream)
                  : launch_strip_2<128, MODE>(p, grid, lds, stream);
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

int grid_for(long strips_bound) {
  const long cus = cu_count();
  long grid = strips_bound < cus ? strips_bound : cus;
  if (grid >= kXcds) grid = grid / kXcds * kXcds;
  return static_cast<int>(grid < 1 ? 1 : grid);
}

StripParams base(const float* a, const float* w, float* c, int m, int k, int n, int segments) {
  StripParams p{};
  p.A = a;
  p.W = w;
  p.C = c;
  p.M = m;
  p.K = k;
  p.N = n;
  p.segments = segments;
  return p;
}

}  // namespace

bool strip_shape_ok(int k, int n, const void* a, const void* w) {
  return k > 0 && k <= 256 && (k & 3) == 0 && n > 0 && n <= 128 && (n & 3) == 0 && aligned16(a) &&
         aligned16(w);
}

bool strip_segments_ok(int segments) { return segments >= 1 && segments <= kMaxBlocks * 64; }

bool strip_chain_ok(int tokens, int top_k, int experts, int k, int n, const void* x,
                    const void* w, const void* ids, const void* x_permuted) {
  if (!strip_shape_ok(k, n, x, w) || !aligned16(ids) || !aligned16(x_permuted)) return false;
  if (!strip_segments_ok(experts) || tokens <= 0 || top_k < 1) return false;
  const long routes = static_cast<long>(tokens) * top_k;
  if (routes > kMaxRoutes) return false;
  const long bound = (routes + kRows - 1) / kRows + experts;
  const int grid = grid_for(bound);
  // strips per workgroup: up to ceil(bound / grid) in even contiguous ranges
  // (spanning at most that many segments), one more in segment-aligned ones
  const int max_strips = static_cast<int>((bound + grid - 1) / grid) + 1;
  return max_strips <= kMaxSegs + 1 &&
         strip_lds(bn_for(n), kStripChain, k, experts, max_strips) <= kLdsLimit;
}

hipError_t strip_dense(const float* a, const float* b, float* c, int m, int n, int k,
                       hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  const StripParams p = base(a, b, c, m, k, n, 1);
  return launch_strip<kStripDense>(p, grid_for((m + kRows - 1) / kRows), stream);
}

hipError_t strip_grouped(const float* x, const float* w, const int32_t* offsets, float* y,
                         int experts, int hidden, int output, long rows_bound, hipStream_t stream) {
  StripParams p = base(x, w, y, 0, hidden, output, experts);
  p.offsets = offsets;
  const long bound = (rows_bound + kRows - 1) / kRows + experts;
  return launch_strip<kStripGrouped>(p, grid_for(bound), stream);
}

hipError_t strip_router_gate(const float* x, const float* router_weights, float* logits,
                             int32_t* ids, float* gate_weights, float* y_zero, int y_cols,
                             int tokens, int experts, int hidden, hipStream_t stream) {
  if (tokens <= 0) return hipSuccess;
  StripParams p = base(x, router_weights, logits, tokens, hidden, experts, 1);
  p.gate_ids = ids;
  p.gate_weights = gate_weights;
  p.y_zero = y_zero;
  p.y_cols = y_cols;
  return launch_strip<kStripRouterGate>(p, grid_for((tokens + kRows - 1) / kRows), stream);
}

hipError_t strip_chain(const float* x, const float* expert_weights, const int32_t* ids,
                       const float* route_weights, int32_t* counts, int32_t* offsets,
                       int32_t* cursors, int32_t* route_pos, int32_t* sorted_route,
                       float* x_permuted, float* y_permuted, float* y, int tokens, int top_k,
                       int experts, int hidden, int output, hipStream_t stream) {
  if (tokens <= 0) return hipSuccess;
  if (y != nullptr && top_k != 2) return hipErrorInvalidValue;  // combine is top-2 only
  const int routes = tokens * top_k;
  StripParams p = base(x, expert_weights, y_permuted, routes, hidden, output, experts);
  const long bound = (static_cast<long>(routes) + kRows - 1) / kRows + experts;
  const int grid = grid_for(bound);
  p.max_strips = static_cast<int>((bound + grid - 1) / grid) + 1;
  p.top_k = top_k;
  p.combine = y != nullptr ? 1 : 0;
  p.ids = ids;
  p.route_weights = route_weights;
  p.counts = counts;
  p.offsets_out = offsets;
  p.cursors = cursors;
  p.route_pos = route_pos;
  p.sorted_route = sorted_route;
  p.x_permuted = x_permuted;
  p.y = y;
  if (p.max_strips > kMaxSegs + 1) return hipErrorInvalidValue;  // strip_chain_ok excludes it
  return launch_strip<kStripChain>(p, grid, stream);
}

#ifdef RR_PHASE_STAMPS
// Instrumentation build only: copies the phase stamps of the last chain-mode
// strip launch (kStampBlocks x 8 waves x kStampSlots 64-bit words) to host
// memory; returns the hipError_t of the copy.
extern "C" int rr_debug_phase_stamps(void* dst, size_t bytes) {
  const size_t size = sizeof(g_phase_stamps);
  return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_phase_stamps), bytes < size ? bytes : size, 0,
                                              hipMemcpyDeviceToHost));
}
#endif
}  // namespace rr::kern
