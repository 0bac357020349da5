// gfx950 routing kernels: top-2 gate, histogram / exclusive scan / fused
// histogram+scan, stable token permute, and the weighted unpermute.
//
// All of them are HBM- or launch-bound integer/byte work; they use wave64
// ballots, LDS privatisation and 128-bit global accesses, never MFMA.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "gate.h"
#include "launchers.h"
#include "raggedroute_capi.h"
#include "wave.h"

namespace rr::kern {
namespace {

using rr::dev::bits_for;
using rr::dev::lane_id;
using rr::dev::lanemask_lt;
using rr::dev::match_mask;
using rr::dev::wave_inclusive_scan;
using rr::dev::wave_lds_sync;

constexpr int kBlock = 1024;  // 16 waves
constexpr int kWavesPerBlock = kBlock / 64;
// Route counts up to this size take the single-workgroup metadata kernels.
constexpr int kSingleBlockRoutes = 65536;

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// ============================================================================
// Top-2 gate (semantics and key encoding in gate.h).
// ============================================================================

using rr::dev::gate_key;
using rr::dev::gate_weights;
using rr::dev::insert_key;
using rr::dev::key_expert;
using rr::dev::merge_top2;

// LPR lanes cooperate on one row (LPR in 1..64, a power of two); each lane
// keeps a local top-2 and the row's lanes merge with an xor butterfly.
template <int LPR, bool VEC4>
__global__ __launch_bounds__(256) void rr_topk_gate_kernel(const float* __restrict__ logits,
                                                           int32_t* __restrict__ ids,
                                                           float* __restrict__ weights,
                                                           int tokens, int experts,
                                                           float* __restrict__ y_zero,
                                                           int y_cols) {
  constexpr int kRowsPerWave = 64 / LPR;
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int sub = lane % LPR;
  const long row = (static_cast<long>(blockIdx.x) * 4 + wave) * kRowsPerWave + lane / LPR;
  uint64_t k1 = 0, k2 = 0;
  if (row < tokens) {
    const float* p = logits + row * experts;
    if (VEC4) {
      const int quads = experts >> 2;
      for (int q = sub; q < quads; q += LPR) {
        const float4 v = reinterpret_cast<const float4*>(p)[q];
        insert_key(gate_key(v.x, 4 * q + 0), k1, k2);
        insert_key(gate_key(v.y, 4 * q + 1), k1, k2);
        insert_key(gate_key(v.z, 4 * q + 2), k1, k2);
        insert_key(gate_key(v.w, 4 * q + 3), k1, k2);
      }
    } else {
      for (int e = sub; e < experts; e += LPR) insert_key(gate_key(p[e], e), k1, k2);
    }
  }
  merge_top2<LPR>(k1, k2);
  if (sub == 0 && row < tokens) {
    float w1, w2;
    gate_weights(k1, k2, &w1, &w2);
    ids[2 * row] = key_expert(k1);
    ids[2 * row + 1] = key_expert(k2);
    weights[2 * row] = w1;
    weights[2 * row + 1] = w2;
  }
  // Chain fusion: zero the combined output rows of this block's tokens so the
  // fused grouped GEMM can accumulate both routes of a token into them.
  if (y_zero != nullptr) {
    constexpr int kRowsPerBlock = 4 * kRowsPerWave;
    const long first = static_cast<long>(blockIdx.x) * kRowsPerBlock;
    const long rows = tokens - first < kRowsPerBlock ? tokens - first : kRowsPerBlock;
    float* base = y_zero + first * y_cols;
    for (long i = threadIdx.x; i < rows * y_cols; i += blockDim.x) base[i] = 0.0F;
  }
}

template <int LPR>
hipError_t launch_gate(const float* logits, int32_t* ids, float* weights, int tokens, int experts,
                       bool vec4, float* y_zero, int y_cols, hipStream_t stream) {
  constexpr int kRowsPerBlock = 4 * (64 / LPR);
  const unsigned blocks = static_cast<unsigned>((tokens + kRowsPerBlock - 1) / kRowsPerBlock);
  if (vec4) {
    rr_topk_gate_kernel<LPR, true><<<blocks, 256, 0, stream>>>(logits, ids, weights, tokens, experts,
                                                               y_zero, y_cols);
  } else {
    rr_topk_gate_kernel<LPR, false><<<blocks, 256, 0, stream>>>(logits, ids, weights, tokens, experts,
                                                                y_zero, y_cols);
  }
  return hipGetLastError();
}

// ============================================================================
// Histogram / exclusive scan.
// ============================================================================

// Counts the valid ids of routes [begin, end) into an LDS row, one LDS atomic
// add per route. Rows may be shared by several waves, hence the atomic. (An
// aggregated add per distinct id per 64 routes, found with ballot matches,
// took ~25 instructions per 64 routes against one: C5 route preparation 22.5
// -> 15.3 us, the headline permute stage 10.6 -> 8.1 us.) Loads are batched 8
// deep to keep them in flight.
__device__ __forceinline__ void wave_count_ids(int32_t* row, const int32_t* __restrict__ ids,
                                               int begin, int end, int experts, int wave,
                                               int waves) {
  constexpr int kBatch = 8;
  const int lane = lane_id();
  const int stride = waves * 64;
  for (int base = begin + wave * 64; base < end; base += stride * kBatch) {
    int32_t v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int r = base + u * stride + lane;
      v[u] = r < end ? ids[r] : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (static_cast<unsigned>(v[u]) < static_cast<unsigned>(experts)) atomicAdd(row + v[u], 1);
    }
  }
}

// Number of LDS histogram rows: one per wave while 16 rows fit in 32 KB.
__host__ __device__ __forceinline__ int private_rows(int experts) {
  return experts <= 512 ? kWavesPerBlock : kWavesPerBlock / 2;
}

// Exclusive scan of one value per thread across a 1024-thread block.
// wsum holds kWavesPerBlock ints of LDS. Returns the exclusive prefix and the
// block total (wrapping int32 sums, as in the reference).
__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v, int32_t* wsum, int32_t* total) {
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int32_t x = wave_inclusive_scan(v);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int32_t s = lane < kWavesPerBlock ? wsum[lane] : 0;
    s = wave_inclusive_scan(s);
    if (lane < kWavesPerBlock) wsum[lane] = s;
  }
  __syncthreads();
  const int32_t before = wave > 0 ? wsum[wave - 1] : 0;
  *total = wsum[kWavesPerBlock - 1];
  return static_cast<int32_t>(static_cast<uint32_t>(before) + static_cast<uint32_t>(x) -
                              static_cast<uint32_t>(v));
}

// Single workgroup: ids -> counts (and offsets when offsets != nullptr).
// Overwrites counts, so no external reset is needed.
__global__ __launch_bounds__(kBlock) void rr_hist_scan_single_kernel(
    const int32_t* __restrict__ ids, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int routes, int experts) {
  extern __shared__ int32_t lds[];
  const int rows = private_rows(experts);
  int32_t* bins = lds;                   // [rows][experts]
  int32_t* wsum = lds + rows * experts;  // [16]
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid >> 6;
  for (int i = tid; i < rows * experts; i += kBlock) bins[i] = 0;
  __syncthreads();
  wave_count_ids(bins + (wave % rows) * experts, ids, 0, routes, experts, wave, kWavesPerBlock);
  __syncthreads();
  // experts <= kBlock: thread e owns expert e.
  int32_t c = 0;
  if (tid < experts) {
    for (int w = 0; w < rows; ++w) c += bins[w * experts + tid];
    counts[tid] = c;
  }
  if (offsets != nullptr) {
    int32_t total = 0;
    const int32_t excl = block_exclusive_scan(c, wsum, &total);
    if (tid < experts) offsets[tid] = excl;
    if (tid == 0) offsets[experts] = total;
  }
}

// Single workgroup exclusive scan; every count is read before any offset is
// written, so counts and offsets may alias (in-place scan).
__global__ __launch_bounds__(kBlock) void rr_scan_kernel(const int32_t* counts, int32_t* offsets,
                                                         int experts) {
  __shared__ int32_t wsum[kWavesPerBlock];
  const int tid = static_cast<int>(threadIdx.x);
  const int32_t v = tid < experts ? counts[tid] : 0;
  int32_t total = 0;
  const int32_t excl = block_exclusive_scan(v, wsum, &total);  // contains __syncthreads
  if (tid < experts) offsets[tid] = excl;
  if (tid == 0) offsets[experts] = total;
}

// E == 1: every valid route belongs to expert 0, so counts[0] = routes without
// reading the ids (same O(1) path as the reference's single-bin kernel).
__global__ void rr_single_bin_kernel(int32_t* counts, int32_t* offsets, int routes) {
  counts[0] = routes;
  if (offsets != nullptr) {
    offsets[0] = 0;
    offsets[1] = routes;
  }
}

std::size_t bins_bytes(int experts) {
  return (static_cast<std::size_t>(private_rows(experts)) * experts + kWavesPerBlock) *
         sizeof(int32_t);
}

// ---- large R: LDS histograms per block, device atomics, last-block scan ----
// 512 threads, 16 ids per thread per pass (four 16-byte loads issued before
// any is used), one LDS row per wave, one direct ds_add per id. A wave whose
// first 64 ids show a dominant expert (one of four probed lanes' ids held by
// at least 12 of them) counts that expert with a ballot per load instead: its
// ids skip the LDS atomic (a hot expert would serialise every instruction's
// lanes on one address) and their popcounts are summed in a scalar register.
// At R = 2^20 (warm, E = 33 / 256): hot50 9.98 / 10.83 -> 8.1 / 8.8 us,
// uniform 7.73 / 8.51 -> 7.6 / 8.4 us (the ballot loop is a separate copy of
// the id loop: a per-id test in one loop cost uniform 0.8 us). Eight waves of
// 16 ids instead of four of 32 (same 8192 ids per block): uniform 7.62 / 8.50
// -> 7.30 / 8.05 us, hot50 8.16 / 8.90 -> 7.95 / 8.79 (two interleaved runs;
// sixteen waves of 8 ids measured the same as eight). Probing 8 or 16 lanes
// for the hot expert instead of 4 made every case slower (E33 uniform 7.25 ->
// 7.41 / 7.74 us, hot50 7.95 -> 8.10 / 8.37).
constexpr int kHistThreads = 512;
constexpr int kHistIds = 16;
constexpr int kHistPass = kHistThreads * kHistIds;  // ids per block per pass

// counts[0, experts) = 0, and with offsets given offsets[experts] = 0 (the
// last-block ticket counter of the counting kernel). A kernel, not a memset
// node, so that the path can be captured into a graph.
__global__ void rr_hist_zero_kernel(int32_t* counts, int32_t* offsets, int experts) {
  for (int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); i < experts;
       i += static_cast<int>(gridDim.x * blockDim.x)) {
    counts[i] = 0;
  }
  if (offsets != nullptr && blockIdx.x == 0 && threadIdx.x == 0) offsets[experts] = 0;
}

// Block b counts routes [b * chunk, min((b + 1) * chunk, routes)) (chunk a
// multiple of kHistPass) and adds its non-zero expert counts into counts
// (zeroed before) with returning device atomics. With offsets given (the
// fused operator) the last block also scans, which saves the scan launch:
// each block waits for its atomics to return (returned means performed at the
// device's coherence point, where every other block's device-scope loads see
// them) before one thread draws a ticket from offsets[experts]; the block
// that draws the last ticket reads the counts with device-scope loads and
// writes every offset (offsets[experts] = the total replaces the ticket).
// Only device atomics cross blocks, so no release fence is needed (one per
// block writes back the XCD's L2: 21.2 us for the operator at R = 2^20).
template <bool VEC>
__global__ __launch_bounds__(kHistThreads) void rr_hist_atomic_kernel(
    const int32_t* __restrict__ ids, int32_t* counts, int32_t* offsets, int routes, int experts,
    int chunk) {
  extern __shared__ int32_t lds[];  // [waves][experts] rows
  __shared__ int s_last;
  constexpr int kWaves = kHistThreads / 64;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid >> 6;
  int32_t* row = lds + wave * experts;
  for (int i = tid; i < kWaves * experts; i += kHistThreads) lds[i] = 0;
  __syncthreads();
  const long begin = static_cast<long>(blockIdx.x) * chunk;
  const long end = begin + chunk < routes ? begin + chunk : routes;
  int hot = -1;        // the wave's dominant expert (-1: none)
  int32_t hot_n = 0;   // its ids so far (wave-uniform)
  bool probed = false;
  for (long base = begin; base < end; base += kHistPass) {
    int32_t v[kHistIds];
    if (VEC) {  // ids 16-byte aligned; base is a multiple of 4
#pragma unroll
      for (int u = 0; u < kHistIds / 4; ++u) {
        const long r = base + 4L * (tid + kHistThreads * u);
        const long rc = r + 3 < routes ? r : ((routes - 4) & ~3L);  // aligned, in bounds
        const int4 q = routes >= 4 ? *reinterpret_cast<const int4*>(ids + rc) : make_int4(-1, -1, -1, -1);
        v[4 * u] = q.x; v[4 * u + 1] = q.y; v[4 * u + 2] = q.z; v[4 * u + 3] = q.w;
      }
#pragma unroll
      for (int u = 0; u < kHistIds / 4; ++u) {
        const long r = base + 4L * (tid + kHistThreads * u);
        if (r + 3 >= end) {  // the last pass's ragged end (rare): exact reads
#pragma unroll
          for (int k = 0; k < 4; ++k) v[4 * u + k] = r + k < end ? ids[r + k] : -1;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kHistIds; ++j) {
        const long r = base + tid + static_cast<long>(kHistThreads) * j;
        v[j] = ids[r < end ? r : begin];
      }
#pragma unroll
      for (int j = 0; j < kHistIds; ++j) {
        if (base + tid + static_cast<long>(kHistThreads) * j >= end) v[j] = -1;
      }
    }
    if (!probed) {
      probed = true;
      int best = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int cand = __builtin_amdgcn_readlane(v[0], 16 * k);
        const int n = __popcll(__ballot(v[0] == cand));
        if (static_cast<unsigned>(cand) < static_cast<unsigned>(experts) && n > best) {
          best = n;
          hot = cand;
        }
      }
      if (best < 12) hot = -1;
    }
    if (hot >= 0) {  // (wave-uniform)
#pragma unroll
      for (int j = 0; j < kHistIds; ++j) {
        const bool mine = v[j] == hot;
        hot_n += __popcll(__ballot(mine));
        if (!mine && static_cast<unsigned>(v[j]) < static_cast<unsigned>(experts)) atomicAdd(row + v[j], 1);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kHistIds; ++j) {
        if (static_cast<unsigned>(v[j]) < static_cast<unsigned>(experts)) atomicAdd(row + v[j], 1);
      }
    }
  }
  if (hot >= 0 && lane == 0) atomicAdd(row + hot, hot_n);
  __syncthreads();
  int32_t sink = 0;
  for (int e = tid; e < experts; e += kHistThreads) {
    int32_t c = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) c += lds[w * experts + e];
    if (c != 0) sink += __hip_atomic_fetch_add(counts + e, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (offsets == nullptr) return;
  // (the returned values are consumed, so every atomic above returns before this)
  asm volatile("" : : "v"(sink));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    s_last = __hip_atomic_fetch_add(offsets + experts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             static_cast<int>(gridDim.x) - 1;
  }
  __syncthreads();
  if (!s_last || wave != 0) return;
  // the last block's first wave: lane l scans counts [16 l, 16 l + 16)
  int32_t c16[16];
  int32_t mine = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int e = 16 * lane + k;
    c16[k] = e < experts ? __hip_atomic_load(counts + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    mine += c16[k];
  }
  const int32_t incl = wave_inclusive_scan(mine);
  int32_t run = incl - mine;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int e = 16 * lane + k;
    if (e < experts) offsets[e] = run;
    run += c16[k];
  }
  if (lane == 63) offsets[experts] = incl;
}

// Large R: zero kernel + counting kernel (whose last block scans when offsets
// is given).
hipError_t histogram_atomic(const int32_t* ids, int32_t* counts, int32_t* offsets, int routes,
                            int experts, hipStream_t stream) {
  rr_hist_zero_kernel<<<(experts + 255) / 256, 256, 0, stream>>>(counts, offsets, experts);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // one pass of kHistPass ids per block up to 128 blocks; larger R (or many
  // experts, whose per-block global adds grow with E) take several passes.
  // Every block adds its nonzero bins into the global counts, so each count
  // takes one atomic per block, serialised at the memory side: at R = 2^20,
  // 128 blocks measured 8.8 / 9.2 us (E = 33 / 256) against 9.4 / 11.1 with
  // 256 and 11.1 / 11.6 with 32 (fewer blocks crowd the hot-expert bins); with
  // 512-thread blocks 7.3 / 8.1 against 8.6 / 10.1 with 256 blocks and 7.4 /
  // 7.7 with 64, whose hot50 cases then lose 1 / 0.4 us. Two bins per 64-bit
  // atomic (half the atomics) was slower: 7.3 / 8.0 -> 8.0 / 8.6 us.
  const long passes = (static_cast<long>(routes) + kHistPass - 1) / kHistPass;
  long blocks = passes < 128 ? passes : 128;
  const long by_experts = static_cast<long>(routes) / (8L * experts);  // >= 8 ids per global add
  if (blocks > by_experts) blocks = by_experts > 0 ? by_experts : 1;
  const long per_block = (passes + blocks - 1) / blocks;
  const int chunk = static_cast<int>(per_block * kHistPass);
  blocks = (routes + static_cast<long>(chunk) - 1) / chunk;
  const std::size_t lds = (kHistThreads / 64) * static_cast<std::size_t>(experts) * sizeof(int32_t);
  if (aligned16(ids)) {
    rr_hist_atomic_kernel<true><<<static_cast<unsigned>(blocks), kHistThreads, lds, stream>>>(
        ids, counts, offsets, routes, experts, chunk);
  } else {
    rr_hist_atomic_kernel<false><<<static_cast<unsigned>(blocks), kHistThreads, lds, stream>>>(
        ids, counts, offsets, routes, experts, chunk);
  }
  return hipGetLastError();
}

// ============================================================================
// Stable token permute.
// route_pos[r] = offsets[e] + #{r' < r : ids[r'] == e} (route index ascending
// inside each expert segment), the closed form of the reference's stable map
// generator (reference benchmarks/adapters/unpermute_adapter.cpp:47-53).
// Kernel 1 ranks the routes; kernel 2 copies token rows (x read once, written
// top_k times).
// ============================================================================

// Block b ranks routes [b*chunk, (b+1)*chunk). It first counts every earlier
// route per expert (a recomputed prefix: no inter-block communication and no
// global scratch), then ranks its own routes WAVES*64 at a time: ballot-match
// gives the rank inside a wave and per-wave counts, an LDS pass turns those
// into the per-wave exclusive prefix of every expert. LDS: (WAVES + 1) * E ints.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void rr_permute_rank_kernel(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ offsets, int32_t* cursors,
    int32_t* __restrict__ route_pos, int32_t* __restrict__ sorted_route, int routes, int experts,
    int bits, int chunk) {
  constexpr int kThreads = WAVES * 64;
  extern __shared__ int32_t lds[];
  int32_t* wc = lds;                      // [WAVES][experts]
  int32_t* base = lds + WAVES * experts;  // [experts]
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid >> 6;
  const int begin = static_cast<int>(blockIdx.x) * chunk;
  const int end = begin + chunk < routes ? begin + chunk : routes;

  for (int i = tid; i < WAVES * experts; i += kThreads) wc[i] = 0;
  __syncthreads();
  wave_count_ids(wc + wave * experts, ids, 0, begin, experts, wave, WAVES);
  __syncthreads();
  for (int e = tid; e < experts; e += kThreads) {
    int32_t s = 0;
    for (int w = 0; w < WAVES; ++w) {
      s += wc[w * experts + e];
      wc[w * experts + e] = 0;
    }
    base[e] = s;
  }
  __syncthreads();

  for (int sub = begin; sub < end; sub += kThreads) {
    const int r = sub + tid;
    const int id = r < end ? ids[r] : -1;
    const bool valid = id >= 0 && id < experts;
    const uint64_t active = __ballot(valid);
    const uint64_t mask = match_mask(static_cast<uint32_t>(valid ? id : 0), bits, active);
    const int rank = __popcll(mask & lanemask_lt());
    const bool leader = valid && rank == 0;
    if (leader) wc[wave * experts + id] = __popcll(mask);
    __syncthreads();
    // Per expert: replace each wave's count by the number of earlier routes of
    // that expert (base plus earlier waves); untouched entries stay zero.
    for (int e = tid; e < experts; e += kThreads) {
      int32_t running = base[e];
      for (int w = 0; w < WAVES; ++w) {
        const int32_t c = wc[w * experts + e];
        if (c != 0) {
          wc[w * experts + e] = running;
          running += c;
        }
      }
      base[e] = running;
    }
    __syncthreads();
    if (r < end) {
      int32_t pos = -1;
      if (valid) {
        pos = offsets[id] + wc[wave * experts + id] + rank;
        if (pos < 0 || pos >= routes) pos = -1;  // offsets inconsistent with ids
      }
      route_pos[r] = pos;
      if (sorted_route != nullptr && pos >= 0) sorted_route[pos] = r;
    }
    // Leaders restore their entry to zero; the wave's own reads above precede
    // this store in program order, and other waves read only their own rows.
    if (leader) wc[wave * experts + id] = 0;
  }
  if (blockIdx.x == gridDim.x - 1) {
    __syncthreads();
    // base now counts every route of the expert: the cursor value a per-route
    // atomic placement would leave behind.
    for (int e = tid; e < experts; e += kThreads) cursors[e] = base[e];
  }
}

// Route preparation for the fused chain: ids -> counts, offsets, stable
// route_pos, sorted_route and cursors in one launch. Block b ranks routes
// [b*chunk, (b+1)*chunk) like rr_permute_rank_kernel, but derives the offsets
// itself: it counts every route per expert (routes before its chunk give the
// stable base, all routes give the totals) and scans the totals in LDS, so no
// block waits for another. LDS: (WAVES + 2) * E + 1 + 16 ints.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void rr_route_prep_kernel(
    const int32_t* __restrict__ ids, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ cursors, int32_t* __restrict__ route_pos,
    int32_t* __restrict__ sorted_route, int routes, int experts, int bits, int chunk) {
  constexpr int kThreads = WAVES * 64;
  extern __shared__ int32_t lds[];
  int32_t* wc = lds;                       // [WAVES][experts]
  int32_t* base = wc + WAVES * experts;    // [experts]: earlier routes of each expert
  int32_t* soff = base + experts;          // [experts + 1]: segment offsets
  int32_t* wsum = soff + experts + 1;      // [16]
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int begin = static_cast<int>(blockIdx.x) * chunk;
  const int end = begin + chunk < routes ? begin + chunk : routes;

  for (int i = tid; i < WAVES * experts; i += kThreads) wc[i] = 0;
  __syncthreads();
  wave_count_ids(wc + wave * experts, ids, 0, begin, experts, wave, WAVES);
  __syncthreads();
  for (int e = tid; e < experts; e += kThreads) {
    int32_t sum = 0;
    for (int w = 0; w < WAVES; ++w) {
      sum += wc[w * experts + e];
      wc[w * experts + e] = 0;
    }
    base[e] = sum;
  }
  __syncthreads();
  wave_count_ids(wc + wave * experts, ids, begin, routes, experts, wave, WAVES);
  __syncthreads();
  for (int e = tid; e < experts; e += kThreads) {
    int32_t sum = base[e];
    for (int w = 0; w < WAVES; ++w) {
      sum += wc[w * experts + e];
      wc[w * experts + e] = 0;
    }
    soff[e] = sum;  // total count; scanned in place below
  }
  __syncthreads();
  // Exclusive scan of the totals: thread t owns `per` consecutive experts.
  {
    const int per = (experts + kThreads - 1) / kThreads;
    int32_t local = 0;
    for (int j = 0; j < per; ++j) {
      const int e = tid * per + j;
      if (e < experts) local += soff[e];
    }
    const int32_t incl_wave = wave_inclusive_scan(local);
    if (lane == 63) wsum[wave] = incl_wave;
    __syncthreads();
    if (wave == 0) {
      int32_t v = lane < WAVES ? wsum[lane] : 0;
      v = wave_inclusive_scan(v);
      if (lane < WAVES) wsum[lane] = v;
    }
    __syncthreads();
    int32_t run = (wave > 0 ? wsum[wave - 1] : 0) + incl_wave - local;
    for (int j = 0; j < per; ++j) {
      const int e = tid * per + j;
      if (e < experts) {
        const int32_t c = soff[e];
        soff[e] = run;
        run += c;
      }
    }
    if (tid == 0) soff[experts] = wsum[WAVES - 1];
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int e = tid; e < experts; e += kThreads) {
      const int32_t c = soff[e + 1] - soff[e];
      counts[e] = c;
      cursors[e] = c;
      offsets[e] = soff[e];
    }
    if (tid == 0) offsets[experts] = soff[experts];
  }

  for (int sub = begin; sub < end; sub += kThreads) {
    const int r = sub + tid;
    const int id = r < end ? ids[r] : -1;
    const bool valid = id >= 0 && id < experts;
    const uint64_t active = __ballot(valid);
    const uint64_t mask = match_mask(static_cast<uint32_t>(valid ? id : 0), bits, active);
    const int rank = __popcll(mask & lanemask_lt());
    const bool leader = valid && rank == 0;
    if (leader) wc[wave * experts + id] = __popcll(mask);
    __syncthreads();
    for (int e = tid; e < experts; e += kThreads) {
      int32_t running = base[e];
      for (int w = 0; w < WAVES; ++w) {
        const int32_t c = wc[w * experts + e];
        if (c != 0) {
          wc[w * experts + e] = running;
          running += c;
        }
      }
      base[e] = running;
    }
    __syncthreads();
    if (r < end) {
      const int32_t pos = valid ? soff[id] + wc[wave * experts + id] + rank : -1;
      route_pos[r] = pos;
      if (pos >= 0) sorted_route[pos] = r;
    }
    if (leader) wc[wave * experts + id] = 0;
  }
}

// Token-owned row copy: element (t, c) of x is read once and stored to every
// valid destination row of token t. VEC4: c indexes float4 columns.
// Quad items: item (t, c) moves elements [4c, 4c + 4) of a row with one
// 16-byte access that needs only 4-byte alignment (gfx950 global memory takes
// unaligned vector accesses), and the last 1-3 elements of a row whose width
// is not a multiple of 4 element by element. Rows of any width and offset
// stay on vector loads and stores.
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));
typedef int i4u __attribute__((ext_vector_type(4), aligned(4)));

__host__ __device__ inline uint32_t quads_of(int width) { return (static_cast<uint32_t>(width) + 3u) / 4u; }

// Narrow rows (under 1024 floats): one thread per (token, quad) item, items
// in token-major order, grid-stride. A wave per token would leave most lanes
// idle here (the 128-float rows of the headline unpermute ran at 6.4 us that
// way, 4.0 us with items).
// KMAX > 0 (top_k <= KMAX): a token's route positions (and weights) are all
// loaded before any is used, reloading route top_k - 1 in the slots past
// top_k, so a token costs one round trip for its positions and one for its
// rows instead of one per route. KMAX = 0: any top_k, one route at a time.
// Whole quads are written with nontemporal stores, as in the wide-row kernels
// (headline permute stage 8.0 -> 7.5 us).
template <int KMAX>
__global__ __launch_bounds__(256) void rr_permute_copy_kernel(const float* __restrict__ x,
                                                              const int32_t* __restrict__ route_pos,
                                                              float* __restrict__ x_permuted,
                                                              int tokens, int top_k, int hidden,
                                                              int routes) {
  const uint32_t cols = quads_of(hidden);
  const uint32_t total = static_cast<uint32_t>(tokens) * cols;
  const uint32_t stride = blockDim.x * gridDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint32_t t = i / cols;
    const uint32_t c = i - t * cols;
    const int k0 = static_cast<int>(4 * c);
    const float* src = x + static_cast<std::size_t>(t) * hidden + k0;
    const std::size_t base = static_cast<std::size_t>(t) * top_k;
    if (k0 + 4 <= hidden) {
      const f4u v = *reinterpret_cast<const f4u*>(src);
      if constexpr (KMAX > 0) {
        int32_t pos[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) pos[j] = route_pos[base + (j < top_k ? j : top_k - 1)];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          if (j < top_k && pos[j] >= 0 && pos[j] < routes) {
            __builtin_nontemporal_store(v, reinterpret_cast<f4u*>(x_permuted + static_cast<std::size_t>(pos[j]) * hidden + k0));
          }
        }
      } else {
        for (int j = 0; j < top_k; ++j) {
          const int32_t pos = route_pos[base + j];
          if (pos >= 0 && pos < routes) {
            *reinterpret_cast<f4u*>(x_permuted + static_cast<std::size_t>(pos) * hidden + k0) = v;
          }
        }
      }
    } else {
      const int n = hidden - k0;  // 1..3
      for (int j = 0; j < top_k; ++j) {
        const int32_t pos = route_pos[base + j];
        if (pos >= 0 && pos < routes) {
          float* dst = x_permuted + static_cast<std::size_t>(pos) * hidden + k0;
          for (int q = 0; q < n; ++q) dst[q] = src[q];
        }
      }
    }
  }
}

// Narrow rows, rank-order sum acc = fl(acc + fl(w * v)) over the token's
// valid routes. KMAX > 0 (top_k <= KMAX): positions and weights of every
// route, then every route's quad (an invalid position reads row 0 and is
// left out of the sum), then the sum in rank order: two round trips per token
// instead of two per route (post-route chain T512 top_k 8 19.6 -> 16.6 us).
// KMAX = 0: any top_k, one route at a time. Whole quads of y leave with
// nontemporal stores.
template <int KMAX>
__global__ __launch_bounds__(256) void rr_unpermute_kernel(const float* __restrict__ y_permuted,
                                                           const int32_t* __restrict__ route_pos,
                                                           const float* __restrict__ route_weights,
                                                           float* __restrict__ y, int tokens,
                                                           int top_k, int output) {
  const uint32_t cols = quads_of(output);
  const uint32_t total = static_cast<uint32_t>(tokens) * cols;
  const uint32_t stride = blockDim.x * gridDim.x;
  const int routes = tokens * top_k;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint32_t t = i / cols;
    const uint32_t c = i - t * cols;
    const int k0 = static_cast<int>(4 * c);
    float* out = y + static_cast<std::size_t>(t) * output + k0;
    const std::size_t base = static_cast<std::size_t>(t) * top_k;
    if (k0 + 4 <= output) {
      f4u acc = f4u{0.0F, 0.0F, 0.0F, 0.0F};
      if constexpr (KMAX > 0) {
        int32_t pos[KMAX];
        float w[KMAX];
        f4u v[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          const std::size_t route = base + (j < top_k ? j : top_k - 1);
          pos[j] = route_pos[route];
          w[j] = route_weights[route];
        }
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          const bool ok = pos[j] >= 0 && pos[j] < routes;
          v[j] = *reinterpret_cast<const f4u*>(y_permuted + static_cast<std::size_t>(ok ? pos[j] : 0) * output + k0);
        }
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
          if (j < top_k) {
            const bool ok = pos[j] >= 0 && pos[j] < routes;
            const float sx = __fadd_rn(acc.x, __fmul_rn(w[j], v[j].x));
            const float sy = __fadd_rn(acc.y, __fmul_rn(w[j], v[j].y));
            const float sz = __fadd_rn(acc.z, __fmul_rn(w[j], v[j].z));
            const float sw = __fadd_rn(acc.w, __fmul_rn(w[j], v[j].w));
            acc.x = ok ? sx : acc.x;
            acc.y = ok ? sy : acc.y;
            acc.z = ok ? sz : acc.z;
            acc.w = ok ? sw : acc.w;
          }
        }
      } else {
        for (int j = 0; j < top_k; ++j) {
          const std::size_t route = base + j;
          const int32_t pos = route_pos[route];
          if (pos < 0 || pos >= routes) continue;
          const float w = route_weights[route];
          const f4u v = *reinterpret_cast<const f4u*>(y_permuted + static_cast<std::size_t>(pos) * output + k0);
          acc.x = __fadd_rn(acc.x, __fmul_rn(w, v.x));
          acc.y = __fadd_rn(acc.y, __fmul_rn(w, v.y));
          acc.z = __fadd_rn(acc.z, __fmul_rn(w, v.z));
          acc.w = __fadd_rn(acc.w, __fmul_rn(w, v.w));
        }
      }
      __builtin_nontemporal_store(acc, reinterpret_cast<f4u*>(out));
    } else {
      const int n = output - k0;  // 1..3
      float acc[3] = {0.0F, 0.0F, 0.0F};
      for (int j = 0; j < top_k; ++j) {
        const std::size_t route = base + j;
        const int32_t pos = route_pos[route];
        if (pos < 0 || pos >= routes) continue;
        const float w = route_weights[route];
        const float* v = y_permuted + static_cast<std::size_t>(pos) * output + k0;
        for (int q = 0; q < n; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(w, v[q]));
      }
      for (int q = 0; q < n; ++q) out[q] = acc[q];
    }
  }
}

// Token-owned rows: wave w of the grid copies rows t = w, w + waves, ...;
// lane j reads route j's position once per row (routes beyond the first 64 of
// a row, possible only in the stand-alone permute, are read 64 at a time),
// then the lanes stride over the row's quads, eight in flight per lane (x read
// once, written top_k times). Rows are read and written with nontemporal
// accesses, four blocks per CU. Measured at C4 (T = 8192, 16 KB rows, 403 MB):
// with cached loads the copy took 61 us while x sat in the Infinity Cache but
// 106-111 us cold (after a read-modify-write scrub the cache holds dirty
// lines, and every allocating load evicts one: extra write-back traffic), for
// any grid of 256-2048 blocks and 4-16 quads in flight; nontemporal loads take
// 79-82 us warm and cold alike (5.0 TB/s). Nontemporal stores: 89 -> 69 us.
constexpr int kRowQuadsInFlight = 8;

__global__ __launch_bounds__(256) void rr_permute_rows_kernel(const float* __restrict__ x,
                                                              const int32_t* __restrict__ route_pos,
                                                              float* __restrict__ x_permuted,
                                                              int tokens, int top_k, int hidden,
                                                              int routes) {
  const int lane = lane_id();
  const int cols = static_cast<int>(quads_of(hidden));
  const int waves = static_cast<int>(gridDim.x) * 4;
  for (int t = static_cast<int>(blockIdx.x) * 4 + (static_cast<int>(threadIdx.x) >> 6); t < tokens;
       t += waves) {
    const int32_t* row_pos = route_pos + static_cast<std::size_t>(t) * top_k;
    const int32_t pos0 = lane < top_k ? row_pos[lane] : -1;
    const float* src = x + static_cast<std::size_t>(t) * hidden;
    for (int q0 = 0; q0 < cols; q0 += 64 * kRowQuadsInFlight) {  // wave-uniform: readlane needs every lane
      f4u v[kRowQuadsInFlight];
#pragma unroll
      for (int u = 0; u < kRowQuadsInFlight; ++u) {
        const int k0 = 4 * (q0 + lane + 64 * u);
        if (k0 + 4 <= hidden) {
          v[u] = __builtin_nontemporal_load(reinterpret_cast<const f4u*>(src + k0));
        } else {
          v[u] = f4u{0.0F, 0.0F, 0.0F, 0.0F};
          for (int e = 0; k0 + e < hidden; ++e) v[u][e] = src[k0 + e];
        }
      }
      for (int j0 = 0; j0 < top_k; j0 += 64) {
        const int32_t my_pos = j0 == 0 ? pos0 : (j0 + lane < top_k ? row_pos[j0 + lane] : -1);
        const int n = min(64, top_k - j0);
        for (int j = 0; j < n; ++j) {
          const int32_t pos = __builtin_amdgcn_readlane(my_pos, j);
          if (pos < 0 || pos >= routes) continue;  // wave-uniform
          float* dst = x_permuted + static_cast<std::size_t>(pos) * hidden;
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            const int k0 = 4 * (q0 + lane + 64 * u);
            if (k0 + 4 <= hidden) {
              __builtin_nontemporal_store(v[u], reinterpret_cast<f4u*>(dst + k0));
            } else {
              for (int e = 0; k0 + e < hidden; ++e) dst[k0 + e] = v[u][e];
            }
          }
        }
      }
    }
  }
}

// Wide rows (hidden >= 1024) with few routes: the stable rank and the row
// copy in one launch. Block b owns tokens [b * tpb, (b + 1) * tpb), so routes
// [b * tpb * top_k, ...). Each wave first issues the nontemporal loads of its
// first row's first quads (top-2 rows on 128-byte lines: also its copy's
// second step, into LDS); then the block recounts every earlier route per
// expert and ranks its own routes (as rr_permute_rank_kernel does), keeping
// their positions in LDS besides route_pos / sorted_route; then the waves copy
// their tokens' rows. The rank phase runs under the first loads' latency and
// the copy waits for no second launch. The recount reads the routes before a
// block's range, so the host keeps this kernel to R <= kFusedRankRoutes.
//
// REALIGN (rows that do not start on a 128-byte line: hidden % 32 != 0 or an
// offset base pointer): a wave reads its row as whole 16-byte quads from the
// 128-byte line that holds the row's first float, kRealignPad quads of margin
// on either side of each 512-quad chunk, into its own LDS strip; every
// destination row is then written as 16-byte quads counted from ITS first
// 128-byte line, each lane gathering its four floats from the strip at the
// source-destination phase difference. A wave's store instruction then covers
// whole 128-byte lines (only a row's first and last line are partial), where
// quads at the row's own offset split each line between two store
// instructions. Measured on an isolated copy of C4's shape (T = 8192, two
// destinations per token, stable destinations, 16 KB rows): K = 4095 82-83 us
// (0.61 of HBM) against 86-88 us at the row's offset, K = 4093 84 against 87;
// K = 4096 (aligned rows) 84 against 80, so aligned rows keep the plain quads.
// This kernel at C4 K = 4095, cold: 92.1 us before, 87.9 with the strip, 86.9
// with the next chunk's loads issued before the current chunk's stores.
// The loads read at most the 128-byte lines that hold a row's first and last
// float (never a line without a float of x), and the stores write only the
// row's own floats.
constexpr int kFusedRankRoutes = 32768;
constexpr int kFusedWaves = 4;
constexpr int kRealignPad = 8;                                                  // quads
constexpr int kRealignStripQuads = 64 * kRowQuadsInFlight + 2 * kRealignPad;  // per wave
typedef float f4a __attribute__((ext_vector_type(4)));                         // 16-byte aligned

// Chunks per realigned row. A row's last float lies in source quad
// (hidden - 1 + hs) / 4 of its lines and in destination quad (hidden - 1 +
// hd) / 4, both at most (hidden + 30) / 4 for phases below 32 floats. A
// chunk's strip holds source quads up to c0 + kChunk + kRealignPad - 1, and
// its last step lets lanes 0..kRealignPad-1 write destination quads c0 +
// kChunk .. + kRealignPad - 1 from it, so the row takes the fewest chunks
// whose last strip reaches that quad: two at K = 4095, where counting every
// destination's quads alone (up to 1025) would take a third chunk for one quad.
__host__ __device__ inline int realign_chunks(int hidden) {
  const int last_q = (hidden + 30) >> 2;
  const int n = (last_q - kRealignPad + 64 * kRowQuadsInFlight) / (64 * kRowQuadsInFlight);
  return n > 1 ? n : 1;
}

__host__ __device__ inline int realign_strip_offset(int experts, int tokens_per_block, int top_k) {
  // int32 offset of the realign strips in the block's LDS, 16-byte aligned
  return ((kFusedWaves + 1) * experts + tokens_per_block * top_k + 3) & ~3;
}

template <bool REALIGN>
__global__ __launch_bounds__(kFusedWaves * 64) void rr_permute_rank_rows_kernel(
    const float* __restrict__ x, const int32_t* __restrict__ ids, const int32_t* __restrict__ offsets,
    int32_t* cursors, float* __restrict__ x_permuted, int32_t* __restrict__ route_pos,
    int32_t* __restrict__ sorted_route, int tokens, int top_k, int hidden, int experts, int bits,
    int tokens_per_block) {
  constexpr int kThreads = kFusedWaves * 64;
  extern __shared__ int32_t lds[];
  int32_t* wc = lds;                           // [waves][experts]
  int32_t* base = lds + kFusedWaves * experts;  // [experts]
  int32_t* slot = base + experts;               // [tokens_per_block * top_k] my routes' positions
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int routes = tokens * top_k;
  const int t_begin = static_cast<int>(blockIdx.x) * tokens_per_block;
  const int t_end = t_begin + tokens_per_block < tokens ? t_begin + tokens_per_block : tokens;
  const int begin = t_begin * top_k;
  const int end = t_end * top_k;
  const int cols = static_cast<int>(quads_of(hidden));

  constexpr int kChunk = 64 * kRowQuadsInFlight;  // quads per chunk
  f4u v[kRowQuadsInFlight];
  // REALIGN == false: rows of whole quads (hidden % 32 == 0); a lane past the
  // row's last quad loads that quad again (the top-2 copy stores it again, the
  // same bytes to the same place; the other copy skips it)
  auto load_chunk = [&](const float* src, int q0) {
#pragma unroll
    for (int u = 0; u < kRowQuadsInFlight; ++u) {
      const int q = q0 + lane + 64 * u;
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f4u*>(src + 4 * (q < cols ? q : cols - 1)));
    }
  };
  // REALIGN: quads [c0, c0 + kChunk) of the row's lines (nq quads from line0)
  // into v, and lanes 0..2 kRealignPad-1 the margin quads c0 - kRealignPad ..
  // c0 - 1 and c0 + kChunk .. c0 + kChunk + kRealignPad - 1 into `edge`.
  f4a edge = f4a{0.0F, 0.0F, 0.0F, 0.0F};
  auto load_lines = [&](const f4a* line0, int nq, int c0) {
#pragma unroll
    for (int u = 0; u < kRowQuadsInFlight; ++u) {
      const int q = c0 + lane + 64 * u;
      if (q < nq) {
        const f4a w = __builtin_nontemporal_load(line0 + q);
        v[u] = f4u{w.x, w.y, w.z, w.w};
      } else {
        v[u] = f4u{0.0F, 0.0F, 0.0F, 0.0F};
      }
    }
    const int eq = lane < kRealignPad ? c0 - kRealignPad + lane : c0 + kChunk + lane - kRealignPad;
    edge = f4a{0.0F, 0.0F, 0.0F, 0.0F};
    if (lane < 2 * kRealignPad && eq >= 0 && eq < nq) edge = __builtin_nontemporal_load(line0 + eq);
  };
  auto row_phase = [](const float* row) {  // floats from the row's 128-byte line to the row
    return static_cast<int>((reinterpret_cast<uintptr_t>(row) >> 2) & 31);
  };
  // The first row's first chunk stays in flight while the block ranks.
  const int t_first = t_begin + wave;
  int pre_t = -1, pre_c = 0;  // REALIGN: the chunk that v / edge hold
  if (t_first < t_end) {
    const float* src = x + static_cast<std::size_t>(t_first) * hidden;
    if constexpr (REALIGN) {
      // the first chunk straight into the wave's strip (global_load_lds,
      // nontemporal; the left margin of chunk 0 is never stored), the next
      // chunk into v / edge: two chunks in flight while the block ranks (C4
      // K = 4095: cold 88.3 -> 86.1 us, warm 84.4 -> 81.9 us)
      const int hs = row_phase(src);
      const float* l0 = src - hs;
      const int nq = (hidden + hs + 3) >> 2;
      float* strip0 = reinterpret_cast<float*>(lds + realign_strip_offset(experts, tokens_per_block, top_k)) +
                      wave * kRealignStripQuads * 4;
#pragma unroll
      for (int u = 0; u < kRowQuadsInFlight; ++u) {
        const int q = lane + 64 * u;
        __builtin_amdgcn_global_load_lds(l0 + 4 * (q < nq ? q : nq - 1), strip0 + 4 * (kRealignPad + 64 * u), 16, 0,
                                         2 /* nt */);
      }
      if (lane >= kRealignPad && lane < 2 * kRealignPad) {  // right margin: strip quads kChunk + lane
        const int q = kChunk + lane - kRealignPad;
        __builtin_amdgcn_global_load_lds(l0 + 4 * (q < nq ? q : nq - 1), strip0 + 4 * kChunk, 16, 0, 2 /* nt */);
      }
      pre_t = realign_chunks(hidden) > 1 ? t_first : t_first + kFusedWaves;
      pre_c = realign_chunks(hidden) > 1 ? kChunk : 0;
      if (pre_t < t_end) {
        const float* ps = x + static_cast<std::size_t>(pre_t) * hidden;
        const int hp = row_phase(ps);
        load_lines(reinterpret_cast<const f4a*>(ps - hp), (hidden + hp + 3) >> 2, pre_c);
      } else {
        pre_t = -1;
      }
    } else {
      load_chunk(src, 0);
      if (top_k == 2) {
        // ... and the top-2 copy's second step (this row's chunk 1, or the
        // wave's next row's chunk 0) goes straight into the wave's LDS block
        // (global_load_lds, nontemporal): two steps in flight while the block
        // ranks, no registers held (C4 cold 81.9 -> 81.0 us, warm 79.1 -> 76.7)
        const int nch = (cols + kChunk - 1) / kChunk;
        const int t1 = nch > 1 ? t_first : t_first + kFusedWaves;
        const int c1 = nch > 1 ? 1 : 0;
        if (t1 < t_end) {
          const float* s1 = x + static_cast<std::size_t>(t1) * hidden;
          float* pre = reinterpret_cast<float*>(lds + realign_strip_offset(experts, tokens_per_block, top_k)) +
                       wave * (kChunk * 4);
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            const int q = c1 * kChunk + lane + 64 * u;
            __builtin_amdgcn_global_load_lds(s1 + 4 * (q < cols ? q : cols - 1), pre + u * 256, 16, 0, 2 /* nt */);
          }
        }
      }
    }
  }

  // ---- rank phase (block-wide) ----
  for (int i = tid; i < kFusedWaves * experts; i += kThreads) wc[i] = 0;
  __syncthreads();
  // Count the shorter side of the block's first route: the routes before it,
  // or (past the middle) the routes from it on, whose per-expert counts are
  // subtracted from the expert's total offsets[e + 1] - offsets[e] below.
  const bool suffix = begin > routes - begin;
  const int c_lo = suffix ? begin : 0;
  const int c_hi = suffix ? routes : begin;
  {
    // 16-byte id loads, eight per lane in flight. E <= 16: per-lane packed
    // 8-bit counters (expert e in bits 8 (e % 8) of word e / 8; a lane counts
    // at most R / 256 <= 128 ids here), summed over the wave afterwards;
    // else one LDS atomic per id into the wave's row.
    constexpr int kBatch = 8;
    const bool few = experts <= 16;
    uint64_t packed[2] = {0, 0};
    for (int b0 = c_lo; b0 < c_hi; b0 += 4 * kThreads * kBatch) {
      i4u id[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int r = b0 + 4 * (tid + kThreads * u);
        if (r + 4 <= c_hi) {
          id[u] = *reinterpret_cast<const i4u*>(ids + r);
        } else {
          id[u] = i4u{-1, -1, -1, -1};
          for (int c = 0; r + c < c_hi; ++c) id[u][c] = ids[r + c];
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int v = id[u][c];
          if (static_cast<unsigned>(v) >= static_cast<unsigned>(experts)) continue;
          if (few) {
            const uint64_t one = uint64_t{1} << (8 * (v & 7));
            packed[0] += v < 8 ? one : 0;
            packed[1] += v < 8 ? 0 : one;
          } else {
            atomicAdd(wc + wave * experts + v, 1);
          }
        }
      }
    }
    if (few) {
      for (int e = 0; e < experts; ++e) {
        const int32_t n = static_cast<int32_t>((packed[e >> 3] >> (8 * (e & 7))) & 0xff);
        const int32_t total = __builtin_amdgcn_readlane(wave_inclusive_scan(n), 63);
        if (lane == 0) wc[wave * experts + e] = total;
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < experts; e += kThreads) {
    int32_t sum = 0;
    for (int w = 0; w < kFusedWaves; ++w) {
      sum += wc[w * experts + e];
      wc[w * experts + e] = 0;
    }
    base[e] = suffix ? offsets[e + 1] - offsets[e] - sum : sum;
  }
  __syncthreads();
  for (int sub = begin; sub < end; sub += kThreads) {
    const int r = sub + tid;
    const int id = r < end ? ids[r] : -1;
    const bool valid = id >= 0 && id < experts;
    const uint64_t active = __ballot(valid);
    const uint64_t mask = match_mask(static_cast<uint32_t>(valid ? id : 0), bits, active);
    const int rank = __popcll(mask & lanemask_lt());
    const bool leader = valid && rank == 0;
    if (leader) wc[wave * experts + id] = __popcll(mask);
    __syncthreads();
    for (int e = tid; e < experts; e += kThreads) {
      int32_t running = base[e];
      for (int w = 0; w < kFusedWaves; ++w) {
        const int32_t c = wc[w * experts + e];
        if (c != 0) {
          wc[w * experts + e] = running;
          running += c;
        }
      }
      base[e] = running;
    }
    __syncthreads();
    if (r < end) {
      int32_t pos = -1;
      if (valid) {
        pos = offsets[id] + wc[wave * experts + id] + rank;
        if (pos < 0 || pos >= routes) pos = -1;  // offsets inconsistent with ids
      }
      route_pos[r] = pos;
      slot[r - begin] = pos;
      if (sorted_route != nullptr && pos >= 0) sorted_route[pos] = r;
    }
    if (leader) wc[wave * experts + id] = 0;  // (as in rr_permute_rank_kernel)
    __syncthreads();  // slot entries and cleared rows before the next sub-chunk / the copy
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int e = tid; e < experts; e += kThreads) cursors[e] = base[e];
  }

  // ---- copy phase: wave w copies rows t_begin + w, + waves, ... ----
  if constexpr (REALIGN) {
    f4a* strip = reinterpret_cast<f4a*>(lds + realign_strip_offset(experts, tokens_per_block, top_k)) +
                 wave * kRealignStripQuads;
    const float* strip_f = reinterpret_cast<const float*>(strip);
    // Once a chunk sits in the strip its registers are free: the next chunk's
    // loads (this row's next or the wave's next row's first) are issued before
    // the current chunk's stores, so their latency runs under the stores.
    const int nch = realign_chunks(hidden);
    for (int t = t_first; t < t_end; t += kFusedWaves) {
      const float* src = x + static_cast<std::size_t>(t) * hidden;
      const int hs = row_phase(src);
      const f4a* line0 = reinterpret_cast<const f4a*>(src - hs);
      const int nq = (hidden + hs + 3) >> 2;
      const int32_t* my_slots = slot + (t - t_begin) * top_k;
      for (int c = 0; c < nch; ++c) {
        const int c0 = c * kChunk;
        const bool first = t == t_first && c == 0;  // (in the strip since before the rank phase)
        if (first) {
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads have landed
        } else {
          if (t != pre_t || c0 != pre_c) load_lines(line0, nq, c0);  // (not the chunk v holds: rare)
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            strip[kRealignPad + lane + 64 * u] = f4a{v[u].x, v[u].y, v[u].z, v[u].w};
          }
          if (lane < 2 * kRealignPad) strip[lane < kRealignPad ? lane : kChunk + lane] = edge;
        }
        wave_lds_sync();
        if (!first) {
          if (c + 1 < nch) {
            load_lines(line0, nq, c0 + kChunk);
            pre_t = t;
            pre_c = c0 + kChunk;
          } else if (t + kFusedWaves < t_end) {
            const float* next = src + static_cast<std::size_t>(kFusedWaves) * hidden;
            const int hn = row_phase(next);
            load_lines(reinterpret_cast<const f4a*>(next - hn), (hidden + hn + 3) >> 2, 0);
            pre_t = t + kFusedWaves;
            pre_c = 0;
          }
        }
        for (int j = 0; j < top_k; ++j) {
          const int32_t pos = my_slots[j];  // (one LDS address: a broadcast)
          if (pos < 0) continue;            // wave-uniform
          float* dst = x_permuted + static_cast<std::size_t>(pos) * hidden;
          const int hd = row_phase(dst);
          float* dline = dst - hd;
          const int nd = (hidden + hd + 3) >> 2;
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            const int i = c0 + lane + 64 * u;  // destination quad, from dline
            if (i < nd) {
              // floats 4 i - hd .. +3 of the row = strip floats from the chunk's margin
              const int off = 4 * (kRealignPad + lane + 64 * u) + hs - hd;
              const f4a o = f4a{strip_f[off], strip_f[off + 1], strip_f[off + 2], strip_f[off + 3]};
              const int f0 = 4 * i - hd;
              if (f0 >= 0 && f0 + 4 <= hidden) {
                __builtin_nontemporal_store(o, reinterpret_cast<f4a*>(dline + 4 * i));
              } else {
                for (int e = 0; e < 4; ++e) {
                  if (f0 + e >= 0 && f0 + e < hidden) dst[f0 + e] = o[e];
                }
              }
            }
          }
          if (c + 1 == nch && lane < kRealignPad) {
            // the row's last destination quads, past the chunk: each float of
            // the row (below hidden) lies in the strip (realign_chunks); the
            // others are neither read nor stored
            const int i = c0 + kChunk + lane;
            if (i < nd) {
              const int off = 4 * (kRealignPad + kChunk + lane) + hs - hd;
              const int f0 = 4 * i - hd;
              if (f0 + 4 <= hidden) {
                const f4a o = f4a{strip_f[off], strip_f[off + 1], strip_f[off + 2], strip_f[off + 3]};
                __builtin_nontemporal_store(o, reinterpret_cast<f4a*>(dline + 4 * i));
              } else {
                for (int e = 0; f0 + e < hidden; ++e) dst[f0 + e] = strip_f[off + e];
              }
            }
          }
        }
        wave_lds_sync();  // the strip's reads before the next chunk's writes
      }
    }
    return;
  }
  if (top_k == 2) {
    // Top-2 with every route of the wave's rows placed (one test per wave):
    // the next chunk (this row's next or the wave's next row's first) is
    // loaded before the current chunk's two stores, and every load and store
    // is issued unconditionally (lanes past the row's last quad repeat that
    // quad, the same bytes to the same place), so the compiler's wait before
    // a chunk's stores leaves the previous chunk's stores in flight (C4,
    // cold: 83.7 -> 82.3 us).
    bool placed = true;
    for (int t = t_first; t < t_end; t += kFusedWaves) {
      placed = placed && slot[(t - t_begin) * 2] >= 0 && slot[(t - t_begin) * 2 + 1] >= 0;
    }
    if (__builtin_amdgcn_readfirstlane(placed ? 1 : 0) != 0) {
      const int nchunks = (cols + kChunk - 1) / kChunk;
      f4u w[kRowQuadsInFlight] = {};  // (the last step loads nothing)
      int t = t_first, c = 0;
      while (t < t_end) {  // (wave-uniform)
        const int32_t p0 = __builtin_amdgcn_readfirstlane(slot[(t - t_begin) * 2]);
        const int32_t p1 = __builtin_amdgcn_readfirstlane(slot[(t - t_begin) * 2 + 1]);
        int tn = t, cn = c + 1;
        if (cn == nchunks) {
          cn = 0;
          tn = t + kFusedWaves;
        }
        if (tn < t_end) {
          if (t == t_first && c == 0) {
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads have landed
            const f4a* pre = reinterpret_cast<const f4a*>(lds + realign_strip_offset(experts, tokens_per_block, top_k)) +
                             wave * kChunk;
#pragma unroll
            for (int u = 0; u < kRowQuadsInFlight; ++u) {
              const f4a q4 = pre[64 * u + lane];
              w[u] = f4u{q4.x, q4.y, q4.z, q4.w};
            }
          } else {
            const float* nsrc = x + static_cast<std::size_t>(tn) * hidden;
#pragma unroll
            for (int u = 0; u < kRowQuadsInFlight; ++u) {
              const int q = cn * kChunk + lane + 64 * u;
              w[u] = __builtin_nontemporal_load(reinterpret_cast<const f4u*>(nsrc + 4 * (q < cols ? q : cols - 1)));
            }
          }
        }
        float* d0 = x_permuted + static_cast<std::size_t>(p0) * hidden;
        float* d1 = x_permuted + static_cast<std::size_t>(p1) * hidden;
#pragma unroll
        for (int u = 0; u < kRowQuadsInFlight; ++u) {
          const int q = c * kChunk + lane + 64 * u;
          __builtin_nontemporal_store(v[u], reinterpret_cast<f4u*>(d0 + 4 * (q < cols ? q : cols - 1)));
        }
#pragma unroll
        for (int u = 0; u < kRowQuadsInFlight; ++u) {
          const int q = c * kChunk + lane + 64 * u;
          __builtin_nontemporal_store(v[u], reinterpret_cast<f4u*>(d1 + 4 * (q < cols ? q : cols - 1)));
        }
#pragma unroll
        for (int u = 0; u < kRowQuadsInFlight; ++u) v[u] = w[u];
        t = tn;
        c = cn;
      }
      return;
    }
  }
  for (int t = t_first; t < t_end; t += kFusedWaves) {
    const float* src = x + static_cast<std::size_t>(t) * hidden;
    const int32_t* my_slots = slot + (t - t_begin) * top_k;
    for (int q0 = 0; q0 < cols; q0 += kChunk) {
      if (t != t_first || q0 != 0) load_chunk(src, q0);
      for (int j = 0; j < top_k; ++j) {
        const int32_t pos = my_slots[j];  // (one LDS address: a broadcast)
        if (pos < 0) continue;            // wave-uniform
        float* dst = x_permuted + static_cast<std::size_t>(pos) * hidden;
#pragma unroll
        for (int u = 0; u < kRowQuadsInFlight; ++u) {
          const int q = q0 + lane + 64 * u;
          if (q < cols) __builtin_nontemporal_store(v[u], reinterpret_cast<f4u*>(dst + 4 * q));
        }
      }
    }
  }
}

// ============================================================================
// Unpermute: y[t, :] = sum_j w[t*top_k + j] * y_permuted[route_pos[t*top_k + j], :]
// accumulated in rank order with separately rounded multiply and add, the
// operation order of the reference's FP32 loop (reference
// benchmarks/adapters/unpermute_adapter.cpp:67-73).
// ============================================================================
__global__ __launch_bounds__(256) void rr_unpermute_rows_kernel(const float* __restrict__ y_permuted,
                                                           const int32_t* __restrict__ route_pos,
                                                           const float* __restrict__ route_weights,
                                                           float* __restrict__ y, int tokens,
                                                           int top_k, int output) {
  // Token-owned rows as in the permute copy: lane j < top_k reads route j's
  // position and weight once per row. y_permuted rows are read once, with
  // nontemporal loads (C4 unpermute 265 -> 255 us).
  const int lane = lane_id();
  const int cols = static_cast<int>(quads_of(output));
  const int waves = static_cast<int>(gridDim.x) * 4;
  const int routes = tokens * top_k;
  for (int t = static_cast<int>(blockIdx.x) * 4 + (static_cast<int>(threadIdx.x) >> 6); t < tokens;
       t += waves) {
    const std::size_t r0 = static_cast<std::size_t>(t) * top_k;
    const int32_t my_pos = lane < top_k ? route_pos[r0 + lane] : -1;
    const float my_w = lane < top_k ? route_weights[r0 + lane] : 0.0F;
    float* out = y + static_cast<std::size_t>(t) * output;
    for (int q0 = 0; q0 < cols; q0 += 64 * kRowQuadsInFlight) {  // wave-uniform: readlane needs every lane
      f4u acc[kRowQuadsInFlight];
#pragma unroll
      for (int u = 0; u < kRowQuadsInFlight; ++u) acc[u] = f4u{0.0F, 0.0F, 0.0F, 0.0F};
      for (int j = 0; j < top_k; j += 2) {  // two routes' loads in flight, summed in rank order
        const int32_t p0 = __builtin_amdgcn_readlane(my_pos, j);
        const int32_t p1 = j + 1 < top_k ? __builtin_amdgcn_readlane(my_pos, j + 1) : -1;
        const bool ok0 = p0 >= 0 && p0 < routes;  // wave-uniform
        const bool ok1 = p1 >= 0 && p1 < routes;
        const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), j));
        const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), j + 1 < top_k ? j + 1 : j));
        // An invalid position reads row 0 (present: routes > 0) and is not summed.
        const float* s0 = y_permuted + static_cast<std::size_t>(ok0 ? p0 : 0) * output;
        const float* s1 = y_permuted + static_cast<std::size_t>(ok1 ? p1 : 0) * output;
        f4u v0[kRowQuadsInFlight], v1[kRowQuadsInFlight];
#pragma unroll
        for (int u = 0; u < kRowQuadsInFlight; ++u) {
          const int k0 = 4 * (q0 + lane + 64 * u);
          if (k0 + 4 <= output) {
            v0[u] = __builtin_nontemporal_load(reinterpret_cast<const f4u*>(s0 + k0));
            v1[u] = __builtin_nontemporal_load(reinterpret_cast<const f4u*>(s1 + k0));
          } else {
            v0[u] = f4u{0.0F, 0.0F, 0.0F, 0.0F};
            v1[u] = v0[u];
            for (int e = 0; k0 + e < output; ++e) {
              v0[u][e] = s0[k0 + e];
              v1[u][e] = s1[k0 + e];
            }
          }
        }
        if (ok0) {
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            acc[u].x = __fadd_rn(acc[u].x, __fmul_rn(w0, v0[u].x));
            acc[u].y = __fadd_rn(acc[u].y, __fmul_rn(w0, v0[u].y));
            acc[u].z = __fadd_rn(acc[u].z, __fmul_rn(w0, v0[u].z));
            acc[u].w = __fadd_rn(acc[u].w, __fmul_rn(w0, v0[u].w));
          }
        }
        if (ok1) {
#pragma unroll
          for (int u = 0; u < kRowQuadsInFlight; ++u) {
            acc[u].x = __fadd_rn(acc[u].x, __fmul_rn(w1, v1[u].x));
            acc[u].y = __fadd_rn(acc[u].y, __fmul_rn(w1, v1[u].y));
            acc[u].z = __fadd_rn(acc[u].z, __fmul_rn(w1, v1[u].z));
            acc[u].w = __fadd_rn(acc[u].w, __fmul_rn(w1, v1[u].w));
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kRowQuadsInFlight; ++u) {
        const int k0 = 4 * (q0 + lane + 64 * u);
        if (k0 + 4 <= output) {
          __builtin_nontemporal_store(acc[u], reinterpret_cast<f4u*>(out + k0));
        } else {
          for (int e = 0; k0 + e < output; ++e) out[k0 + e] = acc[u][e];
        }
      }
    }
  }
}

// Row kernels index a row's floats with int (quad offsets run up to 1024 past the width).
constexpr int kMaxRowWidth = INT_MAX - 4096;

// Row width (floats) from which the token-owned row kernels are used.
constexpr int kWideRow = 1024;

unsigned stream_grid(uint64_t items) {
  // Enough blocks to cover 256 CUs several times; grid-stride beyond that.
  const uint64_t blocks = (items + 255) / 256;
  return static_cast<unsigned>(blocks < 8192 ? (blocks == 0 ? 1 : blocks) : 8192);
}

unsigned row_grid(int rows) {
  // One wave per row, four waves per block, one block per CU, grid-stride
  // beyond that (C4 unpermute, 57 KB rows: 324 us with 128 blocks, 264 with
  // 256, 271 with 512, 272 with one wave per token).
  const int blocks = (rows + 3) / 4;
  return static_cast<unsigned>(blocks < 256 ? (blocks == 0 ? 1 : blocks) : 256);
}

unsigned copy_row_grid(int rows) {
  // One wave per row, four waves per block, four blocks per CU (the copy's
  // nontemporal loads want more rows in flight than the unpermute's).
  const int blocks = (rows + 3) / 4;
  return static_cast<unsigned>(blocks < 1024 ? (blocks == 0 ? 1 : blocks) : 1024);
}

hipError_t launch_permute_copy(const float* x, const int32_t* route_pos, float* x_permuted,
                               int tokens, int top_k, int hidden, int routes, hipStream_t stream) {
  if (hidden >= kWideRow) {
    if (hidden > kMaxRowWidth) return hipErrorInvalidValue;
    rr_permute_rows_kernel<<<copy_row_grid(tokens), 256, 0, stream>>>(x, route_pos, x_permuted, tokens,
                                                                      top_k, hidden, routes);
  } else {
    const uint64_t items = static_cast<uint64_t>(tokens) * quads_of(hidden);
    if (items >= (uint64_t{1} << 32)) return hipErrorInvalidValue;  // 32-bit item indices
    const unsigned grid = stream_grid(items);
    if (top_k <= 2) {
      rr_permute_copy_kernel<2><<<grid, 256, 0, stream>>>(x, route_pos, x_permuted, tokens, top_k, hidden, routes);
    } else if (top_k <= 4) {
      rr_permute_copy_kernel<4><<<grid, 256, 0, stream>>>(x, route_pos, x_permuted, tokens, top_k, hidden, routes);
    } else if (top_k <= 8) {
      rr_permute_copy_kernel<8><<<grid, 256, 0, stream>>>(x, route_pos, x_permuted, tokens, top_k, hidden, routes);
    } else {
      rr_permute_copy_kernel<0><<<grid, 256, 0, stream>>>(x, route_pos, x_permuted, tokens, top_k, hidden, routes);
    }
  }
  return hipGetLastError();
}

}  // namespace

hipError_t topk_gate_wave(const float* logits, int32_t* ids, float* weights, int tokens,
                          int experts, hipStream_t stream, float* y_zero, int y_cols) {
  if (tokens <= 0) return hipSuccess;
  const bool vec4 = (experts % 4 == 0) && aligned16(logits);
  const int per_lane_units = vec4 ? experts / 4 : (experts + 3) / 4;
  int lpr = 1;
  while (lpr < per_lane_units && lpr < 64) lpr <<= 1;
  switch (lpr) {
    case 1: return launch_gate<1>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    case 2: return launch_gate<2>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    case 4: return launch_gate<4>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    case 8: return launch_gate<8>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    case 16: return launch_gate<16>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    case 32: return launch_gate<32>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
    default: return launch_gate<64>(logits, ids, weights, tokens, experts, vec4, y_zero, y_cols, stream);
  }
}

hipError_t histogram_native(const int32_t* ids, int32_t* counts, int routes, int experts,
                            hipStream_t stream) {
  if (experts == 1) {
    rr_single_bin_kernel<<<1, 1, 0, stream>>>(counts, nullptr, routes);
    return hipGetLastError();
  }
  if (routes <= kSingleBlockRoutes) {
    rr_hist_scan_single_kernel<<<1, kBlock, bins_bytes(experts), stream>>>(
        ids, counts, nullptr, routes, experts);
    return hipGetLastError();
  }
  return histogram_atomic(ids, counts, nullptr, routes, experts, stream);
}

hipError_t exclusive_scan_native(const int32_t* counts, int32_t* offsets, int experts,
                                 hipStream_t stream) {
  rr_scan_kernel<<<1, kBlock, 0, stream>>>(counts, offsets, experts);
  return hipGetLastError();
}

hipError_t histogram_exclusive_scan_native(const int32_t* ids, int32_t* counts, int32_t* offsets,
                                           int routes, int experts, hipStream_t stream) {
  if (experts == 1) {
    rr_single_bin_kernel<<<1, 1, 0, stream>>>(counts, offsets, routes);
    return hipGetLastError();
  }
  if (routes <= kSingleBlockRoutes) {
    rr_hist_scan_single_kernel<<<1, kBlock, bins_bytes(experts), stream>>>(
        ids, counts, offsets, routes, experts);
    return hipGetLastError();
  }
  return histogram_atomic(ids, counts, offsets, routes, experts, stream);
}

hipError_t token_permute_stable(const float* x, const int32_t* ids, const int32_t* offsets,
                                int32_t* cursors, float* x_permuted, int32_t* route_pos,
                                int32_t* sorted_route, int tokens, int experts, int top_k,
                                int hidden, hipStream_t stream) {
  const int routes = tokens * top_k;
  if (routes <= 0) return hipSuccess;
  if (hidden >= kWideRow && hidden <= kMaxRowWidth && routes <= kFusedRankRoutes) {
    // rank + copy in one launch: up to four blocks per CU, whole tokens each
    const int grid = tokens < 1024 ? tokens : 1024;
    const int tpb = (tokens + grid - 1) / grid;
    const int blocks = (tokens + tpb - 1) / tpb;
    const bool lines = hidden % 32 == 0 && reinterpret_cast<uintptr_t>(x) % 128 == 0 &&
                       reinterpret_cast<uintptr_t>(x_permuted) % 128 == 0;
    if (lines) {
      const std::size_t lds = static_cast<std::size_t>(realign_strip_offset(experts, tpb, top_k)) * sizeof(int32_t) +
                              (top_k == 2 ? static_cast<std::size_t>(kFusedWaves) * 64 * kRowQuadsInFlight * 16 : 0);
      rr_permute_rank_rows_kernel<false><<<blocks, kFusedWaves * 64, lds, stream>>>(
          x, ids, offsets, cursors, x_permuted, route_pos, sorted_route, tokens, top_k, hidden, experts,
          bits_for(experts), tpb);
    } else {
      // top_k <= E <= 1024 (the entry's checks) and tpb * top_k <= 32 + top_k: under 59 KB
      const std::size_t lds = static_cast<std::size_t>(realign_strip_offset(experts, tpb, top_k)) * sizeof(int32_t) +
                              static_cast<std::size_t>(kFusedWaves) * kRealignStripQuads * sizeof(f4a);
      if (lds > 64 * 1024) return hipErrorInvalidValue;
      rr_permute_rank_rows_kernel<true><<<blocks, kFusedWaves * 64, lds, stream>>>(
          x, ids, offsets, cursors, x_permuted, route_pos, sorted_route, tokens, top_k, hidden, experts,
          bits_for(experts), tpb);
    }
    return hipGetLastError();
  }
  // One sub-chunk per block up to 64 blocks; beyond that the chunk grows so the
  // recomputed prefix stays bounded by 64 chunks. 16 waves while (16 + 1) LDS
  // rows of E ints fit in 34 KB, else 8 waves.
  const bool wide = experts > 512;
  const int threads = wide ? 512 : 1024;
  int chunk = threads;
  if (routes > 64 * threads) chunk = ((routes + 63) / 64 + threads - 1) / threads * threads;
  const int blocks = (routes + chunk - 1) / chunk;
  const std::size_t lds = (static_cast<std::size_t>(threads / 64) + 1) * experts * sizeof(int32_t);
  if (wide) {
    rr_permute_rank_kernel<8><<<blocks, threads, lds, stream>>>(
        ids, offsets, cursors, route_pos, sorted_route, routes, experts, bits_for(experts), chunk);
  } else {
    rr_permute_rank_kernel<16><<<blocks, threads, lds, stream>>>(
        ids, offsets, cursors, route_pos, sorted_route, routes, experts, bits_for(experts), chunk);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || hidden == 0) return err;
  return launch_permute_copy(x, route_pos, x_permuted, tokens, top_k, hidden, routes, stream);
}

hipError_t route_prep(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* cursors,
                      int32_t* route_pos, int32_t* sorted_route, int routes, int experts,
                      hipStream_t stream) {
  if (routes <= 0) return hipSuccess;
  const bool wide = experts > 512;
  const int threads = wide ? 512 : 1024;
  int chunk = threads;
  if (routes > 64 * threads) chunk = ((routes + 63) / 64 + threads - 1) / threads * threads;
  const int blocks = (routes + chunk - 1) / chunk;
  const std::size_t lds =
      ((static_cast<std::size_t>(threads / 64) + 2) * experts + 1 + kWavesPerBlock) * sizeof(int32_t);
  if (wide) {
    rr_route_prep_kernel<8><<<blocks, threads, lds, stream>>>(ids, counts, offsets, cursors, route_pos,
                                                              sorted_route, routes, experts,
                                                              bits_for(experts), chunk);
  } else {
    rr_route_prep_kernel<16><<<blocks, threads, lds, stream>>>(ids, counts, offsets, cursors, route_pos,
                                                               sorted_route, routes, experts,
                                                               bits_for(experts), chunk);
  }
  return hipGetLastError();
}

hipError_t permute_copy(const float* x, const int32_t* route_pos, float* x_permuted, int tokens,
                        int top_k, int hidden, hipStream_t stream) {
  const int routes = tokens * top_k;
  if (routes <= 0 || hidden <= 0) return hipSuccess;
  return launch_permute_copy(x, route_pos, x_permuted, tokens, top_k, hidden, routes, stream);
}

hipError_t unpermute_gather(const float* y_permuted, const int32_t* route_pos,
                            const float* route_weights, float* y, int tokens, int top_k,
                            int output, hipStream_t stream) {
  if (tokens <= 0 || output <= 0) return hipSuccess;
  if (output >= kWideRow) {
    if (output > kMaxRowWidth) return hipErrorInvalidValue;
    rr_unpermute_rows_kernel<<<row_grid(tokens), 256, 0, stream>>>(y_permuted, route_pos,
                                                                   route_weights, y, tokens, top_k,
                                                                   output);
  } else {
    const uint64_t items = static_cast<uint64_t>(tokens) * quads_of(output);
    if (items >= (uint64_t{1} << 32)) return hipErrorInvalidValue;  // 32-bit item indices
    const unsigned grid = stream_grid(items);
    if (top_k <= 2) {
      rr_unpermute_kernel<2><<<grid, 256, 0, stream>>>(y_permuted, route_pos, route_weights, y, tokens, top_k, output);
    } else if (top_k <= 4) {
      rr_unpermute_kernel<4><<<grid, 256, 0, stream>>>(y_permuted, route_pos, route_weights, y, tokens, top_k, output);
    } else if (top_k <= 8) {
      rr_unpermute_kernel<8><<<grid, 256, 0, stream>>>(y_permuted, route_pos, route_weights, y, tokens, top_k, output);
    } else {
      rr_unpermute_kernel<0><<<grid, 256, 0, stream>>>(y_permuted, route_pos, route_weights, y, tokens, top_k, output);
    }
  }
  return hipGetLastError();
}

}  // namespace rr::kern
