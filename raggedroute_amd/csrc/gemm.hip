// FP32 GEMMs on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// One persistent kernel serves the router dense GEMM (one segment of M rows),
// the ragged grouped GEMM (segments [offsets[e], offsets[e+1]) with weights
// W[e]) and the chain's gathered expert GEMM with the unpermute in its
// epilogue, for shapes the narrow-output strip kernel (strip.hip) does not
// cover. The host never
// reads offsets: every workgroup loads them to LDS, builds the per-expert
// row-tile prefix and walks the tile space (row tiles of every expert x column
// tiles) with a grid-stride loop.
//
// Tile: BM x BN per workgroup, BK per LDS stage (32 for the large tile, 64 for
// short-K tiles), two LDS stages plus a register prefetch of the next stage.
// LDS holds both operands k-contiguous ([m][k] and [n][k], rows padded by 4
// floats) so every MFMA operand fetch is one ds_read_b128 covering four
// consecutive MFMA k-steps. Lane l (group g = l / 16, index i = l % 16)
// supplies A[m0 + i][k] and B[k][n0 + i] for k = kk + 4g + s at MFMA step s,
// which is the same k for both operands. The k order of the accumulation does
// not depend on the tile shape, so every tile configuration (and every fused
// form) produces bit-identical products.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "launchers.h"
#include "raggedroute_capi.h"
#include "wave.h"

namespace rr::kern {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kGroupM = 8;  // row tiles per swizzle group
constexpr int kXcds = 8;    // MI355X: 8 XCDs, workgroups dispatched round-robin

enum Mode : int {
  kDense = 0,         // one segment [0, dense_rows), weights W
  kGrouped = 1,       // segments from offsets, weights W[e]
  kChainGrouped = 2,  // grouped with A rows gathered through sorted_route, x_permuted
                      // written, and the top-2 unpermute folded into the epilogue
};

struct GemmParams {
  const float* X;
  const float* W;
  const int32_t* offsets;
  float* Y;
  int experts;
  int dense_rows;
  int K;
  int N;
  // kChainGrouped: segment row r holds token sorted_route[r] / top_k of X; the
  // gathered rows go to x_permuted (when given) and, when y_out is given
  // (top-2), y_out[token] += route_weights[route] * Y[r].
  const int32_t* sorted_route;
  const float* route_weights;
  float* x_permuted;
  float* y_out;
  int top_k;
};

template <int BM_, int BN_, int WM_, int WN_, int BK_>
struct TileShape {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int WM = WM_;
  static constexpr int WN = WN_;
  static constexpr int BK = BK_;
  static constexpr int kLd = BK + 4;  // padded LDS row (floats)
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int kTM = BM / WM / 16;  // 16x16 MFMA tiles per wave along M
  static constexpr int kTN = BN / WN / 16;
  static constexpr int kALoads = BM * BK / 4 / kThreads;  // float4 slots per thread
  static constexpr int kBLoads = BN * BK / 4 / kThreads;
  static constexpr int kStageFloats = (BM + BN) * kLd;
  // BK >= 128 tiles stage the whole K extent of a short-K problem at once: one
  // global round trip and one barrier per tile, a single LDS stage.
  static constexpr int kStages = BK >= 128 ? 1 : 2;
  static_assert(BK % 16 == 0 && (BK & (BK - 1)) == 0, "BK is a power of two >= 16");
  static_assert(kTM >= 1 && kTN >= 1, "wave tile below one MFMA tile");
  static_assert(kALoads >= 1 && kBLoads >= 1, "tile too small for the block");
  static_assert(BM * BK / 4 % kThreads == 0 && BN * BK / 4 % kThreads == 0, "uneven loads");
};

// Global -> register staging of one BK slice. A rows are k-contiguous in
// global memory; B rows are n-contiguous and are transposed on the LDS store.
// set_rows resolves, once per tile, the A row behind each of the thread's A
// slots: src_rows (LDS, optional) maps tile row r to its source row of A (-1:
// none); without it tile row r is row row0 + r, valid below row_end. (Loading from
// clamped addresses and zeroing at the LDS store, as the strip kernel does,
// measured slower here: C4 grouped GEMM 17.1 ms against 15.6 ms, the selects
// adding VALU work to every k step of an MFMA-bound loop.)
// 16-byte vector that needs only 4-byte alignment: gfx950 global memory takes
// unaligned vector accesses, so rows of widths that are not multiples of 4 load
// whole quads with one instruction.
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

template <class S, bool VEC>
struct Stage {
  float a[S::kALoads][4];
  float b[S::kBLoads][4];
  // A slot p reads row src[p] of A (-1: no row; the slot loads zeros). The
  // slots keep row indices, not pointers: per-slot 64-bit addresses of both
  // prefetch stages pushed the 128 x 128 register-staged tile past 256 VGPRs.
  int src[S::kALoads];
  const float* a_base;
  float* xp_base;  // chain: x_permuted (nullptr: not written)
  int xp_row0;     // x_permuted row of the tile's first row

  // Once per tile: the thread's A slots (and x_permuted rows, when given).
  __device__ __forceinline__ void set_rows(const float* __restrict__ A, const int32_t* src_rows,
                                           int row0, int row_end, int K, float* x_permuted,
                                           int tid) {
    (void)K;
    a_base = A;
    xp_base = x_permuted;
    xp_row0 = row0;
#pragma unroll
    for (int p = 0; p < S::kALoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int r = f / (S::BK / 4);  // BK / 4 float4 per row
      src[p] = src_rows != nullptr ? src_rows[r] : (row0 + r < row_end ? row0 + r : -1);
    }
  }

  __device__ __forceinline__ void load(const float* __restrict__ B, int n0, int N, int K, int k0,
                                       int tid) {
#pragma unroll
    for (int p = 0; p < S::kALoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int c = (f % (S::BK / 4)) * 4;
      const int k = k0 + c;
      const bool has_row = src[p] >= 0;
      const float* ptr = a_base + static_cast<std::size_t>(has_row ? src[p] : 0) * K + k;
      if (VEC) {
        if (has_row && k < K) {
          const float4 v = *reinterpret_cast<const float4*>(ptr);
          a[p][0] = v.x; a[p][1] = v.y; a[p][2] = v.z; a[p][3] = v.w;
        } else {
          a[p][0] = a[p][1] = a[p][2] = a[p][3] = 0.0F;
        }
      } else if (has_row && k + 3 < K) {  // whole quad: one 16-byte load (4-byte aligned)
        const f4u v = *reinterpret_cast<const f4u*>(ptr);
        a[p][0] = v.x; a[p][1] = v.y; a[p][2] = v.z; a[p][3] = v.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) a[p][j] = (has_row && k + j < K) ? ptr[j] : 0.0F;
      }
    }
#pragma unroll
    for (int p = 0; p < S::kBLoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int kr = f & (S::BK - 1);  // k varies fastest across lanes
      const int n = (f / S::BK) * 4;
      const int k = k0 + kr;
      const int col = n0 + n;
      const float* ptr = B + static_cast<std::size_t>(k) * N + col;
      if (VEC) {
        if (k < K && col < N) {
          const float4 v = *reinterpret_cast<const float4*>(ptr);
          b[p][0] = v.x; b[p][1] = v.y; b[p][2] = v.z; b[p][3] = v.w;
        } else {
          b[p][0] = b[p][1] = b[p][2] = b[p][3] = 0.0F;
        }
      } else if (k < K && col + 3 < N) {  // whole quad: one 16-byte load (4-byte aligned)
        const f4u v = *reinterpret_cast<const f4u*>(ptr);
        b[p][0] = v.x; b[p][1] = v.y; b[p][2] = v.z; b[p][3] = v.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) b[p][j] = (k < K && col + j < N) ? ptr[j] : 0.0F;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ lds, int tid) const {
    float* As = lds;
    float* Bs = lds + S::BM * S::kLd;
#pragma unroll
    for (int p = 0; p < S::kALoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int r = f / (S::BK / 4);
      const int c = (f % (S::BK / 4)) * 4;
      *reinterpret_cast<float4*>(As + r * S::kLd + c) =
          make_float4(a[p][0], a[p][1], a[p][2], a[p][3]);
    }
#pragma unroll
    for (int p = 0; p < S::kBLoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int kr = f & (S::BK - 1);
      const int n = (f / S::BK) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) Bs[(n + j) * S::kLd + kr] = b[p][j];
    }
  }

  // Writes the staged A slice to the x_permuted rows of the tile (the gathered
  // rows of the chain), valid rows and columns only.
  __device__ __forceinline__ void store_a_rows(int K, int k0, int tid) const {
#pragma unroll
    for (int p = 0; p < S::kALoads; ++p) {
      const int f = tid + p * S::kThreads;
      const int c = (f % (S::BK / 4)) * 4;
      const int k = k0 + c;
      if (xp_base == nullptr || src[p] < 0) continue;
      float* ptr = xp_base + static_cast<std::size_t>(xp_row0 + f / (S::BK / 4)) * K + k;
      if (VEC) {
        if (k < K) __builtin_nontemporal_store(v4f{a[p][0], a[p][1], a[p][2], a[p][3]}, reinterpret_cast<v4f*>(ptr));
      } else if (k + 3 < K) {
        *reinterpret_cast<f4u*>(ptr) = f4u{a[p][0], a[p][1], a[p][2], a[p][3]};
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (k + j < K) ptr[j] = a[p][j];
        }
      }
    }
  }
};

// Direct global -> LDS staging (gfx950 global_load_lds_dwordx4) for the
// 128 x 128 x 32 tile when K is a multiple of 32: one wave instruction fills
// one contiguous KiB of LDS, lane L the 16 bytes at L * 16, so the layouts are
// chosen by which global chunk each lane fetches. No staging registers, no LDS
// store instructions, no transposition.
//   A stage [128 rows][8 slots of 4 k]: slot s of row r holds k chunk
//     s ^ swa(r). A lane of an MFMA operand read takes row r = base + li and
//     one k chunk: the 16 rows of a lane group land in 16 distinct 16-byte
//     bank groups (and any 8 consecutive rows in 8).
//   B stage [32 k rows][32 slots of 4 n] (B's own row-major order): slot s of
//     row k holds n chunk s ^ swb(k). An operand read takes one float per lane
//     at rows k = kk + 4g + s: the four lane groups read XOR-separated chunks,
//     64 distinct banks, and rows s, s + 1 pair into one ds_read2st64_b32.
// The MFMA k order is the register-staged kernel's (k = kk + 4g + s at step s),
// so both staging paths give bit-identical products.
struct DmaLayout {
  static constexpr int kRowsA = 128, kBK = 32, kColsB = 128;
  static constexpr int kAFloats = kRowsA * kBK;   // 4096
  static constexpr int kStageFloats = kAFloats + kBK * kColsB;  // 8192 = 32 KiB
  static constexpr int kBlockFloats = 256;         // one wave instruction: 64 lanes x 16 B
  __device__ static int swa(int r) { return (r ^ (r >> 3)) & 7; }
  __device__ static int swb(int k) { return 4 * ((k >> 2) & 3); }
};

// One 16-deep k chunk of a wave tile: MFMA step s (k = kk + 4g + s) of every
// 16x16 tile before step s + 1 of any. Each accumulator still sums its steps
// in ascending order, so the products are those of a tile-by-tile loop, but
// consecutive MFMAs write different accumulators: a step never waits for the
// result of the one issued just before it (a dependent MFMA on the same
// accumulator issues about 12 cycles later than an independent one).
template <int TM, int TN>
__device__ __forceinline__ void mfma_steps(v4f (&acc)[TM][TN], const v4f (&af)[TM], const v4f (&bf)[TN]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
      }
    }
  }
}

// Tile space decode: row tiles are grouped kGroupM at a time so that workgroups
// running together share both A row blocks and B column strips.
__device__ __forceinline__ void decode_tile(int t, int row_tiles, int col_tiles, int* rt, int* ct) {
  const int group_size = kGroupM * col_tiles;
  const int group = t / group_size;
  const int first = group * kGroupM;
  const int rows_in_group = row_tiles - first < kGroupM ? row_tiles - first : kGroupM;
  const int within = t - group * group_size;
  *rt = first + within % rows_in_group;
  *ct = within / rows_in_group;
}

// Wave layouts of a tile's MFMA work. WaveLayout: the tile shape's WM x WN
// grid of (BM / WM) x (BN / WN) wave tiles. SlabLayout: every wave takes all
// TM 16-row blocks of the tile's top rows and a COLS-wide column slab.
template <int TM_, int TN_, class S>
struct WaveLayout {
  static constexpr int kTM = TM_;
  static constexpr int kTN = TN_;
  __device__ static int wm0(int wave) { return (wave / S::WN) * (S::BM / S::WM); }
  __device__ static int wn0(int wave) { return (wave % S::WN) * (S::BN / S::WN); }
};
template <int TM_, int TN_, int COLS>
struct SlabLayout {
  static constexpr int kTM = TM_;
  static constexpr int kTN = TN_;
  __device__ static int wm0(int) { return 0; }
  __device__ static int wn0(int wave) { return wave * COLS; }
};

// Staging of the k slices: registers, or direct loads into LDS (whole
// 32-deep slices and 16-byte rows), or direct loads at any row alignment and
// any K (the last slice's chunks past K, and at the end of W past N, fixed up
// in LDS).
enum Staging : int { kRegisters = 0, kDirect = 1, kDirectAnyAlign = 2 };

template <class S, bool VEC, int MODE, int DMA>
__global__ __launch_bounds__(S::kThreads, 2) void rr_gemm_mfma_kernel(GemmParams prm) {
  constexpr bool kGroupedRows = MODE == kGrouped || MODE == kChainGrouped;
  // slab layouts for tiles of at most 64 rows (the 128 x 128 tile, 2 x 2 waves)
  constexpr bool kSlabs = S::BM == 128 && S::BN == 128 && S::WM == 2 && S::WN == 2;
  static_assert(DMA == kRegisters || (kSlabs && S::BK == DmaLayout::kBK && (VEC || DMA == kDirectAnyAlign)),
                "DMA staging: the 128 x 128 x 32 tile");
  static_assert(DMA != kDirectAnyAlign || MODE != kChainGrouped, "any-alignment staging: dense and grouped");
  constexpr int kStageFloats = DMA ? DmaLayout::kStageFloats : S::kStageFloats;
  extern __shared__ float lds[];
  float* stages = lds;                                                             // kStages
  int32_t* s_off = reinterpret_cast<int32_t*>(lds + S::kStages * kStageFloats);  // [E + 1]
  int32_t* s_pre = s_off + prm.experts + 1;   // [E + 1] full row tiles before expert e
  int32_t* s_pre2 = s_pre + prm.experts + 1;  // [E + 1] short row tiles before expert e
  int32_t* s_src = s_pre2 + prm.experts + 1;  // [BM] chain: token row of X per tile row
  float* s_w = reinterpret_cast<float*>(s_src + S::BM);  // [BM] chain: route weight per tile row
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = rr::dev::lane_id();
  const int wave = tid >> 6;
  const int experts = prm.experts;
  const int K = prm.K;
  const int N = prm.N;

  // ---- device-side scheduler: per-expert row-tile prefixes in LDS ----
  // With slab layouts (below) an expert's last row tile is "short" when it
  // holds at most BM / 2 rows: its MFMA work is a fraction of a full tile's.
  // The tile space lists every full tile first and the short ones after, so
  // the grid-stride rounds finish on cheap tiles instead of putting a short
  // tile's worker behind a full round.
  for (int e = tid; e <= experts; e += S::kThreads) {
    s_off[e] = kGroupedRows ? prm.offsets[e] : (e == 0 ? 0 : prm.dense_rows);
  }
  __syncthreads();
  auto full_tiles = [](int32_t cnt) -> int32_t {
    if (cnt <= 0) return 0;
    if constexpr (kSlabs) return cnt / S::BM + (cnt % S::BM > S::BM / 2 ? 1 : 0);
    return (cnt + S::BM - 1) / S::BM;
  };
  auto short_tiles = [](int32_t cnt) -> int32_t {
    if constexpr (kSlabs) return cnt > 0 && cnt % S::BM != 0 && cnt % S::BM <= S::BM / 2 ? 1 : 0;
    return 0;
  };
  if (wave == 0) {
    // Lane l owns experts [l*per, (l+1)*per); experts <= 1024 -> per <= 16.
    const int per = (experts + 63) / 64;
    int32_t local = 0, local2 = 0;
    for (int j = 0; j < per; ++j) {
      const int e = lane * per + j;
      if (e < experts) {
        const int32_t cnt = s_off[e + 1] - s_off[e];
        local += full_tiles(cnt);
        local2 += short_tiles(cnt);
      }
    }
    const int32_t incl = rr::dev::wave_inclusive_scan(local);
    const int32_t incl2 = rr::dev::wave_inclusive_scan(local2);
    int32_t run = incl - local, run2 = incl2 - local2;
    for (int j = 0; j < per; ++j) {
      const int e = lane * per + j;
      if (e < experts) {
        s_pre[e] = run;
        s_pre2[e] = run2;
        const int32_t cnt = s_off[e + 1] - s_off[e];
        run += full_tiles(cnt);
        run2 += short_tiles(cnt);
      }
    }
    if (lane == 63) {
      s_pre[experts] = incl;
      s_pre2[experts] = incl2;
    }
  }
  __syncthreads();
  const int full_rows = s_pre[experts];
  const int short_rows = s_pre2[experts];
  const int col_tiles = (N + S::BN - 1) / S::BN;
  const long total_full = static_cast<long>(full_rows) * col_tiles;
  const long total = total_full + static_cast<long>(short_rows) * col_tiles;

  // Workgroups are dispatched round-robin over the XCDs; give the workgroups
  // of one XCD consecutive tile ids so their operands meet in the same L2.
  const int grid = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  const int worker = (grid % kXcds == 0) ? (b % kXcds) * (grid / kXcds) + b / kXcds : b;

  const int g = lane >> 4;
  const int li = lane & 15;
  const int nk = (K + S::BK - 1) / S::BK;

  for (long t = worker; t < total; t += grid) {
    const bool is_short = t >= total_full;
    const int32_t* pre = is_short ? s_pre2 : s_pre;
    int rt, ct;
    decode_tile(static_cast<int>(is_short ? t - total_full : t), is_short ? short_rows : full_rows,
                col_tiles, &rt, &ct);
    // expert = last e with pre[e] <= rt (binary search over the prefix)
    int lo = 0, hi = experts - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= rt) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    // a short tile is its expert's last: the rows past its full tiles
    const int row0 = s_off[e] + (is_short ? (s_off[e + 1] - s_off[e]) / S::BM : rt - s_pre[e]) * S::BM;
    const int row_end = s_off[e + 1];
    const int n0 = ct * S::BN;
    const float* B = prm.W + static_cast<std::size_t>(kGroupedRows ? e : 0) * K * N;

    const int32_t* src_rows = nullptr;
    if constexpr (MODE == kChainGrouped) {
      __syncthreads();  // the previous tile's epilogue is done with s_src / s_w
      for (int r = tid; r < S::BM; r += S::kThreads) {
        const int row = row0 + r;
        int32_t token = -1;
        float w = 0.0F;
        if (row < row_end) {
          const int32_t route = prm.sorted_route[row];
          token = route / prm.top_k;  // route = top_k * token + rank
          if (prm.y_out != nullptr) w = prm.route_weights[route];
        }
        s_src[r] = token;
        s_w[r] = w;
      }
      __syncthreads();
      src_rows = s_src;
    }
    // Gathered rows go to x_permuted spread over the column tiles: tile ct
    // writes the k slices kt with kt % col_tiles == ct (every column tile
    // loads all of the rows' k slices anyway).
    const bool write_xp = MODE == kChainGrouped && prm.x_permuted != nullptr;
    auto writes_slice = [&](int kt) { return write_xp && kt % col_tiles == ct; };

    // The tile's MFMA work, for one wave layout: TM x TN 16x16 tiles per wave
    // starting at tile row wm0 and column wn0. Every layout accumulates each
    // output in the same k order (slices ascending, 16-wide k chunks, one
    // MFMA step per 4 k), so they give bit-identical results.
    auto run_tile = [&](auto layout) {
      using L = decltype(layout);
      constexpr int TM = L::kTM;
      constexpr int TN = L::kTN;
      const int wm0 = L::wm0(wave);
      const int wn0 = L::wn0(wave);
      v4f acc[TM][TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.0F, 0.0F, 0.0F, 0.0F};

      // One BK slice from the LDS stage of slice kt into the accumulators.
      auto multiply = [&](int kt) {
        const float* cur = stages + (kt % S::kStages) * kStageFloats;
        const float* As = cur;
        const float* Bs = cur + S::BM * S::kLd;
#pragma unroll
        for (int kk = 0; kk < S::BK; kk += 16) {
          v4f af[TM], bf[TN];
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            af[i] = *reinterpret_cast<const v4f*>(As + (wm0 + i * 16 + li) * S::kLd + kk + 4 * g);
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            bf[j] = *reinterpret_cast<const v4f*>(Bs + (wn0 + j * 16 + li) * S::kLd + kk + 4 * g);
          }
          mfma_steps<TM, TN>(acc, af, bf);
        }
      };
      if constexpr (DMA) {
        using D = DmaLayout;
        const int rows = row_end - row0 < S::BM ? row_end - row0 : S::BM;
        // This thread's chunk of each of the wave's four A and four B blocks
        // (block q = 4 p + wave: A rows 8q .. 8q + 7, B k rows 2q, 2q + 1).
        // A rows without a source read row 0 of the tile's source (their
        // products land in output rows that are never stored); B columns past
        // N read the last chunk of the row (likewise never stored).
        const float* asrc[4];
        const float* bsrc[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int q = 4 * p + wave;
          const int r = 8 * q + (lane >> 3);
          const int kc = (lane & 7) ^ D::swa(r);
          int src = -1;
          if constexpr (MODE == kChainGrouped) {
            src = s_src[r];
          } else {
            src = r < rows ? row0 + r : -1;
          }
          if (src < 0) src = MODE == kChainGrouped ? 0 : row0;
          asrc[p] = prm.X + static_cast<std::size_t>(src) * K + 4 * kc;
          const int kl = 2 * q + (lane >> 5);
          const int n = n0 + 4 * ((lane & 31) ^ D::swb(kl));
          bsrc[p] = B + static_cast<std::size_t>(kl) * N + (n < N ? n : N - 4);
        }
        const std::size_t b_slice = static_cast<std::size_t>(D::kBK) * N;
        // Any alignment (rows start at any 4-byte boundary; the 16-byte loads
        // take them): slices before the last hold only k < K, and B quads
        // that cross N read the next k row (in bounds) into columns that are
        // never stored. issue_last loads the last slice: a chunk wholly past
        // K from an in-bounds address (the A row's start, B's row 0), then
        // zeroed; an A chunk across K, and a B chunk across N in row K - 1
        // (which could end W), from the row's last whole quad, then shifted
        // into place with zeros after the row's end. fix holds 4 bits per
        // chunk (A chunk p at bit 4p, B chunk p at 16 + 4p): 0 = as loaded,
        // else v + 1 for v leading floats kept.
        uint32_t fix = 0;
        // The last slice: each chunk's address built and its load issued at
        // once (nothing of it stays live across the slices before).
        auto issue_last = [&](float* As) {
          float* Bs = As + D::kAFloats;
          const int k_last = (nk - 1) * D::kBK;
          // (the lane id passes an empty asm so that none of this is hoisted
          // out of the tile loop and kept live across it)
          int ln = lane;
          asm volatile("" : "+v"(ln));
          fix = 0;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int q = 4 * p + wave;
            const int r = 8 * q + (ln >> 3);
            const int kc = (ln & 7) ^ D::swa(r);
            const int k0 = k_last + 4 * kc;
            const float* row = asrc[p] - 4 * kc;  // the row's start
            int keep = 4;
            int at = k0;
            if (k0 >= K) {
              at = 0;
              keep = 0;
            } else if (k0 + 4 > K) {
              at = K - 4;
              keep = K - k0;
            }
            if (keep < 4) fix |= static_cast<uint32_t>(keep + 1) << (4 * p);
            __builtin_amdgcn_global_load_lds(row + at, As + q * D::kBlockFloats, 16, 0, 0);
          }
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int q = 4 * p + wave;
            const int kl = 2 * q + (ln >> 5);
            const int k = k_last + kl;
            const int n = n0 + 4 * ((ln & 31) ^ D::swb(kl));
            const float* brow = B + static_cast<std::size_t>(k < K ? k : 0) * N;
            int bkeep = 4;
            int at = n < N ? n : N - 4;
            if (k >= K) {
              bkeep = 0;
            } else if (k == K - 1 && n < N && n + 4 > N) {
              at = N - 4;
              bkeep = N - n;
            }
            if (bkeep < 4) fix |= static_cast<uint32_t>(bkeep + 1) << (16 + 4 * p);
            __builtin_amdgcn_global_load_lds(brow + at, Bs + q * D::kBlockFloats, 16, 0, 0);
          }
        };
        auto issue = [&](int kt, float* As) {
          float* Bs = As + D::kAFloats;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int q = 4 * p + wave;
            __builtin_amdgcn_global_load_lds(asrc[p] + kt * D::kBK, As + q * D::kBlockFloats, 16, 0, 0);
          }
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int q = 4 * p + wave;
            __builtin_amdgcn_global_load_lds(bsrc[p] + kt * b_slice, Bs + q * D::kBlockFloats, 16, 0, 0);
          }
        };
        // The last slice's chunk fix-ups, by the wave that loaded them, after
        // its loads have landed and before the barrier that publishes them.
        auto fixup = [&](float* As) {
          float* Bs = As + D::kAFloats;
          auto fix_chunk = [&](float* d, uint32_t code) {
            if (code == 0) return;
            const int keep = static_cast<int>(code) - 1;
            const v4f v = *reinterpret_cast<const v4f*>(d);
            v4f o;
            o[0] = keep == 3 ? v[1] : keep == 2 ? v[2] : keep == 1 ? v[3] : 0.0F;
            o[1] = keep == 3 ? v[2] : keep == 2 ? v[3] : 0.0F;
            o[2] = keep == 3 ? v[3] : 0.0F;
            o[3] = 0.0F;
            *reinterpret_cast<v4f*>(d) = o;
          };
          int ln = lane;
          asm volatile("" : "+v"(ln));
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int q = 4 * p + wave;
            fix_chunk(As + q * D::kBlockFloats + 4 * ln, (fix >> (4 * p)) & 15u);
            fix_chunk(Bs + q * D::kBlockFloats + 4 * ln, (fix >> (16 + 4 * p)) & 15u);
          }
        };
        // Operand addresses inside a stage. A: row r = wm0 + 16 i + li, k
        // chunk kk / 4 + g at slot (kk / 4 + g) ^ swa(r). B: row k = kk + 4g + s,
        // column n = wn0 + 16 j + li at (kk + s) * 128 + boff[j] (swb(k) = 4g).
        int aoff[TM][2];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int r = wm0 + 16 * i + li;
#pragma unroll
          for (int h = 0; h < 2; ++h) aoff[i][h] = r * D::kBK + 4 * ((4 * h + g) ^ D::swa(r));
        }
        int boff[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = wn0 + 16 * j + li;
          boff[j] = 4 * g * D::kColsB + 4 * ((n >> 2) ^ (4 * g)) + (n & 3);
        }
        // One slice: the first half's operands are read, the next slice's
        // loads issued, then the MFMAs run with the second half's reads among
        // them. (The reads come first so that the loads of the next slice,
        // which write the other stage, are never ordered before them.)
        // (restrict: the stage read and the stage loaded are disjoint, which
        // lets the compiler leave the reads after the loads unwaited)
        auto multiply_dma = [&](const float* __restrict__ As, float* __restrict__ next, auto iss) {
          const float* Bs = As + D::kAFloats;
          v4f af[2][TM];
          v4f bf[2][TN];
          auto read = [&](int h) {
#pragma unroll
            for (int i = 0; i < TM; ++i) af[h][i] = *reinterpret_cast<const v4f*>(As + aoff[i][h]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
              for (int s = 0; s < 4; ++s) bf[h][j][s] = Bs[(16 * h + s) * D::kColsB + boff[j]];
            }
          };
          read(0);
          iss(next);
          read(1);
#pragma unroll
          for (int h = 0; h < 2; ++h) mfma_steps<TM, TN>(acc, af[h], bf[h]);
          // Issue order: the first half's reads, then the next slice's loads
          // and the second half's reads spread over the first half's MFMAs.
          __builtin_amdgcn_sched_group_barrier(0x100, TM + 2 * TN, 0);  // LDS reads
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load into LDS
          }
#pragma unroll
          for (int r = 0; r < TM + 2 * TN; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);  // three MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
          }
        };
        // chain: the gathered rows of slice kt, read back from LDS, go to x_permuted
        auto store_xp = [&](int kt, const float* As) {
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int f = tid + p * S::kThreads;  // chunk f: row f / 8, slot f % 8
            const int r = f >> 3;
            if (r < rows) {
              const int kc = (f & 7) ^ D::swa(r);
              const v4f v = *reinterpret_cast<const v4f*>(As + 4 * f);
              __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(prm.x_permuted + static_cast<std::size_t>(row0 + r) * K +
                                                                   kt * D::kBK + 4 * kc));
            }
          }
        };
        // Slice kt + 1 streams into the other stage while slice kt is
        // multiplied; the barrier after each slice (which waits for the wave's
        // own LDS loads first) makes it visible and frees the stage just read.
        auto slice = [&](int kt, float* cur, float* next, auto iss, bool fix_next) {
          // Wave priority alternates by slice parity. Two workgroups share each
          // CU and the matrix pipe favours the older one's waves: on a tie the
          // first workgroup ran its tiles 1.4x faster than the second, which then
          // finished alone. (C4 grouped GEMM 14.27 -> 14.02 ms.)
          if (kt & 1) {
            __builtin_amdgcn_s_setprio(0);
          } else {
            __builtin_amdgcn_s_setprio(1);
          }
          if (writes_slice(kt)) store_xp(kt, cur);
          multiply_dma(cur, next, iss);
          // (the MFMAs stay ahead of the wait: moved past it, they would idle
          // behind the loads of the next slice)
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of slice kt + 1
          if (fix_next) fixup(next);
          __syncthreads();
        };
        auto stage_of = [&](int kt) { return stages + (kt & 1) * kStageFloats; };
        if constexpr (DMA == kDirect) {
          if (nk > 0) issue(0, stages);
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
          __syncthreads();
          for (int kt = 0; kt < nk; ++kt) {
            // (the last slice loads itself again into the unused stage: no
            // branch in the slice, whose waits then stay per operand)
            slice(kt, stage_of(kt), stage_of(kt + 1),
                  [&](float* nx) { issue(kt + 1 < nk ? kt + 1 : kt, nx); }, false);
          }
        } else if (nk > 0) {
          // Slices before the last two issue the next slice; slice nk - 2
          // issues the last one from the clamped addresses (fixed up once
          // landed); the last slice issues nothing. (The last slice's
          // addresses are built only in that branch, so that they are not
          // live across the loop.)
          if (nk == 1) {
            issue_last(stages);
          } else {
            issue(0, stages);
          }
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
          if (nk == 1) fixup(stages);
          __syncthreads();
          for (int kt = 0; kt < nk; ++kt) {
            slice(kt, stage_of(kt), stage_of(kt + 1),
                  [&](float* nx) {
                    if (kt + 2 < nk) {
                      issue(kt + 1, nx);
                    } else if (kt + 2 == nk) {
                      issue_last(nx);
                    }
                  },
                  kt + 2 == nk);
          }
        }
      } else {
        Stage<S, VEC> st;
        st.set_rows(prm.X, src_rows, row0, row_end, K, write_xp ? prm.x_permuted : nullptr, tid);
        if constexpr (S::kStages > 1) {
          // Two LDS stages fed from two register stages: slice kt + 2 is loaded
          // while slice kt is multiplied, so each slice has two slices' compute
          // time to arrive (the B slices of experts with few row tiles come from
          // HBM rather than L2). The register stages swap roles every slice, so
          // the loop runs two slices per trip (static roles, no copies).
          Stage<S, VEC> st2 = st;
          if (nk > 0) {
            st.load(B, n0, N, K, 0, tid);
            st.store(stages, tid);
            if (writes_slice(0)) st.store_a_rows(K, 0, tid);
            if (nk > 1) st2.load(B, n0, N, K, S::BK, tid);
          }
          __syncthreads();
          // held: slice kt (stored to LDS); next: slice kt + 1 (in flight)
          auto step = [&](int kt, Stage<S, VEC>& held, Stage<S, VEC>& next) {
            if (kt + 2 < nk) held.load(B, n0, N, K, (kt + 2) * S::BK, tid);
            multiply(kt);
            if (kt + 1 < nk) {
              next.store(stages + ((kt + 1) % S::kStages) * S::kStageFloats, tid);
              if (writes_slice(kt + 1)) next.store_a_rows(K, (kt + 1) * S::BK, tid);
            }
            __syncthreads();
          };
          for (int kt = 0; kt < nk; kt += 2) {
            step(kt, st, st2);
            if (kt + 1 < nk) step(kt + 1, st2, st);
          }
        } else {
          if (nk > 0) {
            st.load(B, n0, N, K, 0, tid);
            st.store(stages, tid);
            if (writes_slice(0)) st.store_a_rows(K, 0, tid);
          }
          __syncthreads();
          for (int kt = 0; kt < nk; ++kt) {
            multiply(kt);
            if (kt + 1 < nk) {
              __syncthreads();  // every wave is done with the single stage
              st.load(B, n0, N, K, (kt + 1) * S::BK, tid);
              st.store(stages, tid);
              if (writes_slice(kt + 1)) st.store_a_rows(K, (kt + 1) * S::BK, tid);
            }
            __syncthreads();
          }
        }
      }

      // Epilogue: acc[i][j][r] is D[4g + r][li] of the 16x16 tile (i, j).
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rl = wm0 + i * 16 + 4 * g + r;
          const int row = row0 + rl;
          if (row >= row_end) continue;
          float* yrow = prm.Y + static_cast<std::size_t>(row) * N;
          float* comb = nullptr;
          float w = 0.0F;
          if constexpr (MODE == kChainGrouped) {
            if (prm.y_out != nullptr) comb = prm.y_out + static_cast<std::size_t>(s_src[rl]) * N;
            w = s_w[rl];
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn0 + j * 16 + li;
            if (col < N) {
              if (comb != nullptr) {
                // combined: y_permuted is not read again by the chain
                __builtin_nontemporal_store(acc[i][j][r], yrow + col);
              } else {
                yrow[col] = acc[i][j][r];
              }
              if constexpr (MODE == kChainGrouped) {
                // Both routes of a token add into the zeroed output: fl(0 + a) + b
                // is the same in either order, so the combine is deterministic
                // and equals the rank-order unpermute.
                if (comb != nullptr) unsafeAtomicAdd(comb + col, __fmul_rn(w, acc[i][j][r]));
              }
            }
          }
        }
      }
    };
    // Tile rows past the expert's end are padding: a tile with at most 64,
    // 32 or 16 rows gives each of the four waves a 32-column slab of that
    // height instead of the 2 x 2 layout of 64 x 64, so the padding costs no
    // MFMA work beyond the 16-row granule and every SIMD stays busy.
    if constexpr (kSlabs) {
      const int rows = row_end - row0;
      if (rows > 64) {
        run_tile(WaveLayout<S::kTM, S::kTN, S>{});
      } else if (rows > 32) {
        run_tile(SlabLayout<4, 2, 32>{});
      } else if (rows > 16) {
        run_tile(SlabLayout<2, 2, 32>{});
      } else {
        run_tile(SlabLayout<1, 2, 32>{});
      }
    } else {
      run_tile(WaveLayout<S::kTM, S::kTN, S>{});
    }
  }
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices] = {};

int device_cu_count() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 256;
  if (device >= 0 && device < kMaxDevices) {
    const int cached = g_cu_count[device].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0) {
    cus = 256;
  }
  if (device >= 0 && device < kMaxDevices) g_cu_count[device].store(cus, std::memory_order_relaxed);
  return cus;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// Allows a kernel instantiation to use the whole 160 KB of gfx950 LDS as
// dynamic shared memory (once per instantiation).
template <class Kernel>
hipError_t allow_full_lds(Kernel kernel) {
  static const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return status;
}

template <class S, bool VEC, int MODE, int DMA>
hipError_t launch_one(dim3 grid, std::size_t lds, const GemmParams& prm, hipStream_t stream) {
  const hipError_t attr = allow_full_lds(rr_gemm_mfma_kernel<S, VEC, MODE, DMA>);
  if (attr != hipSuccess) return attr;
  rr_gemm_mfma_kernel<S, VEC, MODE, DMA><<<grid, S::kThreads, lds, stream>>>(prm);
  return hipGetLastError();
}

// Staging override for tests and A/B runs: RR_GEMM_STAGING=registers keeps the
// register-staged path where the direct LDS loads would otherwise run. Read at
// every launch (one getenv).
bool registers_forced() {
  const char* v = std::getenv("RR_GEMM_STAGING");
  return v != nullptr && std::strcmp(v, "registers") == 0;
}

// RR_GEMM_STAGING=aligned keeps the direct loads to aligned shapes (the
// register path then takes the others), for A/B runs.
bool direct_any_disabled() {
  const char* v = std::getenv("RR_GEMM_STAGING");
  return v != nullptr && std::strcmp(v, "aligned") == 0;
}

template <class S, int MODE>
hipError_t launch_gemm(const GemmParams& prm, long tile_bound, hipStream_t stream) {
  const bool vec = (prm.K % 4 == 0) && (prm.N % 4 == 0) && aligned16(prm.X) && aligned16(prm.W) &&
                   (MODE != kChainGrouped || aligned16(prm.x_permuted));
  const long cap = static_cast<long>(device_cu_count()) * 2;
  long grid = tile_bound < cap ? tile_bound : cap;
  if (grid >= kXcds) grid = grid / kXcds * kXcds;
  if (grid < 1) grid = 1;
  const std::size_t meta = 3 * static_cast<std::size_t>(prm.experts + 1) * sizeof(int32_t) +
                           2 * static_cast<std::size_t>(S::BM) * sizeof(int32_t);
  const dim3 g(static_cast<unsigned>(grid));
  if constexpr (S::BM == 128 && S::BN == 128 && S::WM == 2 && S::WN == 2 && S::BK == DmaLayout::kBK) {
    const std::size_t lds = S::kStages * DmaLayout::kStageFloats * sizeof(float) + meta;
    if (!registers_forced()) {
      // whole 32-deep slices and 16-byte rows: direct LDS loads
      if (vec && prm.K % DmaLayout::kBK == 0) return launch_one<S, true, MODE, kDirect>(g, lds, prm, stream);
      // other K, N or 4-byte row alignment (dense and grouped): direct loads
      // with the last slice fixed up
      if constexpr (MODE != kChainGrouped) {
        if (prm.K >= DmaLayout::kBK && prm.N >= 4 && !direct_any_disabled()) {
          return launch_one<S, false, MODE, kDirectAnyAlign>(g, lds, prm, stream);
        }
      }
    }
  }
  const std::size_t lds = S::kStages * S::kStageFloats * sizeof(float) + meta;
  return vec ? launch_one<S, true, MODE, kRegisters>(g, lds, prm, stream)
             : launch_one<S, false, MODE, kRegisters>(g, lds, prm, stream);
}

// 128x128, four 64x64 waves, BK 32: large problems (C4, C5 grouped). (BK 16,
// one barrier per 64 MFMAs of a wave instead of 128, measured 1-2 % slower:
// C4 grouped GEMM 15.23 against 15.02 ms, C5 expert launch 1116 against 1091 us.)
using TileLarge = TileShape<128, 128, 2, 2, 32>;
// 64x64, four 32x32 waves, BK 64: medium problems with short K loops.
using TileSmall = TileShape<64, 64, 2, 2, 64>;
// 32x64, four 16x32 waves, BK 64: small ragged segments (tens of rows per expert).
using TileMedium = TileShape<32, 64, 2, 2, 64>;
// 16x64, four 16x16 waves side by side, BK 64: narrow router GEMMs (N = E <= 64).
using TileNarrow = TileShape<16, 64, 1, 4, 64>;

// Whole-K tiles (K <= 256): one LDS stage holds all of K.
using TileSmallK256 = TileShape<64, 64, 2, 2, 256>;    // 133 KB LDS
using TileMediumK256 = TileShape<32, 64, 2, 2, 256>;   // 100 KB LDS
using TileNarrowK256 = TileShape<16, 64, 1, 4, 256>;   // 83 KB LDS

// Tile override for tuning sweeps and tests: RR_GEMM_TILE = large | small |
// medium | narrow | small256 | medium256 | narrow256 forces one of the
// (equally correct) tile configurations of the dense and grouped GEMMs, also
// where the narrow-output strip kernels (strip.hip) would otherwise run. Read
// at every launch (one getenv), so a process can switch configurations.
int tile_override() {
  const char* v = std::getenv("RR_GEMM_TILE");
  if (v == nullptr) return 0;
  if (std::strcmp(v, "large") == 0) return 1;
  if (std::strcmp(v, "small") == 0) return 2;
  if (std::strcmp(v, "medium") == 0) return 3;
  if (std::strcmp(v, "narrow") == 0) return 4;
  if (std::strcmp(v, "small256") == 0) return 5;
  if (std::strcmp(v, "medium256") == 0) return 6;
  if (std::strcmp(v, "narrow256") == 0) return 7;
  return 0;
}

long ceil_div(long a, long b) { return (a + b - 1) / b; }

// Upper bound on the tile count given a per-expert row bound.
long tile_bound(int experts, long rows_per_expert, int bm, int n, int bn) {
  return static_cast<long>(experts) * ceil_div(rows_per_expert, bm) * ceil_div(n, bn);
}

// Expected tile count: full tiles of the rows plus one partial tile per segment.
long tile_estimate(long rows, int segments, int bm, int n, int bn) {
  return (ceil_div(rows, bm) + segments) * ceil_div(n, bn);
}

template <class S, int MODE>
hipError_t launch_tile(const GemmParams& prm, long rows_per_expert, hipStream_t stream) {
  const int segments = MODE == kDense ? 1 : prm.experts;
  return launch_gemm<S, MODE>(prm, tile_bound(segments, rows_per_expert, S::BM, prm.N, S::BN),
                              stream);
}

template <int MODE>
hipError_t gemm_dispatch(const GemmParams& prm, long rows_per_expert, long total_rows_estimate,
                         hipStream_t stream) {
  const long cus = device_cu_count();
  const int segments = MODE == kDense ? 0 : prm.experts;
  const int n = prm.N;
  switch (tile_override()) {
    case 1: return launch_tile<TileLarge, MODE>(prm, rows_per_expert, stream);
    case 2: return launch_tile<TileSmall, MODE>(prm, rows_per_expert, stream);
    case 3: return launch_tile<TileMedium, MODE>(prm, rows_per_expert, stream);
    case 4: return launch_tile<TileNarrow, MODE>(prm, rows_per_expert, stream);
    case 5: return launch_tile<TileSmallK256, MODE>(prm, rows_per_expert, stream);
    case 6: return launch_tile<TileMediumK256, MODE>(prm, rows_per_expert, stream);
    case 7: return launch_tile<TileNarrowK256, MODE>(prm, rows_per_expert, stream);
    default: break;
  }
  // Largest tile that still gives every CU work (two tiles per CU for the
  // large tile, whose LDS and registers allow two resident workgroups).
  if (tile_estimate(total_rows_estimate, segments, TileLarge::BM, n, TileLarge::BN) >= 2 * cus) {
    return launch_tile<TileLarge, MODE>(prm, rows_per_expert, stream);
  }
  if (tile_estimate(total_rows_estimate, segments, TileSmall::BM, n, TileSmall::BN) >= cus) {
    return launch_tile<TileSmall, MODE>(prm, rows_per_expert, stream);
  }
  return launch_tile<TileNarrow, MODE>(prm, rows_per_expert, stream);
}

GemmParams base_params(const float* x, const float* w, const int32_t* offsets, float* y,
                       int experts, int dense_rows, int K, int N) {
  GemmParams p{};
  p.X = x;
  p.W = w;
  p.offsets = offsets;
  p.Y = y;
  p.experts = experts;
  p.dense_rows = dense_rows;
  p.K = K;
  p.N = N;
  return p;
}

}  // namespace

hipError_t dense_gemm_mfma(const float* a, const float* b, float* c, int m, int n, int k,
                           hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  if (tile_override() == 0 && strip_shape_ok(k, n, a, b)) return strip_dense(a, b, c, m, n, k, stream);
  return gemm_dispatch<kDense>(base_params(a, b, nullptr, c, 1, m, k, n), m, m, stream);
}

hipError_t grouped_gemm_mfma(const float* x, const float* w, const int32_t* offsets, float* y,
                             int experts, int hidden, int output, int max_expert_tokens,
                             hipStream_t stream) {
  if (max_expert_tokens <= 0 || output <= 0) return hipSuccess;
  // The host never reads offsets; the caller's bound sizes the grid and the
  // device scheduler covers every row of every segment.
  if (tile_override() == 0 && strip_shape_ok(hidden, output, x, w) && strip_segments_ok(experts)) {
    return strip_grouped(x, w, offsets, y, experts, hidden, output,
                         static_cast<long>(experts) * max_expert_tokens, stream);
  }
  return gemm_dispatch<kGrouped>(
      base_params(x, w, offsets, y, experts, 0, hidden, output), max_expert_tokens,
      max_expert_tokens, stream);
}

hipError_t router_gate_mfma(const float* x, const float* router_weights, float* logits,
                            int32_t* ids, float* gate_weights, float* y_zero, int y_cols,
                            int tokens, int experts, int hidden, hipStream_t stream) {
  if (tokens <= 0) return hipSuccess;
  // The strip kernel carries the gate epilogue (E <= 128, K <= 256); callers
  // run the dense GEMM and the gate kernel for other shapes.
  if (experts > 128 || !strip_shape_ok(hidden, experts, x, router_weights)) return hipErrorInvalidValue;
  return strip_router_gate(x, router_weights, logits, ids, gate_weights, y_zero, y_cols, tokens,
                           experts, hidden, stream);
}

hipError_t chain_grouped_mfma(const float* x, const float* expert_weights, const int32_t* offsets,
                              const int32_t* sorted_route, const float* route_weights,
                              float* x_permuted, float* y_permuted, float* y, int tokens,
                              int top_k, int experts, int hidden, int output, hipStream_t stream) {
  if (tokens <= 0 || output <= 0) return hipSuccess;
  if (y != nullptr && top_k != 2) return hipErrorInvalidValue;  // combine is top-2 only
  GemmParams p = base_params(x, expert_weights, offsets, y_permuted, experts, 0, hidden, output);
  p.sorted_route = sorted_route;
  p.route_weights = route_weights;
  p.x_permuted = x_permuted;
  p.y_out = y;
  p.top_k = top_k;
  const long routes = static_cast<long>(tokens) * top_k;
  return gemm_dispatch<kChainGrouped>(p, routes, routes, stream);
}

}  // namespace rr::kern
