// Plan internals shared by the plan builders (plan.hip, plan_bucket.hip, plan_radix.hip): the
// workspace layout, the bucketed and radix plans' geometry, block reductions and the expert-table
// sources.
#pragma once

#include <algorithm>

#include "common.h"

namespace fmoe {

constexpr int kScanThreads = 1024;

// ---- bucketed plan geometry -------------------------------------------------------------------
// The T + 1 token bins (bin T: out-of-range rows) are grouped into buckets of 2^shift consecutive
// bins; the rows are partitioned by bucket in slices of S rows (k_plan_part), then each bucket is
// ordered by one wave (k_plan_bucket).
constexpr int kPartThreads = 1024;
constexpr int kPartWaves = kPartThreads / kWave;  // 16
constexpr int kMaxBuckets = 1024;                 // bucket ids fit 10 bits
constexpr int kMaxBucketBins = 4096;              // bins per bucket (one wave's LDS counters)
constexpr int kMaxSlices = 512;                   // partition slices
constexpr int64_t kBucketRows = 128;              // rows per bucket aimed at
constexpr int64_t kMinSlice = 2048;               // rows per slice at least (multiple of 1024)

struct PlanGeom {
  int64_t S;   // rows per slice, a multiple of kPartThreads
  int G1;      // slices (>= 1)
  int shift;   // log2(bins per bucket)
  int nbk;     // buckets
  bool ok;     // within the bucketed plan's limits (else the radix plan)
};

__host__ __device__ inline PlanGeom plan_geom(int64_t N, int64_t T) {
  PlanGeom g;
  const int64_t nb = T + 1;
  // bins per bucket: the power of two at or below the count that holds about kBucketRows rows
  // (at most kMaxBucketBins), raised until the buckets number at most kMaxBuckets
  const int64_t target = N > 0 ? nb * kBucketRows / N : nb;
  int shift = 0;
  while ((int64_t(2) << shift) <= target && (int64_t(2) << shift) <= kMaxBucketBins) ++shift;
  while (((nb + (int64_t(1) << shift) - 1) >> shift) > kMaxBuckets) ++shift;
  g.shift = shift;
  g.nbk = (int)((nb + (int64_t(1) << shift) - 1) >> shift);
  g.ok = (int64_t(1) << shift) <= kMaxBucketBins;
  const int64_t per_slice = (N + kMaxSlices - 1) / kMaxSlices;
  const int64_t S = (per_slice + kPartThreads - 1) / kPartThreads * kPartThreads;
  g.S = S > kMinSlice ? S : kMinSlice;
  g.G1 = (int)(N > 0 ? (N + g.S - 1) / g.S : 1);
  return g;
}

// ---- ranged plan geometry ---------------------------------------------------------------------
// Two launches for larger N: the rows are partitioned by token range in slices of kRangeSlice rows
// (k_plan_split, one row per thread, stable within each range), then one 1024-thread workgroup per
// range of at most kRangeMaxBins consecutive bins gathers the range's rows, slice after slice, and
// orders them like the one-launch plan (k_plan_range).  There are about kRangeGroups ranges (one
// per CU), more when the bins or the rows would not fit (a range's workgroup stashes up to
// kRangeRows rows without re-reading them), at most kRangeMaxGroups.  A row's range is bin / bins,
// computed as (bin * magic) >> 32 with magic = ceil(2^32 / bins): exact for bin < 2^32 / bins,
// which T + 1 <= kRangeMaxBinsTotal guarantees.
constexpr int kRangeSlice = 1024;                 // rows per slice (one per thread)
constexpr int kRangeMaxSlices = 4096;             // slices: N <= 2^22
constexpr int kRangeSlicesPerThread = 4;          // k_plan_range reads 4 slices' words per thread
constexpr int kRangeGroups = 256;                 // ranges aimed at (about one per CU)
constexpr int kRangeMaxGroups = 1024;             // ranges at most (k_plan_split's LDS counters)
constexpr int kRangeMaxBins = 512;                // bins per range (the per-wave LDS counters)
constexpr int kRangeRows = 4096;                  // rows a range's stashes hold (16 waves x 256)
constexpr int64_t kRangeMaxBinsTotal = int64_t(kRangeMaxGroups) * kRangeMaxBins;

struct RangeGeom {
  int Q;           // ranges (>= 1), each non-empty
  int bins;        // bins per range
  uint64_t magic;  // ceil(2^32 / bins)
  int G1;          // slices (>= 1)
  bool ok;         // within the ranged plan's limits
};

__host__ __device__ inline RangeGeom range_geom(int64_t N, int64_t T) {
  RangeGeom r;
  const int64_t nb = T + 1;
  int64_t q = nb < kRangeGroups ? nb : kRangeGroups;
  const int64_t by_bins = (nb + kRangeMaxBins - 1) / kRangeMaxBins;
  const int64_t by_rows = (N + kRangeRows - 1) / kRangeRows;
  q = q > by_bins ? q : by_bins;
  q = q > by_rows ? q : by_rows;
  q = q < nb ? q : nb;
  const int64_t bins = (nb + q - 1) / q;
  q = (nb + bins - 1) / bins;
  r.Q = (int)(q < kRangeMaxGroups ? q : kRangeMaxGroups);
  r.bins = (int)bins;
  r.magic = ((uint64_t(1) << 32) + (uint64_t)bins - 1) / (uint64_t)bins;
  const int64_t g1 = (N + kRangeSlice - 1) / kRangeSlice;
  r.G1 = (int)(g1 > 1 ? (g1 < kRangeMaxSlices ? g1 : kRangeMaxSlices) : 1);
  r.ok = nb <= kRangeMaxBinsTotal && bins <= kRangeMaxBins && q <= kRangeMaxGroups &&
         g1 <= kRangeMaxSlices;
  return r;
}

// ---- radix plan geometry ----------------------------------------------------------------------
// Beyond the bucketed plan's limits: a stable least-significant-digit radix sort of the rows by
// token bin (plan_radix.hip), 8-bit digits, in tiles of whole 1024-row chunks -- about
// kRadixTargetTiles tiles (several workgroups per CU), at most kRadixMaxTiles (so each pass's
// per-tile digit table stays small).
constexpr int kRadixThreads = 1024;
constexpr int kRadixDigits = 256;
constexpr int kRadixMaxPasses = 4;       // bins T + 1 <= 2^30 need at most 30 bits
constexpr int64_t kRadixMaxTiles = 4096;
constexpr int64_t kRadixTargetTiles = 2048;

struct RadixGeom {
  int passes;    // ceil(bits of T / 8): the largest bin is T (out-of-range rows)
  int ntiles;    // >= 1
  int64_t tile;  // rows per tile, a multiple of kRadixThreads
};

__host__ __device__ inline RadixGeom radix_geom(int64_t N, int64_t T) {
  RadixGeom r;
  int bits = 1;
  while (bits < 62 && (T >> bits) != 0) ++bits;
  r.passes = (bits + 7) / 8;
  const int64_t per = kRadixThreads * kRadixTargetTiles;
  const int64_t chunks = std::max<int64_t>(1, (N + per - 1) / per);
  r.tile = chunks * kRadixThreads;
  r.ntiles = (int)std::max<int64_t>(1, (N + r.tile - 1) / r.tile);
  return r;
}

// ---- plan workspace layout --------------------------------------------------------------------
//   status   int32[3] (+ padding)
//   cursor   int32[T + 1]      the radix plan's per-block maxima of its row_ptr scan
//   row_ptr  int32[T + 2]
//   tmp      the radix plan's two (bin, g) pair buffers (2 x N x int2), or the bucketed plan's
//            partition (N x int2) followed by its per-slice bucket counts and prefixes
//            (2 x G1 x nbk int32)
//   rec      N x 16-byte records
//   radix    the radix plan's digit totals (kRadixMaxPasses x 256 int32) and per-tile digit
//            table (256 x ntiles int32)
struct PlanLayout {
  int64_t status, cursor, row_ptr, rec_tmp, part, bcnt, bpre, rcnt, rpre, rec, radix_tot, radix_hist,
      total;
};

__host__ __device__ inline PlanLayout plan_layout(int64_t N, int64_t T) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const PlanGeom g = plan_geom(N, T);
  const int64_t tab = (int64_t)g.G1 * g.nbk * 4;
  PlanLayout L;
  L.status = 0;
  L.cursor = 256;
  L.row_ptr = L.cursor + up((T + 1) * 4);
  L.rec_tmp = L.row_ptr + up((T + 2) * 4);
  L.part = L.rec_tmp;
  L.bcnt = L.part + up(N * 8);
  L.bpre = L.bcnt + up(tab);
  // the ranged plan's per-range, per-slice row counts and prefixes follow its partition
  const RangeGeom rg = range_geom(N, T);
  const int64_t rtab = (int64_t)rg.Q * rg.G1 * 4;
  L.rcnt = L.part + up(N * 8);
  L.rpre = L.rcnt + up(rtab);
  const int64_t tmp_end =
      std::max(std::max(L.rec_tmp + up(N * 16), L.bpre + up(tab)), L.rpre + up(rtab));
  L.rec = tmp_end;
  L.radix_tot = L.rec + up(N * 16);
  L.radix_hist = L.radix_tot + up(kRadixMaxPasses * kRadixDigits * 4);
  L.total = L.radix_hist + up((int64_t)kRadixDigits * radix_geom(N, T).ntiles * 4);
  return L;
}

// ---- wave scans -------------------------------------------------------------------------------
// Inclusive prefix sum over the 64 lanes of a wave with gfx9 DPP: row_shr 1, 2, 4, 8 scan each row
// of 16 lanes (a lane with no source lane adds 0), row_bcast:15 adds row 0's total to row 1 and
// row 2's to row 3, row_bcast:31 adds the first 32 lanes' total to rows 2 and 3.  Six register
// moves instead of six LDS permutes.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
  return x;
}

// ---- 1024-thread block reductions -------------------------------------------------------------
// Exclusive scan of one int per thread over a 1024-thread block; *total gets the block sum.
__device__ __forceinline__ int block_exclusive_scan_1024(int v, int* total) {
  __shared__ int wave_tot[kScanThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int incl = wave_incl_sum(v);
  if (lane == kWave - 1) wave_tot[wv] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kScanThreads / kWave; ++i) {
    const int x = wave_tot[i];
    before += (i < wv) ? x : 0;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return before + incl - v;
}

// Max of one int per thread over a 1024-thread block (all threads get it).
__device__ __forceinline__ int block_max_1024(int v) {
  __shared__ int wave_max[kScanThreads / kWave];
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v = max(v, __shfl_xor(v, d, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) wave_max[threadIdx.x / kWave] = v;
  __syncthreads();
  int m = 0;
#pragma unroll
  for (int i = 0; i < kScanThreads / kWave; ++i) m = max(m, wave_max[i]);
  __syncthreads();
  return m;
}

// ---- where a plan builder gets the expert table from --------------------------------------------
// TokMetaGlobal: the device arrays of fmoe_build_metadata.  TokMetaArgs: the table in the kernel
// arguments (at most 256 experts), prefixed on the host -- each expert's address and first packed
// row, and the largest row count -- so a workgroup only copies it into LDS; workgroup 0 also
// writes the metadata outputs, so metadata and plan need no separate launch.
struct TokMetaGlobal {
  const int64_t* ptr_table;
  const int64_t* offsets;
};
struct HostTable {
  int64_t ptr[kMetaChunk];
  int32_t off[kMetaChunk + 1];  // exclusive prefix of the row counts; off[count] = N < 2^31
  int32_t count;
  int32_t max_rows;
};
struct TokMetaArgs {
  HostTable a;
  int64_t* ptr_table;
  int32_t* chunk_sizes;
  int64_t* offsets;
  int32_t* max_rows;
};
static_assert(sizeof(TokMetaArgs) <= 3200, "kernel-argument table too large");

// The host side of TokMetaArgs: E <= kMetaChunk (address, rows) pairs, rows in [0, 2^31) and
// summing below 2^31 (checked by the callers).
inline void fill_host_table(TokMetaArgs* m, const int64_t* host_ptrs, const int64_t* host_rows,
                            int64_t E, int64_t* ptr_table, int32_t* chunk_sizes, int64_t* offsets,
                            int32_t* max_rows) {
  int64_t run = 0, mx = 0;
  for (int i = 0; i < kMetaChunk; ++i) {
    const int64_t n = i < E ? host_rows[i] : 0;
    m->a.ptr[i] = i < E ? host_ptrs[i] : 0;
    m->a.off[i] = (int32_t)run;
    run += n;
    mx = std::max(mx, n);
  }
  m->a.off[kMetaChunk] = (int32_t)run;
  m->a.count = (int32_t)E;
  m->a.max_rows = (int32_t)mx;
  m->ptr_table = ptr_table;
  m->chunk_sizes = chunk_sizes;
  m->offsets = offsets;
  m->max_rows = max_rows;
}

// ---- small inputs without a plan (fmoe_combine_fwd_small / fmoe_combine_bwd_small) ------------
// Rows of the small path: every forward workgroup stages their token ids in LDS.
constexpr int kSmallRows = 4096;

// Host side of the small path: checks the (address, rows) pairs as fmoe_build_metadata does, fills
// the argument table, returns the row count and whether every row is 16-byte aligned (the plan's
// misaligned-flag rule: a nonempty expert's address, and row_bytes when it has several rows).
inline int small_host_table(const char* who, const int64_t* host_ptrs, const int64_t* host_rows,
                            int64_t E, int64_t row_bytes, HostTable* t, int64_t* n_rows,
                            bool* aligned) {
  FMOE_REQUIRE(host_ptrs && host_rows, "%s: null host table", who);
  FMOE_REQUIRE(E >= 1 && E <= kMetaChunk, "%s: num_experts must be in [1, %d] (got %lld)", who,
               kMetaChunk, (long long)E);
  int64_t run = 0, mx = 0;
  bool al = true;
  for (int64_t e = 0; e < kMetaChunk; ++e) {
    const int64_t n = e < E ? host_rows[e] : 0;
    FMOE_REQUIRE(n >= 0, "%s: expert %lld has invalid row count %lld", who, (long long)e,
                 (long long)n);
    FMOE_REQUIRE(n == 0 || host_ptrs[e] != 0, "%s: expert %lld has rows but a null address", who,
                 (long long)e);
    if (n > kSmallRows - run) {
      fmoe_host::set_error("%s: more than %d rows (the small path's limit)", who, kSmallRows);
      return FMOE_ERANGE;
    }
    t->ptr[e] = e < E ? host_ptrs[e] : 0;
    t->off[e] = (int32_t)run;
    if (n > 0 && ((host_ptrs[e] & 15) || (n > 1 && (row_bytes & 15)))) al = false;
    run += n;
    mx = std::max(mx, n);
  }
  t->off[kMetaChunk] = (int32_t)run;
  t->count = (int32_t)E;
  t->max_rows = (int32_t)mx;
  *n_rows = run;
  *aligned = al;
  return FMOE_OK;
}

// The argument table into LDS, one expert per thread (E <= kMetaChunk == the workgroup size).
__device__ __forceinline__ void small_table_to_lds(const HostTable& t, int* off_lds,
                                                   uint64_t* ptr_lds) {
  const int e = threadIdx.x;
  if (e < t.count) {
    off_lds[e] = t.off[e];
    ptr_lds[e] = (uint64_t)t.ptr[e];
  }
  if (e == 0) off_lds[t.count] = t.off[t.count];
}

// For the first kn of K keys (kn wave-uniform), the largest a in [0, n) with arr[a] <= key[k]
// (arr non-decreasing over [0, n), n >= 1, arr[0] <= every key; out[k] = 0 for k >= kn): binary
// lifting, whose trip count depends on n alone, so the searches run side by side and their
// dependent LDS reads overlap (a loop per key would wait for each read in turn).  Only
// arr[0 .. n) is read.
template <int K>
__device__ __forceinline__ void last_le(const int* __restrict__ arr, int n, const int (&key)[K],
                                        int (&out)[K], int kn = K) {
#pragma unroll
  for (int k = 0; k < K; ++k) out[k] = 0;
  if (n <= 1) return;
  for (int step = 1 << (31 - __builtin_clz((unsigned)(n - 1))); step > 0; step >>= 1) {
    int val[K];
#pragma unroll
    for (int k = 0; k < K; ++k)  // all the reads first
      if (k < kn) val[k] = arr[min(out[k] + step, n - 1)];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (k < kn) {
        const int c = out[k] + step;
        out[k] = c < n && val[k] <= key[k] ? c : out[k];
      }
    }
  }
}

// Largest e in [0, E) with off[e] <= g (int32 offsets, off[0] == 0 <= g < off[E]).
__device__ __forceinline__ int expert_of_row32(const int* __restrict__ off, int E, int g) {
  int lo = 0, hi = E;  // invariant: off[lo] <= g < off[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (off[mid] <= g) lo = mid; else hi = mid;
  }
  return lo;
}

// Lanes below this one in a 64-bit lane mask.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// Mask of the active lanes whose `bits`-bit key equals this lane's (bits wave-uniform).
__device__ __forceinline__ uint64_t match_key(bool active, int key, int bits) {
  uint64_t m = __ballot(active);
  for (int q = 0; q < bits; ++q) {
    const bool bit = (key >> q) & 1;
    const uint64_t b = __ballot(bit);
    m &= bit ? b : ~b;
  }
  return m;
}

// cnt[j] += 1 in LDS for every active lane (called by the whole wave).  The lanes whose bin is
// the first active lane's add their number with one atomic: LDS atomics to one address execute
// one lane at a time, so a token holding most rows of a wave (a hot token) would otherwise cost
// 64 serialised atomics per row batch.
__device__ __forceinline__ void count_bins(int* cnt, bool active, uint32_t j) {
  const uint64_t am = __ballot(active);
  if (am == 0) return;  // wave-uniform
  const uint32_t j0 = (uint32_t)__builtin_amdgcn_readlane((int)j, __builtin_ctzll(am));
  const bool same = active && j == j0;
  const uint64_t sm = __ballot(same);
  if (same) {
    if (lanes_below(sm) == 0) atomicAdd(&cnt[j0], __popcll(sm));
  } else if (active) {
    atomicAdd(&cnt[j], 1);
  }
}

}  // namespace fmoe

// Launchers of the bucketed plan (plan_bucket.hip).  BARE: write row numbers (the bare CSR of
// fmoe_invert_scatter_index) instead of records.
namespace fmoe_plan {
int launch_bucketed(const fmoe::TokMetaGlobal* gmeta, const fmoe::TokMetaArgs* ameta,
                    const void* d_indices, int idx_dtype, const void* d_weights, int w_dtype,
                    int64_t N, int64_t T, int64_t E, int64_t row_bytes, void* d_workspace,
                    bool bare, int32_t* d_rows_bare, int32_t* d_row_ptr_bare, hipStream_t s,
                    const char* who);

// Launcher of the radix plan (plan_radix.hip): row_ptr (d_row_ptr), the status words and the
// records (gmeta) or, bare, the row numbers (d_rows_bare), in 3 + 3 x passes launches (two more
// when T + 2 exceeds 16384 bins).
int launch_radix(const fmoe::TokMetaGlobal* gmeta, const void* d_indices, int idx_dtype,
                 const void* d_weights, int w_dtype, int64_t N, int64_t T, int64_t E,
                 int64_t row_bytes, void* d_workspace, int32_t* d_row_ptr, bool bare,
                 int32_t* d_rows_bare, hipStream_t s, const char* who);
}  // namespace fmoe_plan
