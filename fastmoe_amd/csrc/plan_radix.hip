// Radix plan: the token-major inverse of the scatter index for index ranges beyond the bucketed
// plan's (more than 2^22 token bins), or when the "plan" option asks for it (value 1).
//
// A stable least-significant-digit radix sort of the rows by token bin b(g) (idx[g] if it lies in
// [0, T), else T): P = ceil(bits(T) / 8) passes of 8-bit digits.  Pass p moves (bin, g) pairs from
// one buffer to the other; pass 0 reads idx itself, and the last pass writes the plan's records,
// or the bare row numbers, at their final places.  Each pass is three launches over tiles of whole
// 1024-row chunks:
//   k_radix_hist     one 1024-thread workgroup per tile: the tile's digit counts, into the
//                    digit-major table hist[d][tile] and, by atomics, the pass's digit totals;
//   k_radix_scan     one workgroup per digit: the digit's first place (the totals of the lower
//                    digits) plus the exclusive prefix over the tiles, in place in hist;
//   k_radix_scatter  one workgroup per tile, its chunks in order: a row's place is its digit's
//                    cursor + the rows of lower waves with that digit + the lower lanes of its
//                    wave with that digit (ballot match), so every pass is stable.
// Stable passes from the lowest digit up leave the rows sorted by bin with ties in input order,
// i.e. in ascending g: row g lands at row_ptr[b(g)] + (rows of bin b(g) below g), whatever the
// segment lengths.  Every row is read and written once per pass, no workgroup waits for another,
// and the result depends only on the inputs.
//
// row_ptr comes from the last pass too: it also writes each row's bin at its final place (into the
// free pair buffer), k_radix_ends marks where every bin's rows end (end[bin] = place + 1 at the last
// place of each run of equal bins: one plain store per non-empty bin, no atomics), and row_ptr[b]
// = max(end[0 .. b)) is an exclusive max-scan over the bins (k_radix_rp_*), which also gives the
// longest segment and the out-of-range count; a bin's length is max(end[b] - row_ptr[b], 0).
#include <type_traits>

#include "plan.h"

namespace fmoe {

constexpr int kRadixWaves = kRadixThreads / kWave;  // 16
constexpr int kRadixLdsExperts = 4096;              // expert offsets staged in LDS up to this
constexpr int kRpPer = 16;                          // row_ptr bins per scanning thread
constexpr int64_t kRpBlock = (int64_t)kRadixThreads * kRpPer;
static_assert(kRadixThreads == kScanThreads, "the radix scan uses the 1024-thread block scan");
static_assert(kRadixMaxTiles % kRadixThreads == 0, "whole tiles per scanning thread");

// ---- pass inputs: the scatter index (pass 0) or the previous pass's (bin, g) pairs -----------
template <typename TI>
struct RadixFromIdx {
  const TI* idx;
  int64_t T;
  __device__ __forceinline__ void load(int64_t i, int* key, int* g) const {
    const int64_t t = (int64_t)idx[i];
    *key = (uint64_t)t < (uint64_t)T ? (int)t : (int)T;
    *g = (int)i;
  }
};
struct RadixFromPairs {
  const int2* p;
  __device__ __forceinline__ void load(int64_t i, int* key, int* g) const {
    const int2 v = p[i];
    *key = v.x;
    *g = v.y;
  }
};

// ---- pass outputs: pairs for the next pass, or the final records / row numbers ---------------
struct RadixToPairs {
  static constexpr int kLdsExperts = 0;
  int2* p;
  __device__ __forceinline__ void prologue(int64_t*) const {}
  __device__ __forceinline__ void put(int pos, int key, int g, const int64_t*) const {
    p[pos] = make_int2(key, g);
  }
};
struct RadixToRows {
  static constexpr int kLdsExperts = 0;
  int32_t* rows;
  int32_t* skey;  // each place's bin
  __device__ __forceinline__ void prologue(int64_t*) const {}
  __device__ __forceinline__ void put(int pos, int key, int g, const int64_t*) const {
    rows[pos] = g;
    skey[pos] = key;
  }
};
template <typename TW>
struct RadixToRecs {
  static constexpr int kLdsExperts = kRadixLdsExperts;
  Rec* rec;
  int32_t* skey;  // each place's bin
  const TW* w;
  const int64_t* ptr_table;
  const int64_t* offsets;
  int64_t E, row_bytes;
  int32_t* status;
  __device__ __forceinline__ void prologue(int64_t* off_lds) const {
    if (E <= kLdsExperts)
      for (int64_t i = threadIdx.x; i <= E; i += kRadixThreads) off_lds[i] = offsets[i];
  }
  __device__ __forceinline__ void put(int pos, int key, int g, const int64_t* off_lds) const {
    skey[pos] = key;
    const int64_t* off = E <= kLdsExperts ? off_lds : offsets;
    const int64_t e = expert_of_row(off, E, g);
    Rec r;
    r.src = (uint64_t)ptr_table[e] + (uint64_t)(((int64_t)g - off[e]) * row_bytes);
    r.w = ld1(w + g);
    r.g = g;
    rec[pos] = r;
    if (r.src & 15) atomicOr(&status[kStatusMisaligned], 1);
  }
};

__device__ __forceinline__ int64_t radix_tile_end(int64_t lo, int64_t tile, int64_t N) {
  return lo + tile < N ? lo + tile : N;
}

// end[0 .. T + 2) = 0 (grid-strided), the digit totals and the status words cleared.
__global__ __launch_bounds__(kRadixThreads) void k_radix_prep(int32_t* __restrict__ end,
                                                              int64_t nb2,
                                                              int32_t* __restrict__ tot, int ntot,
                                                              int32_t* __restrict__ status) {
  for (int64_t i = (int64_t)blockIdx.x * kRadixThreads + threadIdx.x; i < nb2;
       i += (int64_t)gridDim.x * kRadixThreads)
    end[i] = 0;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < ntot; i += kRadixThreads) tot[i] = 0;
    if (threadIdx.x < 3) status[threadIdx.x] = 0;  // invalid, misaligned, longest
  }
}

template <typename In>
__global__ __launch_bounds__(kRadixThreads) void k_radix_hist(const In in, int64_t N, int64_t tile,
                                                              int ntiles, int shift,
                                                              int32_t* __restrict__ hist,
                                                              int32_t* __restrict__ tot) {
  __shared__ int h[kRadixDigits];
  if (threadIdx.x < kRadixDigits) h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * tile;
  const int64_t hi = radix_tile_end(lo, tile, N);
  constexpr int kU = 4;  // rows per thread in flight
  for (int64_t base = lo; base < hi; base += (int64_t)kRadixThreads * kU) {
    int key[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = base + (int64_t)u * kRadixThreads + threadIdx.x;
      int g;
      key[u] = -1;
      if (i < hi) in.load(i, &key[u], &g);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (key[u] >= 0) atomicAdd(&h[(key[u] >> shift) & (kRadixDigits - 1)], 1);
  }
  __syncthreads();
  if (threadIdx.x < kRadixDigits) {
    const int c = h[threadIdx.x];
    hist[(int64_t)threadIdx.x * ntiles + blockIdx.x] = c;
    if (c) atomicAdd(&tot[threadIdx.x], c);
  }
}

// Workgroup d: hist[d][tile] (counts) becomes the first place of digit d's rows of each tile.
__global__ __launch_bounds__(kRadixThreads) void k_radix_scan(int32_t* __restrict__ hist,
                                                              const int32_t* __restrict__ tot,
                                                              int ntiles) {
  const int d = blockIdx.x;
  __shared__ int base_s;
  if (threadIdx.x < kWave) {  // the rows of the lower digits
    int s = 0;
    for (int j = threadIdx.x; j < d; j += kWave) s += tot[j];
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
    if (threadIdx.x == 0) base_s = s;
  }
  constexpr int kPer = (int)(kRadixMaxTiles / kRadixThreads);
  int32_t* row = hist + (int64_t)d * ntiles;
  const int t0 = (int)threadIdx.x * kPer;
  int v[kPer];
  int local = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    v[u] = t0 + u < ntiles ? row[t0 + u] : 0;
    local += v[u];
  }
  int total;
  const int pre = block_exclusive_scan_1024(local, &total);  // its barriers publish base_s
  int run = base_s + pre;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (t0 + u < ntiles) row[t0 + u] = run;
    run += v[u];
  }
}

// One tile per workgroup, 1024 rows (one per thread) at a time, in order.  Per chunk: each wave's
// rows of each digit are counted by ballot match (the lowest lane of a digit writes the count),
// 256 threads turn the counts into places (digit cursor + lower waves) and advance the cursors,
// and every row goes to its place plus its rank among the lower lanes of its digit.  The wave
// counts alternate between two LDS buffers, the one not in use cleared by the place step, so a
// chunk needs two barriers.
template <typename In, typename Out>
__global__ __launch_bounds__(kRadixThreads) void k_radix_scatter(const In in, const Out out,
                                                                 int64_t N, int64_t tile,
                                                                 int ntiles, int shift,
                                                                 const int32_t* __restrict__ hist) {
  __shared__ int cur[kRadixDigits];
  __shared__ int wcnt[2][kRadixWaves][kRadixDigits];
  __shared__ int64_t off_lds[Out::kLdsExperts + 1];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  out.prologue(off_lds);
  if (tid < kRadixDigits) cur[tid] = hist[(int64_t)tid * ntiles + blockIdx.x];
  for (int i = tid; i < kRadixWaves * kRadixDigits; i += kRadixThreads) (&wcnt[0][0][0])[i] = 0;
  const int64_t lo = (int64_t)blockIdx.x * tile;
  const int64_t hi = radix_tile_end(lo, tile, N);
  bool act = lo + tid < hi;
  int key = 0, g = 0;
  if (act) in.load(lo + tid, &key, &g);
  __syncthreads();
  int buf = 0;
  for (int64_t base = lo; base < hi; base += kRadixThreads) {
    const int d = (key >> shift) & (kRadixDigits - 1);
    const uint64_t m = match_key(act, d, 8);
    const int rank = lanes_below(m);
    const int64_t nxt = base + kRadixThreads + tid;  // the next chunk's row, loaded meanwhile
    const bool act_n = nxt < hi;
    int key_n = 0, g_n = 0;
    if (act_n) in.load(nxt, &key_n, &g_n);
    if (act && rank == 0) wcnt[buf][wv][d] = __popcll(m);
    __syncthreads();
    if (tid < kRadixDigits) {
      int run = cur[tid];
#pragma unroll
      for (int v = 0; v < kRadixWaves; ++v) {
        const int x = wcnt[buf][v][tid];
        wcnt[buf][v][tid] = run;
        wcnt[buf ^ 1][v][tid] = 0;
        run += x;
      }
      cur[tid] = run;
    }
    __syncthreads();
    // places lie in [0, N) when the counts match the rows; the check keeps every store inside the
    // output whatever the inputs
    const int pos = wcnt[buf][wv][d] + rank;
    if (act && (uint32_t)pos < (uint32_t)N) out.put(pos, key, g, off_lds);
    key = key_n;
    g = g_n;
    act = act_n;
    buf ^= 1;
  }
}

// end[skey[i]] = i + 1 where place i is the last of its bin (the next place holds another bin, or
// i = N - 1): exactly one store per non-empty bin.  Bins lie in [0, T]; the check keeps the store
// inside end[] whatever the buffer holds.
__global__ __launch_bounds__(kRadixThreads) void k_radix_ends(const int32_t* __restrict__ skey,
                                                              int64_t N, int64_t T,
                                                              int32_t* __restrict__ end) {
  const int64_t i = (int64_t)blockIdx.x * kRadixThreads + threadIdx.x;
  if (i >= N) return;
  const int k = skey[i];
  if ((uint32_t)k <= (uint32_t)T && (i == N - 1 || skey[i + 1] != k)) end[k] = (int)(i + 1);
}

// ---- row_ptr: exclusive max-scan of end[] over the T + 2 bins --------------------------------
// Exclusive max of one non-negative int per thread over a 1024-thread block; *all gets the block
// max.
__device__ __forceinline__ int block_exclusive_max_1024(int v, int* all) {
  __shared__ int wave_max[kRadixWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  int incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl = max(incl, o);
  }
  int excl = __shfl_up(incl, 1, kWave);
  if (lane == 0) excl = 0;
  if (lane == kWave - 1) wave_max[wv] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kRadixWaves; ++i) {
    const int x = wave_max[i];
    if (i < wv) before = max(before, x);
    tot = max(tot, x);
  }
  __syncthreads();
  *all = tot;
  return max(before, excl);
}

// Per block of kRpBlock bins: the block's max of end[] (for the carries of k_radix_rp_final).
__global__ __launch_bounds__(kRadixThreads) void k_radix_rp_blockmax(const int32_t* __restrict__ end,
                                                                     int64_t nb2,
                                                                     int32_t* __restrict__ bmax) {
  const int64_t b0 = (int64_t)blockIdx.x * kRpBlock + (int64_t)threadIdx.x * kRpPer;
  int m = 0;
#pragma unroll
  for (int u = 0; u < kRpPer; ++u)
    if (b0 + u < nb2) m = max(m, end[b0 + u]);
  int all;
  block_exclusive_max_1024(m, &all);
  if (threadIdx.x == 0) bmax[blockIdx.x] = all;
}

// One workgroup: bmax[0 .. nblk) becomes its exclusive max-scan (each block's carry).
__global__ __launch_bounds__(kRadixThreads) void k_radix_rp_carry(int32_t* __restrict__ bmax,
                                                                  int64_t nblk) {
  int carry = 0;
  for (int64_t base = 0; base < nblk; base += kRpBlock) {
    const int64_t b0 = base + (int64_t)threadIdx.x * kRpPer;
    int v[kRpPer];
    int m = 0;
#pragma unroll
    for (int u = 0; u < kRpPer; ++u) {
      v[u] = b0 + u < nblk ? bmax[b0 + u] : 0;
      m = max(m, v[u]);
    }
    int all;
    int run = max(carry, block_exclusive_max_1024(m, &all));
#pragma unroll
    for (int u = 0; u < kRpPer; ++u) {
      if (b0 + u < nblk) bmax[b0 + u] = run;
      run = max(run, v[u]);
    }
    carry = max(carry, all);
  }
}

// Per block of kRpBlock bins (carry: the max of end[] over the earlier blocks, none for a single
// block): row_ptr[b] = max(end[0 .. b)) in place, the longest segment among bins b < T and the
// rows of bin T (out of range) into the status words.
__global__ __launch_bounds__(kRadixThreads) void k_radix_rp_final(int32_t* __restrict__ rp,
                                                                  int64_t nb2, int64_t T,
                                                                  const int32_t* __restrict__ carry,
                                                                  int32_t* __restrict__ status) {
  const int64_t b0 = (int64_t)blockIdx.x * kRpBlock + (int64_t)threadIdx.x * kRpPer;
  int e[kRpPer];
  int m = 0;
#pragma unroll
  for (int u = 0; u < kRpPer; ++u) {
    e[u] = b0 + u < nb2 ? rp[b0 + u] : 0;
    m = max(m, e[u]);
  }
  int all;
  int run = block_exclusive_max_1024(m, &all);
  if (carry) run = max(run, carry[blockIdx.x]);
  int longest = 0;
#pragma unroll
  for (int u = 0; u < kRpPer; ++u) {
    const int64_t b = b0 + u;
    if (b < nb2) {
      rp[b] = run;
      const int len = max(e[u] - run, 0);
      if (b < T) longest = max(longest, len);
      if (b == T) status[kStatusInvalid] = len;
    }
    run = max(run, e[u]);
  }
  longest = block_max_1024(longest);
  if (threadIdx.x == 0 && longest > 0) atomicMax(&status[kStatusLongest], longest);
}

}  // namespace fmoe

namespace fmoe_plan {

using namespace fmoe;

// The radix plan into the workspace d_workspace of plan_layout(N, T): row_ptr into d_row_ptr, the
// status words, and the records (gmeta: the device expert table) or, bare, the row numbers into
// d_rows_bare.  The caller has checked the arguments.
int launch_radix(const TokMetaGlobal* gmeta, const void* d_indices, int idx_dtype,
                 const void* d_weights, int w_dtype, int64_t N, int64_t T, int64_t E,
                 int64_t row_bytes, void* d_workspace, int32_t* d_row_ptr, bool bare,
                 int32_t* d_rows_bare, hipStream_t s, const char* who) {
  if (!bare && !gmeta) {
    fmoe_host::set_error("%s: no expert table for the plan's records", who);
    return FMOE_EINVAL;
  }
  const RadixGeom rg = radix_geom(N, T);
  const PlanLayout L = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* bmax = reinterpret_cast<int32_t*>(ws + L.cursor);  // T + 1 >= the row_ptr blocks
  int2* pairs[2] = {reinterpret_cast<int2*>(ws + L.rec_tmp),
                    reinterpret_cast<int2*>(ws + L.rec_tmp) + N};
  int32_t* tot = reinterpret_cast<int32_t*>(ws + L.radix_tot);
  int32_t* hist = reinterpret_cast<int32_t*>(ws + L.radix_hist);
  Rec* rec = reinterpret_cast<Rec*>(ws + L.rec);
  const dim3 tiles((unsigned)rg.ntiles), block(kRadixThreads);
  const int64_t nb2 = T + 2;
  const int64_t nblk = (nb2 + kRpBlock - 1) / kRpBlock;

  const unsigned prep_groups = (unsigned)std::min<int64_t>((nb2 + kRadixThreads - 1) / kRadixThreads, 2048);
  hipLaunchKernelGGL(k_radix_prep, dim3(prep_groups), block, 0, s, d_row_ptr, nb2, tot,
                     rg.passes * kRadixDigits, status);
  if (int rc = fmoe_host::check_launch(who)) return rc;

  auto with_input = [&](int p, auto&& f) {
    if (p > 0) f(RadixFromPairs{pairs[(p - 1) & 1]});
    else if (idx_dtype == FMOE_I64) f(RadixFromIdx<int64_t>{static_cast<const int64_t*>(d_indices), T});
    else f(RadixFromIdx<int32_t>{static_cast<const int32_t*>(d_indices), T});
  };
  // the last pass's bins by place, in the pair buffer that pass does not read
  int32_t* skey = reinterpret_cast<int32_t*>(pairs[(rg.passes - 1) & 1]);
  auto with_output = [&](int p, auto&& f) {
    if (p < rg.passes - 1) f(RadixToPairs{pairs[p & 1]});
    else if (bare) f(RadixToRows{d_rows_bare, skey});
    else if (w_dtype == FMOE_F32)
      f(RadixToRecs<float>{rec, skey, static_cast<const float*>(d_weights), gmeta->ptr_table,
                           gmeta->offsets, E, row_bytes, status});
    else if (w_dtype == FMOE_BF16)
      f(RadixToRecs<bf16_t>{rec, skey, static_cast<const bf16_t*>(d_weights), gmeta->ptr_table,
                            gmeta->offsets, E, row_bytes, status});
    else
      f(RadixToRecs<f16_t>{rec, skey, static_cast<const f16_t*>(d_weights), gmeta->ptr_table,
                           gmeta->offsets, E, row_bytes, status});
  };
  for (int p = 0; N > 0 && p < rg.passes; ++p) {
    const int shift = 8 * p;
    int32_t* tot_p = tot + p * kRadixDigits;
    with_input(p, [&](const auto& in) {
      using In = std::decay_t<decltype(in)>;
      hipLaunchKernelGGL((k_radix_hist<In>), tiles, block, 0, s, in, N, rg.tile, rg.ntiles, shift,
                         hist, tot_p);
    });
    if (int rc = fmoe_host::check_launch(who)) return rc;
    hipLaunchKernelGGL(k_radix_scan, dim3(kRadixDigits), block, 0, s, hist, tot_p, rg.ntiles);
    if (int rc = fmoe_host::check_launch(who)) return rc;
    with_input(p, [&](const auto& in) {
      with_output(p, [&](const auto& out) {
        using In = std::decay_t<decltype(in)>;
        using Out = std::decay_t<decltype(out)>;
        hipLaunchKernelGGL((k_radix_scatter<In, Out>), tiles, block, 0, s, in, out, N, rg.tile,
                           rg.ntiles, shift, hist);
      });
    });
    if (int rc = fmoe_host::check_launch(who)) return rc;
  }
  if (N > 0) {
    hipLaunchKernelGGL(k_radix_ends, dim3((unsigned)((N + kRadixThreads - 1) / kRadixThreads)), block,
                       0, s, skey, N, T, d_row_ptr);
    if (int rc = fmoe_host::check_launch(who)) return rc;
  }
  if (nblk > 1) {
    hipLaunchKernelGGL(k_radix_rp_blockmax, dim3((unsigned)nblk), block, 0, s, d_row_ptr, nb2, bmax);
    if (int rc = fmoe_host::check_launch(who)) return rc;
    hipLaunchKernelGGL(k_radix_rp_carry, dim3(1), block, 0, s, bmax, nblk);
    if (int rc = fmoe_host::check_launch(who)) return rc;
  }
  hipLaunchKernelGGL(k_radix_rp_final, dim3((unsigned)nblk), block, 0, s, d_row_ptr, nb2, T,
                     nblk > 1 ? bmax : nullptr, status);
  return fmoe_host::check_launch(who);
}

}  // namespace fmoe_plan
