// Plan: the token-major inverse of the scatter index, built on the device.
//
// The deterministic forward reduces each output row in ascending packed-row order, and the
// backward reads grad_out[t] once for all rows routed from token t.  Both walk, per token t, the
// rows g with idx[g] == t.  This file builds that list as CSR:
//
//   row_ptr[T + 2]  : segment b = [row_ptr[b], row_ptr[b + 1]); b == T holds the rows whose index
//                     is out of range (they are dropped by the forward, zero-filled by the backward)
//   rec[N]          : 16-byte records {source row address, fp32 gate, g}, ascending g in every
//                     segment
//
// Four builders, each linear in N + T and each writing every segment in ascending g (pick_plan
// below chooses):
//   * one launch (k_plan_tok), below 2^16 rows: token-sliced workgroups that each stream all of
//     idx and fill their own segments stably (below);
//   * the ranged plan (k_plan_split + k_plan_range), up to 2^22 rows and 2^19 tokens: partition
//     the rows by token range, then one token-sliced workgroup per range reads only its rows;
//   * the radix plan (plan_radix.hip), for tokens averaging 64 rows or more and beyond the ranged
//     plan's limits: a stable LSD radix sort of the rows by token bin, with row_ptr from the
//     sorted bins, whatever the segment lengths;
//   * the bucketed plan (plan_bucket.hip), only when asked for (option plan=2): partition the
//     rows by token bucket, then order each bucket with one wave.  Fastest on uniform indices
//     beyond the ranged plan's limits, but a hot token's bucket is ordered by one wave.
//
// fmoe_invert_scatter_index writes bare row numbers instead of records (the radix plan, or the
// bucketed plan when asked for).
#include <algorithm>

#include "plan.h"

namespace fmoe {

constexpr int kLdsExperts = 4096;  // expert offsets staged in LDS for the row -> expert search

// ---- one-launch plan: token-sliced, stable --------------------------------------------------
// P workgroups of 16 waves; workgroup p owns the token bins [p * bins, (p + 1) * bins) of the T + 1
// (bin T: out-of-range rows), so every segment belongs to exactly one workgroup and the workgroups
// never communicate.  Every workgroup streams all of idx (from L2 after the first): wave w takes
// the w-th sixteenth of the rows, in ascending g, RPL rows per lane per 16-byte load, and
//   * counts the rows whose bin lies below its workgroup's range (part of row_ptr of its first bin),
//   * stashes its rows of the range (g, bin) in ascending g, then counts the stash per bin into
//     its own LDS row.
// The workgroup then scans its bins bin-major and wave-minor, which gives row_ptr and each wave's
// first place in every bin, and each wave writes the records of its stashed rows: a row goes to its
// wave's cursor for the bin plus its rank among the lower lanes with the same bin.  Every segment
// thus comes out in ascending g with no ordering pass, in time linear in N per workgroup.  A wave
// whose stash overflows (a heavily skewed index) re-streams its own rows to count them and again
// in the fill.
// Every workgroup reading all of idx makes the total work N * P: from 2^16 rows the ranged plan
// takes over, and kTokMaxRows bounds this plan where the ranged plan's limits do not hold.
constexpr int kTokWaves = kScanThreads / kWave;        // 16
constexpr int kTokBins = 512;                          // bins per workgroup at most
constexpr int kTokWaveStash = 256;                     // stashed rows per wave
constexpr int kTokRows = 256;                          // rows per workgroup aimed at
constexpr int kTokGroups = 256;
constexpr int kTokExperts = 4096;                      // expert tables staged in LDS
constexpr int64_t kTokMaxRows = int64_t(1) << 17;
constexpr int kTokLoads = 8;  // 16-byte int64 index loads per lane per batch (half for int32)
static_assert(kTokBins == kRangeMaxBins, "a range of the ranged plan is a token-sliced workgroup");
static_assert(kRangeMaxSlices <= kScanThreads * kRangeSlicesPerThread,
              "k_plan_range reads kRangeSlicesPerThread slices per thread");
static_assert(kRangeMaxGroups <= kScanThreads, "k_plan_split scans one range per thread");
static_assert(kRangeSlice == kScanThreads, "k_plan_split takes one row per thread");

// The expert table of a plan workgroup, loaded into registers when the workgroup starts and
// written to LDS after the pass over idx, so that its load latency overlaps the pass instead of
// preceding it.
template <typename Meta> struct TokMetaRegs;
template <> struct TokMetaRegs<TokMetaGlobal> {
  static constexpr int Q = kTokExperts / kScanThreads;  // experts per thread (the last thread
  int off[Q + 1];                                       // also holds off[kTokExperts])
  uint64_t ptr[Q];
  __device__ __forceinline__ void load(const TokMetaGlobal& m, int ne) {
#pragma unroll
    for (int q = 0; q <= Q; ++q) {
      const int e = (int)threadIdx.x + q * kScanThreads;
      off[q] = e <= ne ? (int)m.offsets[e] : 0;
      if (q < Q) ptr[q] = e < ne ? (uint64_t)m.ptr_table[e] : 0;
    }
  }
  __device__ __forceinline__ void store(const TokMetaGlobal&, int ne, int* off32,
                                        uint64_t* ptr_lds) const {
#pragma unroll
    for (int q = 0; q <= Q; ++q) {
      const int e = (int)threadIdx.x + q * kScanThreads;
      if (e <= ne) off32[e] = off[q];
      if (q < Q && e < ne) ptr_lds[e] = ptr[q];
    }
  }
};
template <> struct TokMetaRegs<TokMetaArgs> {
  int off, next;  // off[e], off[e + 1]
  uint64_t ptr;
  __device__ __forceinline__ void load(const TokMetaArgs& m, int ne) {
    const int e = threadIdx.x;  // ne <= 256 < kScanThreads: one expert per thread
    off = e <= ne ? m.a.off[e] : 0;
    next = e < ne ? m.a.off[e + 1] : 0;
    ptr = e < ne ? (uint64_t)m.a.ptr[e] : 0;
  }
  __device__ __forceinline__ void store(const TokMetaArgs& m, int ne, int* off32,
                                        uint64_t* ptr_lds) const {
    const int e = threadIdx.x;
    if (e <= ne) off32[e] = off;
    if (e < ne) ptr_lds[e] = ptr;
    if (blockIdx.x == 0) {  // workgroup-uniform: the metadata outputs (fmoe_build_metadata's)
      if (e < ne) {
        m.ptr_table[e] = (int64_t)ptr;
        m.chunk_sizes[e] = next - off;
      }
      if (e <= ne) m.offsets[e] = off;
      if (e == 0) *m.max_rows = m.a.max_rows;
    }
  }
};

// Exclusive scan of v and sum of s over a 1024-thread block, in one barrier round.
__device__ __forceinline__ int tok_scan_and_sum(int v, int s, int* sum_s) {
  __shared__ int wave_v[kTokWaves], wave_s[kTokWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int incl = wave_incl_sum(v);
  s = wave_incl_sum(s);  // the wave's sum in its last lane
  if (lane == kWave - 1) {
    wave_v[wv] = incl;
    wave_s[wv] = s;
  }
  __syncthreads();
  int before = 0, tot_s = 0;
#pragma unroll
  for (int i = 0; i < kTokWaves; ++i) {
    before += (i < wv) ? wave_v[i] : 0;
    tot_s += wave_s[i];
  }
  *sum_s = tot_s;
  return before + incl - v;
}

// LDS of a token-sliced plan workgroup (k_plan_tok, k_plan_range).
struct TokLds {
  int cnt[kTokWaves * kTokBins];                // [wave][bin]: counts, then cursors
  int2 stash[kTokWaves * (kTokWaveStash + 1)];  // per wave: (g, local bin) in ascending g, and a
                                                // slot for the rows past the stash
  int off32[kTokExperts + 1];
  uint64_t ptr_lds[kTokExperts];
  int misaligned;
};

// The end of a token-sliced plan workgroup, after each wave has stashed its rows of the range
// [lo, lo + nloc) in ascending g (wcount of them; past kTokWaveStash the stash holds only the
// first): count them per bin (with kPassCounts the caller's pass has counted the rows past the
// stash into L.cnt, and only the stash's are counted here), scan the bins into row_ptr (rows_part:
// this thread's share of the rows before the range, summed over the workgroup) and the per-wave
// cursors, and write each row's record at its wave's cursor for the bin plus its rank among the
// lower lanes of the same bin.
// rows(fn, gates) replays this wave's rows in ascending g, calling fn(act, g, j, gate, e) once per
// 64 rows with every lane, several batches of loads in flight; with `gates` std::true_type it
// also loads each row's gate and finds its expert e (else both are 0): used when the stash
// overflowed.
template <bool kPassCounts, typename TW, typename Meta, typename Rows>
__device__ __forceinline__ void tok_finish(TokLds& L, const TokMetaRegs<Meta>& mreg,
                                           const Meta& meta, int ne, int64_t row_bytes,
                                           const TW* __restrict__ w, int lo, int nloc, int nb,
                                           int wcount, int rows_part, int32_t* __restrict__ row_ptr,
                                           Rec* __restrict__ rec, int32_t* __restrict__ status,
                                           Rows rows) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  int* mycnt = L.cnt + wave * nloc;
  const int2* mystash = L.stash + wave * (kTokWaveStash + 1);
  mreg.store(meta, ne, L.off32, L.ptr_lds);
  // This wave's rows per bin, counted from the stash (when it overflowed: the stash's rows here and
  // the rest by the caller's pass, or all of them from its rows again), and the gates of the
  // stashed rows, loaded before the scan so that their latency overlaps it.
  constexpr int kStashChunks = kTokWaveStash / kWave;
  int2 se[kStashChunks];
  float sw[kStashChunks];
  const bool stashed = wcount <= kTokWaveStash;  // wave-uniform
  if (stashed || kPassCounts) {
#pragma unroll
    for (int q = 0; q < kStashChunks; ++q) {
      const int at = q * kWave + lane;
      const bool act = at < wcount && at < kTokWaveStash;
      se[q] = act ? mystash[at] : make_int2(0, 0);
      sw[q] = act && stashed ? ld1(w + se[q].x) : 0.f;
      if (act) atomicAdd(&mycnt[se[q].y], 1);
    }
  } else {
    rows([&](bool act, int, uint32_t j, float, int) { count_bins(mycnt, act, j); },
         std::false_type{});
  }
  __syncthreads();  // the expert table and every wave's counts

  if (blockIdx.x == 0) {
    // a source row is misaligned iff its expert's base is, or the expert has two or more rows
    // and the row length is not a multiple of 16 bytes
    int mis = 0;
    for (int e = threadIdx.x; e < ne; e += kScanThreads) {
      const int n = L.off32[e + 1] - L.off32[e];
      if (n > 0 && ((L.ptr_lds[e] & 15) || (n > 1 && (row_bytes & 15)))) mis = 1;
    }
    if (mis) L.misaligned = 1;  // read after the next barrier
  }

  // thread j owns bin j of the range: its rows over all waves, row_ptr, and each wave's first
  // place in it (the cursors)
  const int bj = threadIdx.x;
  int tot = 0;
  if (bj < nloc)
    for (int v = 0; v < kTokWaves; ++v) tot += L.cnt[v * nloc + bj];
  int rows_before;
  const int excl = tok_scan_and_sum(tot, rows_part, &rows_before);
  const int hi = lo + nloc;
  if (bj < nloc) {
    int run = rows_before + excl;
    row_ptr[lo + bj] = run;
    if (lo + bj == nb - 1) status[kStatusInvalid] = tot;  // the out-of-range bin
    for (int v = 0; v < kTokWaves; ++v) {
      const int c = L.cnt[v * nloc + bj];
      L.cnt[v * nloc + bj] = run;
      run += c;
    }
    if (hi == nb && bj == nloc - 1) row_ptr[nb] = run;  // == N
  }
  __syncthreads();  // the cursors (and the misaligned flag)
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    status[kStatusMisaligned] = L.misaligned;
    status[kStatusLongest] = -1;  // not recorded: no workgroup sees every segment
  }

  // fill: each wave its rows in ascending g -- from the stash, or replayed if it overflowed
  const int jbits = nloc > 1 ? 32 - __builtin_clz((unsigned)(nloc - 1)) : 0;
  // e: the row's expert, or -1 to look it up here
  auto place = [&](bool act, int g, int j, float wg, int e) {
    const uint64_t m = match_key(act, j, jbits);
    if (act) {
      const int rank = lanes_below(m);
      const int pos = mycnt[j] + rank;
      if (rank == 0) mycnt[j] = pos + __popcll(m);
      if (e < 0) e = expert_of_row32(L.off32, ne, g);
      Rec r;
      r.src = L.ptr_lds[e] + (uint64_t)((int64_t)(g - L.off32[e]) * row_bytes);
      r.w = wg;
      r.g = g;
      rec[pos] = r;
    }
  };
  if (stashed) {
#pragma unroll
    for (int q = 0; q < kStashChunks; ++q)
      if (q * kWave < wcount) place(q * kWave + lane < wcount, se[q].x, se[q].y, sw[q], -1);
  } else {
    rows([&](bool act, int g, uint32_t j, float wg, int e) { place(act, g, (int)j, wg, e); },
         std::true_type{});
  }
}

template <typename TI, typename TW, typename Meta>
__global__ __launch_bounds__(kScanThreads) void k_plan_tok(
    const TI* __restrict__ idx, const TW* __restrict__ w, int64_t N, int64_t T, int bins,
    const Meta meta, int64_t E, int64_t row_bytes, int32_t* __restrict__ row_ptr,
    Rec* __restrict__ rec, int32_t* __restrict__ status) {
  __shared__ TokLds L;
  const int nb = (int)T + 1;
  const int ne = (int)E;
  const int lo = (int)blockIdx.x * bins;  // the host makes every range non-empty
  const int hi = min(nb, lo + bins);
  const int nloc = hi - lo;
  const bool last = hi == nb;  // this workgroup owns bin T, the out-of-range rows
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);

  // 1. pass over this wave's rows [r0, r1) in ascending g.  Every workgroup reads all of idx, so
  //    the pass is bound by the CU's vector ALU, not by bytes: per row it takes the bin, one
  //    compare for "in the range" and one for "below the range" (both as lane masks, the latter
  //    only popcounted), and a row of the range costs a stash write at a slot found from the
  //    masks.  The index is read with 16-byte loads, RPL consecutive rows per lane (a lane's rows,
  //    then the next lane's, so the wave still sees its rows in ascending g).  The rows past the
  //    last whole vector (fewer than RPL) are read one per lane after the pass.
  constexpr int RPL = 16 / (int)sizeof(TI);
  // 16-byte loads per lane per batch: the same rows per batch for either index width (an int32
  // batch with as many loads as an int64 one needs more registers than the kernel may use)
  constexpr int kLoads = kTokLoads * 2 / RPL;
  const int n32 = (int)N;
  const int n_al = n32 - n32 % RPL;  // rows in whole 16-byte vectors
  const int per = ((n32 + kTokWaves - 1) / kTokWaves + kWave - 1) / kWave * kWave;  // 64 | per
  const int r0 = min(n32, wave * per);
  const int r1 = min(n32, r0 + per);
  const int lim = min(r1, n_al);
  const rsrc_t ri = make_rsrc(idx, (uint32_t)(N * (int64_t)sizeof(TI)));  // element loads
  const rsrc_t rv = make_rsrc(idx, (uint32_t)((int64_t)n_al * (int64_t)sizeof(TI)));  // vectors
  auto load_batch = [&](int base, u32x4* v) {  // past n_al: zeros from the range check, no traffic
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int g0 = base + (i * kWave + lane) * RPL;
      v[i] = Raw<16>::template ld<kCPolCached>(rv, (uint32_t)g0 * (uint32_t)sizeof(TI));
    }
  };
  // Two batch buffers used in turn (no register copies, which would make each iteration wait for
  // the next batch's loads), so one batch is always in flight while the other is counted.  The
  // first batch is issued before the LDS set-up and its barrier.
  u32x4 va[kLoads], vb[kLoads];
  if (r0 < lim) load_batch(r0, va);  // wave-uniform

  TokMetaRegs<Meta> mreg;
  mreg.load(meta, ne);  // used after the pass over idx
  for (int i = threadIdx.x; i < kTokWaves * nloc; i += kScanThreads) L.cnt[i] = 0;
  if (threadIdx.x == 0) L.misaligned = 0;
  __syncthreads();

  int2* mystash = L.stash + wave * (kTokWaveStash + 1);
  int below = 0;   // rows of this wave whose bin precedes the range (wave-uniform)
  int wcount = 0;  // rows of the range seen by this wave (wave-uniform)
  auto bin_at = [&](int g, int lim_g, TI raw) -> uint32_t {  // exact; 0xffffffff: not a row here
    const int64_t t = (int64_t)raw;
    return g < lim_g ? ((uint64_t)t < (uint64_t)T ? (uint32_t)t : (uint32_t)T) : 0xffffffffu;
  };
  // The local bin of a row of the range: lo_j is lo, kept out of the compiler's sight so that
  // it does not fold the subtraction into the "below" compare (whose borrow it would then turn
  // back into a lane mask with two more instructions per row).
  uint32_t lo_j = (uint32_t)lo;
  asm volatile("" : "+s"(lo_j));
  // rows g0 .. g0 + RPL - 1 of this lane, bins b (0xffffffff: no row).  Per row two compares
  // give lane masks, below = b < lo and in = b < hi and not below.  A row of the range goes to
  // the stash slot that counts the range's rows of the lower lanes (all RPL of theirs) and of this
  // lane's lower rows; a slot past the stash goes to the wave's overflow slot (the fill then
  // re-reads the wave's rows).
  auto count_vec = [&](int g0, const uint32_t* b) {
    uint64_t m[RPL];
    uint64_t any = 0;
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      const uint64_t mb = __ballot(b[r] < (uint32_t)lo);
      m[r] = __ballot(b[r] < (uint32_t)hi) & ~mb;
      below += __popcll(mb);
      any |= m[r];
    }
    if (any) {  // wave-uniform
      uint32_t slot = (uint32_t)wcount;
#pragma unroll
      for (int r = 0; r < RPL; ++r)
        slot = __builtin_amdgcn_mbcnt_hi((uint32_t)(m[r] >> 32),
                                         __builtin_amdgcn_mbcnt_lo((uint32_t)m[r], slot));
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        if (m[r]) {  // wave-uniform
          const uint32_t j = b[r] - lo_j;
          const bool in = j < (uint32_t)nloc;
          if (in) mystash[min(slot, (uint32_t)kTokWaveStash)] = make_int2(g0 + r, (int)j);
          slot += in ? 1u : 0u;
          wcount += __popcll(m[r]);
        }
      }
    }
  };
  auto row_of = [](const u32x4& v, int r) -> TI {
    if constexpr (sizeof(TI) == 8)
      return (TI)((uint64_t)v[2 * r] | ((uint64_t)v[2 * r + 1] << 32));
    else
      return (TI)v[r];
  };
  constexpr int kBatchRows = kLoads * kWave * RPL;
  // A whole batch below lim whose rows are all below 2^32 as unsigned 64-bit values (int64: every
  // high word zero; int32 always) takes the low word as the bin as it is: a value of T or more,
  // or a negative int32, is then neither in a range that ends at or below T nor below it, so only
  // the workgroup of bin T clamps it to T.  Anything else takes the exact per-row path.
  auto count_fast = [&](int base, const u32x4* v, auto owns_invalid) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int g0 = base + (i * kWave + lane) * RPL;
      uint32_t b[RPL];
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const uint32_t x = sizeof(TI) == 8 ? v[i][2 * r] : v[i][r];
        b[r] = decltype(owns_invalid)::value ? min(x, (uint32_t)T) : x;
      }
      count_vec(g0, b);
    }
  };
  auto count_batch = [&](int base, const u32x4* v) {
    bool exact = base + kBatchRows > lim;  // wave-uniform
    if constexpr (sizeof(TI) == 8) {
      if (!exact) {
        uint32_t high = 0;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) high |= v[i][1] | v[i][3];
        exact = __ballot(high != 0) != 0;
      }
    }
    if (!exact) {
      if (last) count_fast(base, v, std::true_type{});
      else count_fast(base, v, std::false_type{});
    } else {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int g0 = base + (i * kWave + lane) * RPL;
        uint32_t b[RPL];
#pragma unroll
        for (int r = 0; r < RPL; ++r) b[r] = bin_at(g0 + r, lim, row_of(v[i], r));
        count_vec(g0, b);
      }
    }
  };
  if (r0 < lim) {  // wave-uniform
    // The loads are unconditional: past the range they return zeros without traffic.
    for (int base = r0; base < lim; base += 2 * kBatchRows) {
      load_batch(base + kBatchRows, vb);
      count_batch(base, va);
      if (base + kBatchRows >= lim) break;  // wave-uniform
      load_batch(base + 2 * kBatchRows, va);
      count_batch(base + kBatchRows, vb);
    }
  }
  if (r1 > n_al && r0 < r1) {  // wave-uniform: the rows past the last whole vector
    const int g = max(r0, n_al) + lane;
    const uint32_t b = bin_at(g, r1, __builtin_bit_cast(TI, Raw<sizeof(TI)>::template ld<kCPolCached>(
                                                     ri, (uint32_t)g * (uint32_t)sizeof(TI))));
    // one row per lane: the slot rule of count_vec with a single row
    const uint64_t mb = __ballot(b < (uint32_t)lo);
    const uint64_t m = __ballot(b < (uint32_t)hi) & ~mb;
    below += __popcll(mb);
    if (m) {  // wave-uniform
      const uint32_t slot = (uint32_t)wcount + (uint32_t)lanes_below(m);
      const uint32_t j = b - lo_j;
      if (j < (uint32_t)nloc) mystash[min(slot, (uint32_t)kTokWaveStash)] = make_int2(g, (int)j);
      wcount += __popcll(m);
    }
  }
  // this wave's rows again, for a stash that overflowed: kReplay batches of 64 rows in flight
  // (the index loads past r1 read rows of other waves or, past N, zeros from the range check, and
  // bin_at discards them); a row's gate is loaded only when it is in the range
  constexpr int kReplay = 8;
  auto rows = [&](auto fn, auto gates) {
    constexpr bool kGates = decltype(gates)::value;
    for (int base = r0; base < r1; base += kReplay * kWave) {
      TI raw[kReplay];
#pragma unroll
      for (int k = 0; k < kReplay; ++k)
        raw[k] = __builtin_bit_cast(TI, Raw<sizeof(TI)>::template ld<kCPolCached>(
                                            ri, (uint32_t)(base + k * kWave + lane) * (uint32_t)sizeof(TI)));
      uint32_t j[kReplay];
      float wg[kReplay];
      int gk[kReplay], ek[kReplay];
#pragma unroll
      for (int k = 0; k < kReplay; ++k) {
        const int g = base + k * kWave + lane;
        j[k] = bin_at(g, r1, raw[k]) - (uint32_t)lo;
        wg[k] = kGates && j[k] < (uint32_t)nloc ? ld1(w + g) : 0.f;
        gk[k] = j[k] < (uint32_t)nloc ? g : 0;
      }
      if constexpr (kGates) {
        last_le(L.off32, ne, gk, ek, min(kReplay, (r1 - base + kWave - 1) / kWave));
      } else {
#pragma unroll
        for (int k = 0; k < kReplay; ++k) ek[k] = 0;
      }
#pragma unroll
      for (int k = 0; k < kReplay; ++k)
        if (base + k * kWave < r1)  // wave-uniform
          fn(j[k] < (uint32_t)nloc, base + k * kWave + lane, j[k], wg[k], ek[k]);
    }
  };
  tok_finish<false>(L, mreg, meta, ne, row_bytes, w, lo, nloc, nb, wcount,
                    lane == 0 ? below : 0, row_ptr, rec, status, rows);
}

// ---- ranged plan: two launches, each CU reading only its share of idx -----------------------
// The one-launch plan has every workgroup read all of idx, N * 8 bytes through each CU's L1, which
// bounds it from about 2^16 rows up.  The ranged plan reads idx once:
//   k_plan_split  one 1024-thread workgroup per slice of kRangeSlice rows, one row per thread.  A
//                 row's range is bin / bins (range_geom).  Each wave counts its rows per range by
//                 ballot match, the workgroup scans the counts range-major and wave-minor, and each
//                 row goes to the slice's range-major partition at its wave's cursor plus its rank
//                 among the lower lanes of the same range, so the rows of one range keep ascending
//                 g.  Per range and slice it writes the row count and the rows of lower ranges,
//                 range-major (rcnt[q][s], rpre[q][s]).
//   k_plan_range  one 1024-thread workgroup per range.  The range's rows are, slice after slice,
//                 part[s * S + rpre[q][s] ..] (rcnt[q][s] of them), in ascending g; the rows before
//                 the range number sum_s rpre[q][s].  Wave v takes the v-th sixteenth of the
//                 range's rows in order and stashes them as the one-launch plan's pass does; the
//                 workgroup then ends like it (tok_finish).
template <typename TI>
__global__ __launch_bounds__(kScanThreads) void k_plan_split(
    const TI* __restrict__ idx, int64_t N, int64_t T, int Q, uint64_t magic, int G1,
    int2* __restrict__ part, int32_t* __restrict__ rcnt, int32_t* __restrict__ rpre) {
  __shared__ int cnt[kTokWaves * kRangeMaxGroups];  // [wave][range]: counts, then cursors
  const int wave = threadIdx.x / kWave;
  const int s = blockIdx.x;
  const int64_t g = (int64_t)s * kRangeSlice + threadIdx.x;
  const bool act = g < N;
  int bin = 0, q = 0;
  if (act) {
    const int64_t t = (int64_t)idx[g];
    bin = (uint64_t)t < (uint64_t)T ? (int)t : (int)T;
    q = (int)(((uint64_t)(uint32_t)bin * magic) >> 32);
  }
  for (int i = threadIdx.x; i < kTokWaves * Q; i += kScanThreads) cnt[i] = 0;
  __syncthreads();
  const int qbits = Q > 1 ? 32 - __builtin_clz((unsigned)(Q - 1)) : 0;
  const uint64_t m = match_key(act, q, qbits);
  const int rank = lanes_below(m);
  if (act && rank == 0) cnt[wave * Q + q] = __popcll(m);  // one writer per (wave, range)
  __syncthreads();
  // thread i owns range i: the slice's rows in it, the slice's rows in lower ranges, and each
  // wave's first place in it
  const int qi = threadIdx.x;
  int tot = 0;
  if (qi < Q)
    for (int v = 0; v < kTokWaves; ++v) tot += cnt[v * Q + qi];
  int all;
  const int pre = block_exclusive_scan_1024(tot, &all);
  if (qi < Q) {
    int run = pre;
    for (int v = 0; v < kTokWaves; ++v) {
      const int c = cnt[v * Q + qi];
      cnt[v * Q + qi] = run;
      run += c;
    }
    rcnt[(int64_t)qi * G1 + s] = tot;
    rpre[(int64_t)qi * G1 + s] = pre;
  }
  __syncthreads();
  if (act) part[(int64_t)s * kRangeSlice + cnt[wave * Q + q] + rank] = make_int2((int)g, bin);
}

template <typename TW, typename Meta>
__global__ __launch_bounds__(kScanThreads) void k_plan_range(
    const int2* __restrict__ part, const int32_t* __restrict__ rcnt,
    const int32_t* __restrict__ rpre, int G1, int64_t T, int bins, const TW* __restrict__ w,
    const Meta meta, int64_t E, int64_t row_bytes, int32_t* __restrict__ row_ptr,
    Rec* __restrict__ rec, int32_t* __restrict__ status) {
  __shared__ TokLds L;
  __shared__ int first[kRangeMaxSlices + 1];  // rows of this range in the slices before s
  __shared__ int at[kRangeMaxSlices];         // partition index of slice s's first row of it
  constexpr int SPT = kRangeSlicesPerThread;
  const int nb = (int)T + 1;
  const int ne = (int)E;
  const int q = blockIdx.x;
  const int lo = q * bins;  // the host makes every range non-empty
  const int nloc = min(nb, lo + bins) - lo;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  // this range's rows in every slice: thread t reads the count and prefix of slices
  // [t * SPT, t * SPT + SPT)
  const int s0 = (int)threadIdx.x * SPT;
  int c[SPT], p[SPT];
  int csum = 0, psum = 0;
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const bool in = s0 + r < G1;
    c[r] = in ? rcnt[(int64_t)q * G1 + s0 + r] : 0;
    p[r] = in ? rpre[(int64_t)q * G1 + s0 + r] : 0;
    csum += c[r];
    psum += p[r];
  }
  TokMetaRegs<Meta> mreg;
  mreg.load(meta, ne);  // used after the gather
  for (int i = threadIdx.x; i < kTokWaves * nloc; i += kScanThreads) L.cnt[i] = 0;
  if (threadIdx.x == 0) L.misaligned = 0;
  int before;  // rows of lower ranges: the sum over the slices
  int run = tok_scan_and_sum(csum, psum, &before);
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    if (s0 + r < G1) {
      first[s0 + r] = run;
      at[s0 + r] = (s0 + r) * kRangeSlice + p[r];
      run += c[r];
      if (s0 + r == G1 - 1) first[G1] = run;
    }
  }
  __syncthreads();
  const int nrows = first[G1];

  // Wave v takes rows [p0, p1) of the range in order; row i is in the last slice a with
  // first[a] <= i (first[G1] = nrows > i).
  const int per = ((nrows + kTokWaves - 1) / kTokWaves + kWave - 1) / kWave * kWave;
  const int p0 = min(nrows, wave * per);
  const int p1 = min(nrows, p0 + per);
  constexpr int kGather = 4;  // chunks of at most 64 rows in flight
  // The wave's rows in order, kGather chunks per batch: chunk k holds n[k] rows (0: none), lane
  // l < n[k] gets v[k] = (g, bin) of its row, the others `none`.  A sparse range (fewer than 64
  // rows per slice on average) takes chunks of 64 consecutive rows and finds each lane's slice by
  // binary search over first[].  A dense one (a hot token's range) walks the slices in order, a
  // chunk ending at the end of its slice, with no search per row: its rows are contiguous in the
  // slice's part of the partition.
  const bool dense = nrows >= kWave * G1;  // workgroup-uniform
  struct Walk {
    int i;  // next row of the wave's share
    int s;  // its slice (dense walk)
  };
  auto walk_start = [&]() -> Walk {
    Walk wk{p0, 0};
    if (dense && p0 < p1) {  // wave-uniform
      int a = 0, b = G1;  // the last slice a with first[a] <= p0
      while (b - a > 1) {
        const int mid = (a + b) >> 1;
        if (__builtin_amdgcn_readfirstlane(first[mid]) <= p0) a = mid; else b = mid;
      }
      wk.s = a;
    }
    return wk;
  };
  auto next_batch = [&](Walk& wk, int2 (&v)[kGather], int (&n)[kGather], int2 none) {
#pragma unroll
    for (int k = 0; k < kGather; ++k) {
      v[k] = none;
      n[k] = 0;
      if (wk.i < p1) {  // wave-uniform
        if (dense) {
          int end = __builtin_amdgcn_readfirstlane(first[wk.s + 1]);
          while (end <= wk.i) end = __builtin_amdgcn_readfirstlane(first[++wk.s + 1]);
          const int c = min(kWave, min(end, p1) - wk.i);
          if (lane < c) v[k] = part[at[wk.s] + (wk.i - first[wk.s]) + lane];
          n[k] = c;
        } else {
          const int i = wk.i + lane;
          const int c = min(kWave, p1 - wk.i);
          if (lane < c) {
            int a = 0, b = G1;
            while (b - a > 1) {
              const int mid = (a + b) >> 1;
              if (first[mid] <= i) a = mid; else b = mid;
            }
            v[k] = part[at[a] + (i - first[a])];
          }
          n[k] = c;
        }
        wk.i += n[k];
      }
    }
  };
  int2* mystash = L.stash + wave * (kTokWaveStash + 1);
  int* mycnt = L.cnt + wave * nloc;  // zeroed before the scan's barriers above
  int wcount = 0;  // wave-uniform
  for (Walk wk = walk_start(); wk.i < p1;) {
    int2 v[kGather];
    int n[kGather];
    next_batch(wk, v, n, make_int2(0, -1));
#pragma unroll
    for (int k = 0; k < kGather; ++k) {
      const bool in = lane < n[k];
      const uint64_t m = __ballot(in);
      const uint32_t slot = (uint32_t)wcount + (uint32_t)lanes_below(m);
      if (in) mystash[min(slot, (uint32_t)kTokWaveStash)] = make_int2(v[k].x, v[k].y - lo);
      // the rows past the stash are counted here, so that tok_finish<true> need not replay them
      if (wcount + __popcll(m) > kTokWaveStash)  // wave-uniform
        count_bins(mycnt, in && slot >= (uint32_t)kTokWaveStash, (uint32_t)(v[k].y - lo));
      wcount += __popcll(m);
    }
  }
  // the same walk again; the gates and experts of a batch side by side
  auto rows = [&](auto fn, auto gates) {
    constexpr bool kGates = decltype(gates)::value;
    for (Walk wk = walk_start(); wk.i < p1;) {
      int2 v[kGather];
      int n[kGather];
      next_batch(wk, v, n, make_int2(0, lo));
      float wg[kGather];
      int gk[kGather], ek[kGather];
      int kn = 0;  // chunks with rows: a prefix
#pragma unroll
      for (int k = 0; k < kGather; ++k) {
        wg[k] = kGates && lane < n[k] ? ld1(w + v[k].x) : 0.f;
        gk[k] = v[k].x;  // 0 past the rows
        kn += n[k] > 0 ? 1 : 0;
      }
      if constexpr (kGates) {
        last_le(L.off32, ne, gk, ek, kn);
      } else {
#pragma unroll
        for (int k = 0; k < kGather; ++k) ek[k] = 0;
      }
#pragma unroll
      for (int k = 0; k < kGather; ++k)
        if (n[k] > 0)  // wave-uniform
          fn(lane < n[k], v[k].x, (uint32_t)(v[k].y - lo), wg[k], ek[k]);
    }
  };
  tok_finish<true>(L, mreg, meta, ne, row_bytes, w, lo, nloc, nb, wcount,
                   threadIdx.x == 0 ? before : 0, row_ptr, rec, status, rows);
}

// ---- plan of a combine fed by the dispatch permutation -------------------------------------
// fmoe_permute_build already knows every token's rows: slot t * k + j sits at packed row
// slot_pos[t * k + j].  When every slot is a row of the combine (N == T * k), token t's segment
// is exactly slots [t * k, t * k + k): row_ptr[t] = t * k and one thread per slot writes its
// record -- no count, scan or atomics.  Segments have k <= 64 rows, so the consumers order them in
// registers and the ordering pass is not needed.  A slot_pos entry outside [0, N) (an
// inconsistent caller) yields a zero-gate record on packed row 0, so nothing is ever addressed
// outside the expert buffers.
// Expert offsets (and, from kernel arguments, base addresses) of the slot-map plan in LDS.
__device__ __forceinline__ void slots_load_meta(const TokMetaGlobal& m, int64_t E,
                                                int64_t* off_lds, uint64_t*) {
  for (int i = threadIdx.x; i <= E; i += kGroup) off_lds[i] = m.offsets[i];
}
__device__ __forceinline__ uint64_t slots_ptr(const TokMetaGlobal& m, const uint64_t*, int64_t e) {
  return (uint64_t)m.ptr_table[e];
}
// E <= 256 == kGroup: one expert per thread copies the host-prefixed table into LDS, and
// workgroup 0 writes the metadata outputs (fmoe_build_metadata's).
__device__ __forceinline__ void slots_load_meta(const TokMetaArgs& m, int64_t E, int64_t* off_lds,
                                                uint64_t* ptr_lds) {
  const int e = threadIdx.x;
  if (e < E) {
    off_lds[e] = m.a.off[e];
    ptr_lds[e] = (uint64_t)m.a.ptr[e];
  }
  if (e == 0) off_lds[E] = m.a.off[E];
  if (blockIdx.x == 0) {
    if (e < E) {
      m.ptr_table[e] = m.a.ptr[e];
      m.chunk_sizes[e] = m.a.off[e + 1] - m.a.off[e];
      m.offsets[e] = m.a.off[e];
    }
    if (e == 0) {
      m.offsets[E] = m.a.off[E];
      *m.max_rows = m.a.max_rows;
    }
  }
}
__device__ __forceinline__ uint64_t slots_ptr(const TokMetaArgs&, const uint64_t* ptr_lds,
                                              int64_t e) {
  return ptr_lds[e];
}

template <typename TW, typename Meta>
__global__ __launch_bounds__(kGroup) void k_plan_from_slots(
    const int32_t* __restrict__ slot_pos, int64_t T, int64_t k, const TW* __restrict__ w,
    const Meta meta, int64_t E, int64_t row_bytes, int32_t* __restrict__ row_ptr,
    Rec* __restrict__ rec, int32_t* __restrict__ status) {
  __shared__ int64_t off_lds[kLdsExperts + 1];
  __shared__ uint64_t ptr_lds[kMetaChunk];  // used when the table comes in the arguments
  __shared__ int misaligned;
  slots_load_meta(meta, E, off_lds, ptr_lds);
  if (threadIdx.x == 0) misaligned = 0;
  __syncthreads();
  const int64_t N = T * k;  // == off_lds[E], checked on the host
  const int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x;
  if (i < N) {
    const int64_t p = slot_pos[i];
    const bool ok = p >= 0 && p < N;
    const int64_t g = ok ? p : 0;
    const int64_t e = expert_of_row(off_lds, E, g);
    Rec r;
    r.src = slots_ptr(meta, ptr_lds, e) + (uint64_t)((g - off_lds[e]) * row_bytes);
    r.w = ok ? ld1(w + g) : 0.f;
    r.g = (int32_t)g;
    rec[i] = r;
  }
  if (i <= T + 1) row_ptr[i] = (int32_t)(std::min<int64_t>(i, T) * k);
  // Block 0 also writes the status words: no invalid rows, the longest segment is k, and a row
  // is misaligned iff its expert's base or the row length is not a multiple of 16 bytes.
  if (blockIdx.x == 0) {
    for (int64_t x = threadIdx.x; x < E; x += kGroup)
      if (off_lds[x + 1] > off_lds[x] && ((slots_ptr(meta, ptr_lds, x) & 15) || (row_bytes & 15)))
        misaligned = 1;
    __syncthreads();
    if (threadIdx.x == 0) {
      status[kStatusInvalid] = 0;
      status[kStatusMisaligned] = misaligned;
      status[kStatusLongest] = (int32_t)k;
    }
  }
}

}  // namespace fmoe

namespace {

// Grid of the one-launch plan, or false when its limits do not hold (row count aside: the caller
// weighs N).
bool tok_grid(int64_t N, int64_t T, int64_t E, int64_t* groups_out, int64_t* bins_out) {
  using namespace fmoe;
  const int64_t nb = T + 1;
  int64_t groups = std::max<int64_t>((N + kTokRows - 1) / kTokRows, (nb + kTokBins - 1) / kTokBins);
  groups = std::min<int64_t>(std::min<int64_t>(groups, kTokGroups), nb);
  if (const int64_t forced = fmoe_host::opt(fmoe_host::kOptPlanGroups); forced > 0)
    groups = std::min<int64_t>(std::min<int64_t>(forced, kTokGroups), nb);
  const int64_t bins = (nb + groups - 1) / groups;
  groups = (nb + bins - 1) / bins;  // every workgroup gets a non-empty bin range
  *groups_out = groups;
  *bins_out = bins;
  // index loads use 32-bit byte offsets (rows past N by up to one batch included)
  return E <= kTokExperts && N <= (int64_t(1) << 28) && bins <= kTokBins;
}

template <typename Meta>
int launch_plan_tok(const Meta& meta, const void* d_indices, int idx_dtype, const void* d_weights,
                    int w_dtype, int64_t N, int64_t T, int64_t E, int64_t row_bytes,
                    int64_t groups, int64_t bins, int32_t* row_ptr, fmoe::Rec* rec,
                    int32_t* status, hipStream_t s) {
  using namespace fmoe;
#define FMOE_TOK(TI, TW)                                                                           \
  hipLaunchKernelGGL((k_plan_tok<TI, TW, Meta>), dim3((unsigned)groups), dim3(kScanThreads), 0, s, \
                     static_cast<const TI*>(d_indices), static_cast<const TW*>(d_weights), N, T,   \
                     (int)bins, meta, E, row_bytes, row_ptr, rec, status)
#define FMOE_TOK_W(TI)                                 \
  if (w_dtype == FMOE_F32) FMOE_TOK(TI, float);        \
  else if (w_dtype == FMOE_BF16) FMOE_TOK(TI, bf16_t); \
  else FMOE_TOK(TI, f16_t)
  if (idx_dtype == FMOE_I64) { FMOE_TOK_W(int64_t); } else { FMOE_TOK_W(int32_t); }
#undef FMOE_TOK_W
#undef FMOE_TOK
  return fmoe_host::check_launch("fmoe_build_plan(one launch)");
}

// The ranged plan: k_plan_split, then k_plan_range (range_geom(N, T).ok and E <= kTokExperts,
// checked by the caller).
template <typename Meta>
int launch_plan_ranged(const Meta& meta, const void* d_indices, int idx_dtype,
                       const void* d_weights, int w_dtype, int64_t N, int64_t T, int64_t E,
                       int64_t row_bytes, void* d_workspace, hipStream_t s) {
  using namespace fmoe;
  const RangeGeom g = range_geom(N, T);
  const PlanLayout L = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* row_ptr = reinterpret_cast<int32_t*>(ws + L.row_ptr);
  Rec* rec = reinterpret_cast<Rec*>(ws + L.rec);
  int2* part = reinterpret_cast<int2*>(ws + L.part);
  int32_t* rcnt = reinterpret_cast<int32_t*>(ws + L.rcnt);
  int32_t* rpre = reinterpret_cast<int32_t*>(ws + L.rpre);
  if (idx_dtype == FMOE_I64)
    hipLaunchKernelGGL(k_plan_split<int64_t>, dim3((unsigned)g.G1), dim3(kScanThreads), 0, s,
                       static_cast<const int64_t*>(d_indices), N, T, g.Q, g.magic, g.G1, part,
                       rcnt, rpre);
  else
    hipLaunchKernelGGL(k_plan_split<int32_t>, dim3((unsigned)g.G1), dim3(kScanThreads), 0, s,
                       static_cast<const int32_t*>(d_indices), N, T, g.Q, g.magic, g.G1, part,
                       rcnt, rpre);
  if (int rc = fmoe_host::check_launch("fmoe_build_plan(ranged, split)")) return rc;
#define FMOE_RANGE(TW)                                                                         \
  hipLaunchKernelGGL((k_plan_range<TW, Meta>), dim3((unsigned)g.Q), dim3(kScanThreads), 0, s,  \
                     part, rcnt, rpre, g.G1, T, g.bins, static_cast<const TW*>(d_weights), meta, \
                     E, row_bytes, row_ptr, rec, status)
  if (w_dtype == FMOE_F32) FMOE_RANGE(float);
  else if (w_dtype == FMOE_BF16) FMOE_RANGE(bf16_t);
  else FMOE_RANGE(f16_t);
#undef FMOE_RANGE
  return fmoe_host::check_launch("fmoe_build_plan(ranged)");
}

// Which plan builds the records by default: when the tokens average kRadixRowsPerToken rows or
// more, the radix plan, whose cost does not depend on how the rows spread over the tokens (the
// others give a token's rows to one workgroup or wave); else the one-launch plan below
// kRangedMinRows rows, where reading all of idx in every workgroup costs less than a second
// launch; then the ranged plan wherever its limits hold (from 2^21 rows its ranges outnumber the
// CUs and it is some 7 % slower than the bucketed plan on uniform indices, but a hot token costs it
// one CU's time, against one wave's in the bucketed plan); then the one-launch plan up to
// kTokMaxRows rows, and else the radix plan.  The bucketed plan is taken only when asked for.
// Top-k routing (k <= 64 rows per token) takes the radix plan only beyond the ranged plan's
// limits.  Option "plan": 0 automatic, 1 radix, 2 bucketed, 3 one launch, 4 ranged (a forced path
// whose limits do not hold falls back to the automatic choice).
enum PlanPath { kPathTok, kPathRanged, kPathBucketed, kPathRadix };
constexpr int64_t kRadixRowsPerToken = 64;
constexpr int64_t kRangedMinRows = int64_t(1) << 16;
bool long_segments(int64_t N, int64_t T) { return N >= kRadixRowsPerToken * (T + 1); }
PlanPath pick_plan(int64_t N, int64_t T, int64_t E, int64_t* groups, int64_t* bins) {
  const int64_t algo = fmoe_host::opt(fmoe_host::kOptPlan);
  const bool tok = tok_grid(N, T, E, groups, bins);
  const bool ranged = fmoe::range_geom(N, T).ok && E <= fmoe::kTokExperts;
  const bool bucketed = fmoe::plan_geom(N, T).ok;
  if (algo == 1) return kPathRadix;
  if (algo == 2) return bucketed ? kPathBucketed : kPathRadix;
  if (algo == 3 && tok) return kPathTok;
  if (algo == 4 && ranged) return kPathRanged;
  if (long_segments(N, T)) return kPathRadix;
  if (tok && N < kRangedMinRows) return kPathTok;
  if (ranged) return kPathRanged;
  if (tok && N <= fmoe::kTokMaxRows) return kPathTok;
  return kPathRadix;
}

}  // namespace

extern "C" int fmoe_plan_path(int64_t num_rows, int64_t num_tokens, int64_t num_experts) {
  if (num_rows < 0 || num_tokens < 1 || num_tokens >= (int64_t(1) << 30) ||
      num_rows >= (int64_t(1) << 31) || num_experts < 1)
    return -1;
  int64_t groups = 0, bins = 0;
  switch (pick_plan(num_rows, num_tokens, num_experts, &groups, &bins)) {
    case kPathRadix: return 1;
    case kPathBucketed: return 2;
    case kPathTok: return 3;
    case kPathRanged: return 4;
  }
  return -1;
}

extern "C" int64_t fmoe_plan_workspace_bytes(int64_t num_rows, int64_t num_tokens) {
  if (num_rows < 0 || num_tokens < 1) return -1;
  return fmoe::plan_layout(num_rows, num_tokens).total;
}
extern "C" int64_t fmoe_plan_status_offset(void) { return 0; }
extern "C" int64_t fmoe_plan_row_ptr_offset(int64_t num_rows, int64_t num_tokens) {
  return fmoe::plan_layout(num_rows, num_tokens).row_ptr;
}
extern "C" int64_t fmoe_plan_records_offset(int64_t num_rows, int64_t num_tokens) {
  return fmoe::plan_layout(num_rows, num_tokens).rec;
}
extern "C" int fmoe_build_plan(const void* d_indices, int idx_dtype, const void* d_weights,
                               int w_dtype, int64_t num_rows, int64_t num_tokens,
                               const int64_t* d_ptr_table, const int64_t* d_offsets,
                               int64_t num_experts, int64_t row_bytes, void* d_workspace,
                               void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const int64_t N = num_rows, T = num_tokens, E = num_experts;
  FMOE_REQUIRE(N >= 0, "fmoe_build_plan: num_rows must be >= 0");
  FMOE_REQUIRE(T >= 1, "fmoe_build_plan: num_tokens must be >= 1");
  FMOE_REQUIRE(E >= 1, "fmoe_build_plan: num_experts must be >= 1");
  if (N >= (int64_t(1) << 31) || T >= (int64_t(1) << 30)) {
    fmoe_host::set_error("fmoe_build_plan: N=%lld / T=%lld exceed the 32-bit row counters",
                         (long long)N, (long long)T);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype), "fmoe_build_plan: bad index dtype %d",
               idx_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "fmoe_build_plan: bad weight dtype %d", w_dtype);
  FMOE_REQUIRE(d_workspace && d_ptr_table && d_offsets, "fmoe_build_plan: null device pointer");
  FMOE_REQUIRE(N == 0 || (d_indices && d_weights), "fmoe_build_plan: null indices/weights");
  FMOE_REQUIRE(((uintptr_t)d_workspace & 255) == 0, "fmoe_build_plan: workspace not 256B-aligned");
  FMOE_REQUIRE(row_bytes > 0, "fmoe_build_plan: row_bytes must be > 0");

  hipStream_t s = static_cast<hipStream_t>(stream);
  const PlanLayout L = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* row_ptr = reinterpret_cast<int32_t*>(ws + L.row_ptr);
  Rec* rec = reinterpret_cast<Rec*>(ws + L.rec);

  // The one-launch, ranged, bucketed or radix plan (pick_plan; tests compare the paths through the
  // "plan" option).
  const TokMetaGlobal meta{d_ptr_table, d_offsets};
  int64_t groups = 0, bins = 0;
  const PlanPath path = pick_plan(N, T, E, &groups, &bins);
  if (path == kPathTok)
    return launch_plan_tok(meta, d_indices, idx_dtype, d_weights, w_dtype, N, T, E, row_bytes,
                           groups, bins, row_ptr, rec, status, s);
  if (path == kPathRanged)
    return launch_plan_ranged(meta, d_indices, idx_dtype, d_weights, w_dtype, N, T, E, row_bytes,
                              d_workspace, s);
  if (path == kPathBucketed)
    return fmoe_plan::launch_bucketed(&meta, nullptr, d_indices, idx_dtype, d_weights, w_dtype, N,
                                      T, E, row_bytes, d_workspace, false, nullptr, nullptr, s,
                                      "fmoe_build_plan");

  return fmoe_plan::launch_radix(&meta, d_indices, idx_dtype, d_weights, w_dtype, N, T, E,
                                 row_bytes, d_workspace, row_ptr, false, nullptr, s,
                                 "fmoe_build_plan");
}

extern "C" int fmoe_build_metadata_and_plan(
    const int64_t* host_ptrs, const int64_t* host_rows, int64_t num_experts, int64_t* d_ptr_table,
    int32_t* d_chunk_sizes, int64_t* d_offsets, int32_t* d_max_rows, const void* d_indices,
    int idx_dtype, const void* d_weights, int w_dtype, int64_t num_tokens, int64_t row_bytes,
    void* d_workspace, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const int64_t E = num_experts, T = num_tokens;
  FMOE_REQUIRE(E >= 1 && E < (int64_t(1) << 30),
               "fmoe_build_metadata_and_plan: num_experts must be in [1, 2^30) (got %lld)",
               (long long)E);
  FMOE_REQUIRE(host_ptrs && host_rows, "fmoe_build_metadata_and_plan: null host table");
  int64_t N = 0;
  for (int64_t e = 0; e < E; ++e) {
    if (host_rows[e] < 0 || host_rows[e] >= (int64_t(1) << 31)) break;  // reported below
    N += host_rows[e];
  }
  const bool small_table = E <= kMetaChunk;
  int64_t groups = 0, bins = 0;
  const bool sizes_ok = T >= 1 && T < (int64_t(1) << 30) && N < (int64_t(1) << 31);
  const PlanPath path = sizes_ok ? pick_plan(N, T, E, &groups, &bins) : kPathRadix;
  if (!small_table || path == kPathRadix) {
    // the two calls (each validates its own arguments)
    if (int rc = fmoe_build_metadata(host_ptrs, host_rows, E, d_ptr_table, d_chunk_sizes,
                                     d_offsets, d_max_rows, stream))
      return rc;
    return fmoe_build_plan(d_indices, idx_dtype, d_weights, w_dtype, N, T, d_ptr_table, d_offsets,
                           E, row_bytes, d_workspace, stream);
  }
  // one call (the metadata written by the plan's own kernels): the checks of fmoe_build_metadata
  // and fmoe_build_plan
  for (int64_t e = 0; e < E; ++e) {
    FMOE_REQUIRE(host_rows[e] >= 0 && host_rows[e] < (int64_t(1) << 31),
                 "fmoe_build_metadata_and_plan: expert %lld has invalid row count %lld",
                 (long long)e, (long long)host_rows[e]);
    FMOE_REQUIRE(host_rows[e] == 0 || host_ptrs[e] != 0,
                 "fmoe_build_metadata_and_plan: expert %lld has rows but a null address",
                 (long long)e);
  }
  FMOE_REQUIRE(d_ptr_table && d_chunk_sizes && d_offsets && d_max_rows && d_workspace,
               "fmoe_build_metadata_and_plan: null device output");
  FMOE_REQUIRE(N == 0 || (d_indices && d_weights),
               "fmoe_build_metadata_and_plan: null indices/weights");
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype),
               "fmoe_build_metadata_and_plan: bad index dtype %d", idx_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "fmoe_build_metadata_and_plan: bad weight dtype %d",
               w_dtype);
  FMOE_REQUIRE(((uintptr_t)d_workspace & 255) == 0,
               "fmoe_build_metadata_and_plan: workspace not 256B-aligned");
  FMOE_REQUIRE(row_bytes > 0, "fmoe_build_metadata_and_plan: row_bytes must be > 0");
  TokMetaArgs meta;
  fill_host_table(&meta, host_ptrs, host_rows, E, d_ptr_table, d_chunk_sizes, d_offsets,
                  d_max_rows);
  if (path == kPathRanged)
    return launch_plan_ranged(meta, d_indices, idx_dtype, d_weights, w_dtype, N, T, E, row_bytes,
                              d_workspace, static_cast<hipStream_t>(stream));
  if (path == kPathBucketed)
    return fmoe_plan::launch_bucketed(nullptr, &meta, d_indices, idx_dtype, d_weights, w_dtype, N,
                                      T, E, row_bytes, d_workspace, false, nullptr, nullptr,
                                      static_cast<hipStream_t>(stream),
                                      "fmoe_build_metadata_and_plan");
  const PlanLayout L = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  return launch_plan_tok(meta, d_indices, idx_dtype, d_weights, w_dtype, N, T, E, row_bytes,
                         groups, bins, reinterpret_cast<int32_t*>(ws + L.row_ptr),
                         reinterpret_cast<Rec*>(ws + L.rec),
                         reinterpret_cast<int32_t*>(ws + L.status), static_cast<hipStream_t>(stream));
}

namespace {

// Checks of the slot-map plan's arguments (the expert table's pointers are checked by callers).
int check_slots_args(const char* who, const int32_t* d_slot_pos, int64_t T, int64_t K,
                     const void* d_weights, int w_dtype, int64_t E, int64_t N, int64_t row_bytes,
                     void* d_workspace) {
  using namespace fmoe;
  FMOE_REQUIRE(T >= 1 && K >= 1 && K <= kWave, "%s: need T >= 1 and 1 <= top_k <= %d (T=%lld k=%lld)",
               who, kWave, (long long)T, (long long)K);
  FMOE_REQUIRE(E >= 1 && E <= kLdsExperts, "%s: num_experts not in [1, %d]", who, kLdsExperts);
  if (T >= (int64_t(1) << 30) || T * K >= (int64_t(1) << 31)) {
    fmoe_host::set_error("%s: T*k exceeds the 32-bit row counters", who);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(N == T * K,
               "%s: every slot must be a row of the combine (rows %lld != T*k %lld); build the plan "
               "from the scatter index instead",
               who, (long long)N, (long long)(T * K));
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "%s: bad weight dtype %d", who, w_dtype);
  FMOE_REQUIRE(d_slot_pos && d_weights && d_workspace, "%s: null device pointer", who);
  FMOE_REQUIRE(((uintptr_t)d_workspace & 255) == 0, "%s: workspace not 256B-aligned", who);
  FMOE_REQUIRE(row_bytes > 0, "%s: row_bytes must be > 0", who);
  return FMOE_OK;
}

template <typename Meta>
int launch_from_slots(const Meta& meta, const int32_t* d_slot_pos, int64_t T, int64_t K,
                      const void* d_weights, int w_dtype, int64_t E, int64_t N, int64_t row_bytes,
                      void* d_workspace, hipStream_t s, const char* who) {
  using namespace fmoe;
  const PlanLayout L = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* status = reinterpret_cast<int32_t*>(ws + L.status);
  int32_t* row_ptr = reinterpret_cast<int32_t*>(ws + L.row_ptr);
  Rec* rec = reinterpret_cast<Rec*>(ws + L.rec);
  const int64_t threads = std::max<int64_t>(N, T + 2);
  const dim3 grid((unsigned)((threads + kGroup - 1) / kGroup));
#define FMOE_FROM_SLOTS(TW)                                                                        \
  hipLaunchKernelGGL((k_plan_from_slots<TW, Meta>), grid, dim3(kGroup), 0, s, d_slot_pos, T, K,    \
                     static_cast<const TW*>(d_weights), meta, E, row_bytes, row_ptr, rec, status)
  if (w_dtype == FMOE_F32) FMOE_FROM_SLOTS(float);
  else if (w_dtype == FMOE_BF16) FMOE_FROM_SLOTS(bf16_t);
  else FMOE_FROM_SLOTS(f16_t);
#undef FMOE_FROM_SLOTS
  return fmoe_host::check_launch(who);
}

}  // namespace

extern "C" int fmoe_build_plan_from_slots(const int32_t* d_slot_pos, int64_t num_tokens,
                                          int64_t top_k, const void* d_weights, int w_dtype,
                                          const int64_t* d_ptr_table, const int64_t* d_offsets,
                                          int64_t num_experts, int64_t num_rows,
                                          int64_t row_bytes, void* d_workspace, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const char* who = "fmoe_build_plan_from_slots";
  if (int rc = check_slots_args(who, d_slot_pos, num_tokens, top_k, d_weights, w_dtype,
                                num_experts, num_rows, row_bytes, d_workspace))
    return rc;
  FMOE_REQUIRE(d_ptr_table && d_offsets, "%s: null device pointer", who);
  const TokMetaGlobal meta{d_ptr_table, d_offsets};
  return launch_from_slots(meta, d_slot_pos, num_tokens, top_k, d_weights, w_dtype, num_experts,
                           num_rows, row_bytes, d_workspace, static_cast<hipStream_t>(stream), who);
}

extern "C" int fmoe_build_metadata_and_plan_from_slots(
    const int64_t* host_ptrs, const int64_t* host_rows, int64_t num_experts, int64_t* d_ptr_table,
    int32_t* d_chunk_sizes, int64_t* d_offsets, int32_t* d_max_rows, const int32_t* d_slot_pos,
    int64_t num_tokens, int64_t top_k, const void* d_weights, int w_dtype, int64_t row_bytes,
    void* d_workspace, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const char* who = "fmoe_build_metadata_and_plan_from_slots";
  const int64_t E = num_experts;
  FMOE_REQUIRE(E >= 1 && E < (int64_t(1) << 30), "%s: num_experts must be in [1, 2^30) (got %lld)",
               who, (long long)E);
  FMOE_REQUIRE(host_ptrs && host_rows, "%s: null host table", who);
  int64_t N = 0;
  for (int64_t e = 0; e < E; ++e) {
    if (host_rows[e] < 0 || host_rows[e] >= (int64_t(1) << 31)) break;  // reported below
    N += host_rows[e];
  }
  if (E > kMetaChunk) {  // the two calls (each validates its own arguments)
    if (int rc = fmoe_build_metadata(host_ptrs, host_rows, E, d_ptr_table, d_chunk_sizes,
                                     d_offsets, d_max_rows, stream))
      return rc;
    return fmoe_build_plan_from_slots(d_slot_pos, num_tokens, top_k, d_weights, w_dtype,
                                      d_ptr_table, d_offsets, E, N, row_bytes, d_workspace,
                                      stream);
  }
  for (int64_t e = 0; e < E; ++e) {
    FMOE_REQUIRE(host_rows[e] >= 0 && host_rows[e] < (int64_t(1) << 31),
                 "%s: expert %lld has invalid row count %lld", who, (long long)e,
                 (long long)host_rows[e]);
    FMOE_REQUIRE(host_rows[e] == 0 || host_ptrs[e] != 0,
                 "%s: expert %lld has rows but a null address", who, (long long)e);
  }
  FMOE_REQUIRE(d_ptr_table && d_chunk_sizes && d_offsets && d_max_rows,
               "%s: null device output", who);
  if (int rc = check_slots_args(who, d_slot_pos, num_tokens, top_k, d_weights, w_dtype, E, N,
                                row_bytes, d_workspace))
    return rc;
  TokMetaArgs meta;
  fill_host_table(&meta, host_ptrs, host_rows, E, d_ptr_table, d_chunk_sizes, d_offsets,
                  d_max_rows);
  return launch_from_slots(meta, d_slot_pos, num_tokens, top_k, d_weights, w_dtype, E, N,
                           row_bytes, d_workspace, static_cast<hipStream_t>(stream), who);
}

extern "C" int fmoe_invert_scatter_index(const void* d_indices, int idx_dtype, int64_t num_rows,
                                         int64_t num_tokens, int32_t* d_row_ptr, int32_t* d_rows,
                                         void* d_workspace, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const int64_t N = num_rows, T = num_tokens;
  FMOE_REQUIRE(N >= 0, "fmoe_invert_scatter_index: num_rows must be >= 0");
  FMOE_REQUIRE(T >= 1, "fmoe_invert_scatter_index: num_tokens must be >= 1");
  if (N >= (int64_t(1) << 31) || T >= (int64_t(1) << 30)) {
    fmoe_host::set_error("fmoe_invert_scatter_index: N=%lld / T=%lld exceed the 32-bit row counters",
                         (long long)N, (long long)T);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype), "fmoe_invert_scatter_index: bad index dtype %d",
               idx_dtype);
  FMOE_REQUIRE(d_row_ptr && d_workspace, "fmoe_invert_scatter_index: null device pointer");
  FMOE_REQUIRE(N == 0 || (d_indices && d_rows), "fmoe_invert_scatter_index: null indices/rows");
  FMOE_REQUIRE(((uintptr_t)d_workspace & 255) == 0,
               "fmoe_invert_scatter_index: workspace not 256B-aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the radix plan, or the bucketed plan when asked for (option plan=2) and within its limits
  const int64_t algo = fmoe_host::opt(fmoe_host::kOptPlan);
  const bool bucketed = plan_geom(N, T).ok;
  if (bucketed && algo == 2)
    return fmoe_plan::launch_bucketed(nullptr, nullptr, d_indices, idx_dtype, nullptr, FMOE_F32, N,
                                      T, 0, 0, d_workspace, true, d_rows, d_row_ptr, s,
                                      "fmoe_invert_scatter_index");
  return fmoe_plan::launch_radix(nullptr, d_indices, idx_dtype, nullptr, FMOE_F32, N, T, 0, 0,
                                 d_workspace, d_row_ptr, true, d_rows, s,
                                 "fmoe_invert_scatter_index");
}
