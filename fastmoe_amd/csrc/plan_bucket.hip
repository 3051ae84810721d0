// Bucketed plan: the token-major inverse of the scatter index in two launches, linear in N + T,
// every segment in ascending packed-row order g.
//
//   k_plan_part    one 1024-thread workgroup per slice of S rows.  Each wave owns S/16 consecutive
//                  rows; it counts them per bucket (2^shift consecutive token bins), the workgroup
//                  scans the counts bucket-major, and each wave then writes its rows (g, bin) to
//                  the slice's bucket-major partition -- a lane's place is its bucket's cursor plus
//                  the number of lower lanes with the same bucket (ballot match), so rows of one
//                  bucket keep ascending g.  Per slice and bucket it writes the row count and the
//                  rows of lower buckets (bcnt, bpre).
//   k_plan_bucket  one wave per bucket.  Its rows are, slice after slice, part[s*S + bpre[s][b] ..],
//                  again in ascending g.  The wave counts them per token bin in LDS, scans the bins
//                  into row_ptr (its first row is sum_s bpre[s][b]), and writes each row's record
//                  at its bin's cursor plus its rank among the lower lanes of the same bin.
//
// No workgroup waits for another, nothing needs zero-filled memory, and every row is read a
// constant number of times, so a segment of any length (a scatter index sending every row to one
// token) costs time linear in its rows.  Both kernels are deterministic: the plan's bytes depend
// only on the inputs.
#include "plan.h"

namespace fmoe {

constexpr int kPartCache = 8;  // chunks of 64 rows a k_plan_part wave keeps in registers
constexpr int kBucketWaves = 4;
constexpr int kBucketThreads = kBucketWaves * kWave;
constexpr int kBucketCache = 8;      // chunks of 64 rows a k_plan_bucket wave keeps in registers
constexpr int kLdsMetaExperts = 4096;  // expert tables staged in LDS up to this many experts
static_assert(kPartThreads == kScanThreads, "k_plan_part scans with the 1024-thread block scan");

__device__ __forceinline__ int wave_incl_scan(int v) { return wave_incl_sum(v); }
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v = max(v, __shfl_xor(v, d, kWave));
  return v;
}

// Token bin of row g: its scatter index if in [0, T), else T.
template <typename TI>
__device__ __forceinline__ int bin_of(const TI* __restrict__ idx, int64_t g, int64_t T) {
  const int64_t t = (int64_t)idx[g];
  return (uint64_t)t < (uint64_t)T ? (int)t : (int)T;
}

template <typename TI>
__global__ __launch_bounds__(kPartThreads) void k_plan_part(
    const TI* __restrict__ idx, int64_t N, int64_t T, int64_t S, int shift, int nbk,
    int2* __restrict__ part, int32_t* __restrict__ bcnt, int32_t* __restrict__ bpre,
    int32_t* __restrict__ status) {
  __shared__ int cnt[kPartWaves * kMaxBuckets];  // [wave][bucket]: counts, then cursors
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  for (int i = threadIdx.x; i < kPartWaves * nbk; i += kPartThreads) cnt[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) status[kStatusLongest] = 0;  // k_plan_bucket maxes in
  __syncthreads();
  const int64_t s0 = (int64_t)blockIdx.x * S;
  const int64_t per = S / kPartWaves;  // a multiple of 64
  const int64_t w0 = s0 + (int64_t)wave * per;
  const int64_t w1 = min(N, w0 + per);
  const int nch = w1 > w0 ? (int)((w1 - w0 + kWave - 1) / kWave) : 0;  // wave-uniform
  int* my = cnt + wave * nbk;

  // 1. rows of this wave per bucket (bins of the first chunks kept for step 3)
  int keep[kPartCache];
#pragma unroll
  for (int i = 0; i < kPartCache; ++i) keep[i] = -1;
  for (int c0 = 0; c0 < nch; c0 += kPartCache) {
    int b[kPartCache];
#pragma unroll
    for (int i = 0; i < kPartCache; ++i) {
      const int64_t g = w0 + (int64_t)(c0 + i) * kWave + lane;
      b[i] = g < w1 ? bin_of(idx, g, T) : -1;
    }
#pragma unroll
    for (int i = 0; i < kPartCache; ++i)
      if (b[i] >= 0) atomicAdd(&my[b[i] >> shift], 1);
    if (c0 == 0) {
#pragma unroll
      for (int i = 0; i < kPartCache; ++i) keep[i] = b[i];
    }
  }
  __syncthreads();

  // 2. thread i owns bucket i: the slice's rows in it, the slice's rows in lower buckets, and each
  //    wave's first place in it (the cursors)
  const int bi = threadIdx.x;
  int tot = 0;
  if (bi < nbk)
    for (int w = 0; w < kPartWaves; ++w) tot += cnt[w * nbk + bi];
  int all;
  const int pre = block_exclusive_scan_1024(tot, &all);
  if (bi < nbk) {
    int run = pre;
    for (int w = 0; w < kPartWaves; ++w) {
      const int c = cnt[w * nbk + bi];
      cnt[w * nbk + bi] = run;
      run += c;
    }
    bcnt[(int64_t)blockIdx.x * nbk + bi] = tot;
    bpre[(int64_t)blockIdx.x * nbk + bi] = pre;
  }
  __syncthreads();

  // 3. each row at its bucket's cursor plus its rank among the lower lanes of the same bucket
  const int bits = nbk > 1 ? 32 - __builtin_clz((unsigned)(nbk - 1)) : 0;
  for (int c0 = 0; c0 < nch; c0 += kPartCache) {
    int b[kPartCache];
    if (c0 == 0) {
#pragma unroll
      for (int i = 0; i < kPartCache; ++i) b[i] = keep[i];
    } else {
#pragma unroll
      for (int i = 0; i < kPartCache; ++i) {
        const int64_t g = w0 + (int64_t)(c0 + i) * kWave + lane;
        b[i] = g < w1 ? bin_of(idx, g, T) : -1;
      }
    }
#pragma unroll
    for (int i = 0; i < kPartCache; ++i) {
      const bool act = b[i] >= 0;
      const int key = act ? (b[i] >> shift) : 0;
      const uint64_t m = match_key(act, key, bits);
      if (act) {
        const int rank = lanes_below(m);
        const int at = my[key];
        const int64_t g = w0 + (int64_t)(c0 + i) * kWave + lane;
        part[s0 + at + rank] = make_int2((int)g, b[i]);
        if (rank == 0) my[key] = at + __popcll(m);
      }
    }
  }
}

// ---- k_plan_bucket: where the records' source addresses come from --------------------------------
__device__ __forceinline__ void bucket_load_meta(const TokMetaGlobal& m, int E, int* off32,
                                                 uint64_t* ptr_lds) {
  for (int i = threadIdx.x; i <= E; i += kBucketThreads) {
    off32[i] = (int)m.offsets[i];
    if (i < E) ptr_lds[i] = (uint64_t)m.ptr_table[i];
  }
}
// Workgroup 0 also writes the metadata outputs (those of fmoe_build_metadata).
__device__ __forceinline__ void bucket_load_meta(const TokMetaArgs& m, int E, int* off32,
                                                 uint64_t* ptr_lds) {
  for (int i = threadIdx.x; i <= E; i += kBucketThreads) {
    off32[i] = m.a.off[i];
    if (i < E) ptr_lds[i] = (uint64_t)m.a.ptr[i];
    if (blockIdx.x == 0) {  // workgroup-uniform
      if (i < E) {
        m.ptr_table[i] = m.a.ptr[i];
        m.chunk_sizes[i] = m.a.off[i + 1] - m.a.off[i];
      }
      m.offsets[i] = m.a.off[i];
      if (i == 0) *m.max_rows = m.a.max_rows;
    }
  }
}

// Expert of row g and its base address; from LDS when the table fits, else from the device arrays
// (TokMetaGlobal only: the argument table never exceeds kMetaChunk experts).
__device__ __forceinline__ void expert_lookup(const TokMetaGlobal& m, bool lds, const int* off32,
                                              const uint64_t* ptr_lds, int E, int g,
                                              uint64_t* base, int* first) {
  if (lds) {
    const int e = expert_of_row32(off32, E, g);
    *base = ptr_lds[e];
    *first = off32[e];
  } else {
    const int64_t e = expert_of_row(m.offsets, E, g);
    *base = (uint64_t)m.ptr_table[e];
    *first = (int)m.offsets[e];
  }
}
__device__ __forceinline__ void expert_lookup(const TokMetaArgs&, bool, const int* off32,
                                              const uint64_t* ptr_lds, int E, int g,
                                              uint64_t* base, int* first) {
  const int e = expert_of_row32(off32, E, g);
  *base = ptr_lds[e];
  *first = off32[e];
}
// A source row is misaligned iff its expert's base is, or the expert has two or more rows and the
// row length is not a multiple of 16 bytes.
__device__ __forceinline__ bool expert_misaligned(const TokMetaGlobal& m, bool lds,
                                                  const int* off32, const uint64_t* ptr_lds,
                                                  int e, int64_t row_bytes) {
  const int64_t n = lds ? off32[e + 1] - off32[e] : m.offsets[e + 1] - m.offsets[e];
  const uint64_t p = lds ? ptr_lds[e] : (uint64_t)m.ptr_table[e];
  return n > 0 && ((p & 15) || (n > 1 && (row_bytes & 15)));
}
__device__ __forceinline__ bool expert_misaligned(const TokMetaArgs&, bool, const int* off32,
                                                  const uint64_t* ptr_lds, int e,
                                                  int64_t row_bytes) {
  const int n = off32[e + 1] - off32[e];
  return n > 0 && ((ptr_lds[e] & 15) || (n > 1 && (row_bytes & 15)));
}

template <typename TW, typename Meta, bool BARE>
__global__ __launch_bounds__(kBucketThreads) void k_plan_bucket(
    const int2* __restrict__ part, const int32_t* __restrict__ bcnt,
    const int32_t* __restrict__ bpre, int G1, int64_t S, int64_t T, int shift, int nbk,
    const TW* __restrict__ w, const Meta meta, int E, int64_t row_bytes,
    int32_t* __restrict__ row_ptr, Rec* __restrict__ rec, int32_t* __restrict__ rows,
    int32_t* __restrict__ status) {
  __shared__ int cnt[kBucketWaves][kMaxBucketBins];      // per bin: count, then cursor
  __shared__ int sl_first[kBucketWaves][kMaxSlices + 1]; // bucket rows before slice s
  __shared__ int sl_at[kBucketWaves][kMaxSlices];        // partition index of slice s's first
  __shared__ int off32[BARE ? 1 : kLdsMetaExperts + 1];
  __shared__ uint64_t ptr_lds[BARE ? 1 : kLdsMetaExperts];
  __shared__ int misaligned;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const bool lds_meta = !BARE && E <= kLdsMetaExperts;
  if constexpr (!BARE) {
    if (threadIdx.x == 0) misaligned = 0;
    if (lds_meta) bucket_load_meta(meta, E, off32, ptr_lds);
    __syncthreads();
    if (blockIdx.x == 0) {  // workgroup-uniform
      bool mis = false;
      for (int e = threadIdx.x; e < E; e += kBucketThreads)
        mis = mis || expert_misaligned(meta, lds_meta, off32, ptr_lds, e, row_bytes);
      if (mis) misaligned = 1;
      __syncthreads();
      if (threadIdx.x == 0) status[kStatusMisaligned] = misaligned;
    }
  } else {
    if (blockIdx.x == 0 && threadIdx.x == 0) status[kStatusMisaligned] = 0;
  }
  const int bk = blockIdx.x * kBucketWaves + wave;
  if (bk >= nbk) return;  // no barrier follows
  const int nb = (int)T + 1;
  const int lo = bk << shift;
  const int hi = min(lo + (1 << shift), nb);
  const int nloc = hi - lo;
  int* c = cnt[wave];
  int* first = sl_first[wave];
  int* at = sl_at[wave];
  for (int j = lane; j < nloc; j += kWave) c[j] = 0;

  // slices: this bucket's rows in slice s are part[at[s] .. at[s] + count_s), ascending g
  int L = 0, base = 0;  // rows in this bucket; rows in lower buckets (its first place)
  for (int s0 = 0; s0 < G1; s0 += kWave) {
    const int s = s0 + lane;
    int cs = 0, ps = 0;
    if (s < G1) {
      cs = bcnt[(int64_t)s * nbk + bk];
      ps = bpre[(int64_t)s * nbk + bk];
    }
    const int incl = wave_incl_scan(cs);
    if (s < G1) {
      first[s] = L + incl - cs;
      at[s] = (int)((int64_t)s * S) + ps;
    }
    L += __shfl(incl, kWave - 1, kWave);
    base += wave_sum_i(ps);
  }
  if (lane == 0) first[G1] = L;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // list position p (0 <= p < L) -> (g, bin)
  auto load_chunks = [&](int c0, int2* v) {
#pragma unroll
    for (int i = 0; i < kBucketCache; ++i) {
      const int p = (c0 + i) * kWave + lane;
      if (p < L) {
        int a = 0, b = G1;  // largest slice with first[a] <= p (first[G1] = L > p)
        while (b - a > 1) {
          const int mid = (a + b) >> 1;
          if (first[mid] <= p) a = mid; else b = mid;
        }
        v[i] = part[at[a] + (p - first[a])];
      } else {
        v[i] = make_int2(-1, 0);
      }
    }
  };

  // pass A: rows per token bin
  const int nch = (L + kWave - 1) / kWave;
  int2 keep[kBucketCache];
  for (int c0 = 0; c0 < nch; c0 += kBucketCache) {
    int2 v[kBucketCache];
    load_chunks(c0, v);
#pragma unroll
    for (int i = 0; i < kBucketCache; ++i)
      if (v[i].x >= 0) atomicAdd(&c[v[i].y - lo], 1);
    if (c0 == 0) {
#pragma unroll
      for (int i = 0; i < kBucketCache; ++i) keep[i] = v[i];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // scan: lane owns `per` consecutive bins; bins become row_ptr entries and cursors
  const int per = (nloc + kWave - 1) / kWave;
  const int j0 = min(nloc, lane * per);
  const int j1 = min(nloc, j0 + per);
  int loc = 0, longest = 0;
  for (int j = j0; j < j1; ++j) {
    const int x = c[j];
    loc += x;
    if (lo + j < (int)T) longest = max(longest, x);
  }
  const int incl = wave_incl_scan(loc);
  int run = base + incl - loc;
  for (int j = j0; j < j1; ++j) {
    const int x = c[j];
    c[j] = run;
    row_ptr[lo + j] = run;
    if (lo + j == (int)T) status[kStatusInvalid] = x;
    run += x;
  }
  if (hi == nb && lane == kWave - 1) row_ptr[nb] = base + L;  // == N
  longest = wave_max_i(longest);
  if (lane == 0 && longest > 0) atomicMax(&status[kStatusLongest], longest);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // pass B: each row at its bin's cursor plus its rank among the lower lanes of the same bin
  for (int c0 = 0; c0 < nch; c0 += kBucketCache) {
    int2 v[kBucketCache];
    if (c0 == 0) {
#pragma unroll
      for (int i = 0; i < kBucketCache; ++i) v[i] = keep[i];
    } else {
      load_chunks(c0, v);
    }
    float wg[kBucketCache];
    if constexpr (!BARE) {
#pragma unroll
      for (int i = 0; i < kBucketCache; ++i) wg[i] = v[i].x >= 0 ? ld1(w + v[i].x) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kBucketCache; ++i) {
      const bool act = v[i].x >= 0;
      const int key = act ? v[i].y - lo : 0;
      const uint64_t m = match_key(act, key, shift);
      if (act) {
        const int rank = lanes_below(m);
        const int pos = c[key] + rank;
        if (rank == 0) c[key] = pos + __popcll(m);
        const int g = v[i].x;
        if constexpr (BARE) {
          rows[pos] = g;
        } else {
          uint64_t ebase;
          int efirst;
          expert_lookup(meta, lds_meta, off32, ptr_lds, E, g, &ebase, &efirst);
          Rec r;
          r.src = ebase + (uint64_t)((int64_t)(g - efirst) * row_bytes);
          r.w = wg[i];
          r.g = g;
          rec[pos] = r;
        }
      }
    }
  }
}

}  // namespace fmoe

namespace fmoe_plan {

using namespace fmoe;

template <typename TW, typename Meta, bool BARE>
static void launch_bucket_k(unsigned groups, hipStream_t s, const int2* part, const int32_t* bcnt,
                            const int32_t* bpre, const PlanGeom& g, int64_t T, const void* w,
                            const Meta& meta, int64_t E, int64_t row_bytes, int32_t* row_ptr,
                            Rec* rec, int32_t* rows, int32_t* status) {
  hipLaunchKernelGGL((k_plan_bucket<TW, Meta, BARE>), dim3(groups), dim3(kBucketThreads), 0, s,
                     part, bcnt, bpre, g.G1, g.S, T, g.shift, g.nbk, static_cast<const TW*>(w),
                     meta, (int)E, row_bytes, row_ptr, rec, rows, status);
}

template <typename Meta>
static void launch_bucket_w(int w_dtype, unsigned groups, hipStream_t s, const int2* part,
                            const int32_t* bcnt, const int32_t* bpre, const PlanGeom& g,
                            int64_t T, const void* w, const Meta& meta, int64_t E,
                            int64_t row_bytes, int32_t* row_ptr, Rec* rec, int32_t* status) {
  if (w_dtype == FMOE_F32)
    launch_bucket_k<float, Meta, false>(groups, s, part, bcnt, bpre, g, T, w, meta, E, row_bytes,
                                        row_ptr, rec, nullptr, status);
  else if (w_dtype == FMOE_BF16)
    launch_bucket_k<bf16_t, Meta, false>(groups, s, part, bcnt, bpre, g, T, w, meta, E,
                                         row_bytes, row_ptr, rec, nullptr, status);
  else
    launch_bucket_k<f16_t, Meta, false>(groups, s, part, bcnt, bpre, g, T, w, meta, E, row_bytes,
                                        row_ptr, rec, nullptr, status);
}

// The bucketed plan (k_plan_part, then k_plan_bucket) into the workspace d_workspace of
// plan_layout(N, T).  Records: exactly one of gmeta / ameta is given.  bare: the bare CSR instead
// (row numbers into d_rows_bare, which may be null when N == 0, and row_ptr into d_row_ptr_bare).
// The caller has checked plan_geom(N, T).ok and the arguments.
int launch_bucketed(const TokMetaGlobal* gmeta, const TokMetaArgs* ameta, const void* d_indices,
                    int idx_dtype, const void* d_weights, int w_dtype, int64_t N, int64_t T,
                    int64_t E, int64_t row_bytes, void* d_workspace, bool bare,
                    int32_t* d_rows_bare, int32_t* d_row_ptr_bare, hipStream_t s,
                    const char* who) {
  const PlanGeom g = plan_geom(N, T);
  const PlanLayout Lw = plan_layout(N, T);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* status = reinterpret_cast<int32_t*>(ws + Lw.status);
  int32_t* row_ptr = bare ? d_row_ptr_bare : reinterpret_cast<int32_t*>(ws + Lw.row_ptr);
  int2* part = reinterpret_cast<int2*>(ws + Lw.part);
  int32_t* bcnt = reinterpret_cast<int32_t*>(ws + Lw.bcnt);
  int32_t* bpre = reinterpret_cast<int32_t*>(ws + Lw.bpre);
  Rec* rec = reinterpret_cast<Rec*>(ws + Lw.rec);
  if (idx_dtype == FMOE_I64)
    hipLaunchKernelGGL(k_plan_part<int64_t>, dim3((unsigned)g.G1), dim3(kPartThreads), 0, s,
                       static_cast<const int64_t*>(d_indices), N, T, g.S, g.shift, g.nbk, part,
                       bcnt, bpre, status);
  else
    hipLaunchKernelGGL(k_plan_part<int32_t>, dim3((unsigned)g.G1), dim3(kPartThreads), 0, s,
                       static_cast<const int32_t*>(d_indices), N, T, g.S, g.shift, g.nbk, part,
                       bcnt, bpre, status);
  if (int rc = fmoe_host::check_launch(who)) return rc;
  const unsigned groups = (unsigned)((g.nbk + kBucketWaves - 1) / kBucketWaves);
  if (bare) {
    const TokMetaGlobal none{nullptr, nullptr};
    launch_bucket_k<float, TokMetaGlobal, true>(groups, s, part, bcnt, bpre, g, T, nullptr, none,
                                                0, 0, row_ptr, nullptr, d_rows_bare, status);
  } else if (ameta) {
    launch_bucket_w(w_dtype, groups, s, part, bcnt, bpre, g, T, d_weights, *ameta, E, row_bytes,
                    row_ptr, rec, status);
  } else if (gmeta) {
    launch_bucket_w(w_dtype, groups, s, part, bcnt, bpre, g, T, d_weights, *gmeta, E, row_bytes,
                    row_ptr, rec, status);
  } else {
    fmoe_host::set_error("%s: no expert table for the plan's records", who);
    return FMOE_EINVAL;
  }
  return fmoe_host::check_launch(who);
}

}  // namespace fmoe_plan
