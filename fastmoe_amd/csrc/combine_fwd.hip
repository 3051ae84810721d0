// Forward combine: out[idx[g], :] += w[g] * X_e[g - off[e], :]
//
// Replaces _launch_grouped_kernel + _grouped_weighted_scatter_add_kernel
// (src/fastmoe/kernels/ops.py:277-310, :57-194).  Three modes:
//
// DET (token-major).  A wave owns one (token, column chunk).  It walks the token's plan segment in
// ascending packed-row order (ordering a short segment in registers first), loads 16 bytes per
// lane per row straight from each expert's buffer
// (the record carries the row address), multiplies by the gate in fp32, adds into fp32 registers
// and writes the output chunk once.  Every output byte is written exactly once and every expert
// byte read exactly once, so HBM traffic equals the compulsory bytes; no zero-fill is needed and
// the result is bit-identical run to run (and, in fp32, to the CPU index_add_ path, which adds the
// rounded products in the same ascending order).
//
// ATOMIC (packed-row-major, the reference kernel's order).  A wave owns one (row g, column chunk):
// binary-searches g's expert in the offsets (ops.py:151-154 does offsets + program id instead),
// loads the row, scales it and adds it into out[idx[g]] with global_atomic_add_f32.  A 16-bit
// output is accumulated in an fp32 workspace (initialised from out, or zeroed) and converted once
// at the end, so it is the fp32 sum rounded once, like the deterministic mode's; only the order of
// the fp32 additions differs run to run.
//
// ATOMIC_PACKED.  As ATOMIC, but a 16-bit output takes gfx950's packed atomics
// (global_atomic_pk_add_bf16 / _f16) on element pairs directly: no workspace and half the atomic
// requests, but every add rounds to 16 bits (the reference kernel's behaviour with a bf16 output).
#include <algorithm>

#include "plan.h"

namespace fmoe {

// Tile of one wave unit: U 16-byte vectors per lane per row (64 * V * U columns) and batches of
// R rows, so R * U independent loads per lane are in flight before the first use.
template <typename TX, typename TO, int V, int U, int RB, bool AL>
__device__ __forceinline__ void fwd_det_body(const int32_t* __restrict__ row_ptr,
                                             const Rec* __restrict__ rec, TO* __restrict__ out,
                                             int64_t out_stride, uint32_t D, uint32_t t,
                                             uint32_t chunk, int accumulate) {
  using VX = Vec<TX, V>;
  using VO = Vec<TO, V>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  // The misaligned-row path (element loads) takes one row at a time so that it does not set the
  // register budget of the kernel.
  constexpr int R = AL ? RB : 1;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t col0 = chunk * CW + (uint32_t)lane * V;
  uint32_t xoff[U], ooff[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    xoff[u] = (col0 + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TX);
    ooff[u] = (col0 + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TO);
  }
  const uint32_t xrow_bytes = D * (uint32_t)sizeof(TX);
  const int beg = row_ptr[t];
  const int end = row_ptr[t + 1];
  const rsrc_t ro = make_rsrc(out + (int64_t)t * out_stride, D * (uint32_t)sizeof(TO));

  float acc[U][V];
  if (accumulate) {
    if (beg == end) return;  // nothing routed here: out keeps its contents
#pragma unroll
    for (int u = 0; u < U; ++u) VO::cvt(VO::ld(ro, ooff[u]), acc[u]);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) acc[u][v] = 0.f;
  }

  for (int jb = beg; jb < end; jb += kWave) {
    const int cnt = min(end - jb, kWave);
    LaneRecs lr;
    lr.load(rec, jb, cnt, lane);
    // A segment of up to 64 rows comes unordered from the plan: order it by g here.  Longer
    // segments are already in ascending g.
    if (end - beg <= kWave) lr.sort_by_row(cnt, lane);
    for (int i = 0; i < cnt; i += R) {
      // Batch of R rows.  The spare slots of a partial batch load through an empty range
      // (num_records 0): the hardware range check returns zeros without a memory request, so
      // every load is issued unconditionally and none is wasted.
      raw_t a[R][U];
      float wr[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int ir = min(i + r, cnt - 1);
        const rsrc_t rx = make_rsrc(lr.src(ir), i + r < cnt ? xrow_bytes : 0u);
        wr[r] = lr.w(ir);
#pragma unroll
        for (int u = 0; u < U; ++u) a[r][u] = load_x<TX, V, AL>(rx, xoff[u]);
      }
      // Adds in ascending row order (the order of the plan segment).
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (i + r < cnt) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float x[V];
            VX::cvt(a[r][u], x);
#pragma unroll
            for (int v = 0; v < V; ++v) acc[u][v] = acc[u][v] + x[v] * wr[r];
          }
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u)  // columns >= D: dropped by range check
    VO::template st<FMOE_OUT_CPOL>(ro, ooff[u], acc[u]);
}

template <typename TX, typename TO, int V, int U, int RB>
__global__ __launch_bounds__(kGroup) void k_fwd_det(const int32_t* __restrict__ status,
                                                    const int32_t* __restrict__ row_ptr,
                                                    const Rec* __restrict__ rec,
                                                    TO* __restrict__ out, int64_t out_stride,
                                                    uint32_t D, uint32_t T, uint32_t chunks,
                                                    int accumulate) {
  const bool al = !(V > 1 && status[kStatusMisaligned] != 0);
  const uint32_t units = T * chunks;
  // Wave units (token, column chunk); a grid smaller than units / 4 strides over them.
  for (uint32_t unit = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave);
       unit < units; unit += gridDim.x * kWavesPerGroup) {
    const uint32_t t = unit / chunks;
    const uint32_t chunk = unit - t * chunks;
    if (al)
      fwd_det_body<TX, TO, V, U, RB, true>(row_ptr, rec, out, out_stride, D, t, chunk, accumulate);
    else
      fwd_det_body<TX, TO, V, U, RB, false>(row_ptr, rec, out, out_stride, D, t, chunk,
                                            accumulate);
  }
}

// ---- small inputs: the deterministic forward without a plan --------------------------------
// For at most kSmallRows rows the plan is not worth its own launch.  Every workgroup stages the
// token id of each row in LDS (-1 for an index outside [0, T)); a wave owns one (token, column
// chunk) unit as in k_fwd_det and finds the token's rows by ballots over the staged ids in
// ascending row order, compacting them through a 128-entry window and taking them 64 at a time.
// Lanes look up their row's expert in an LDS copy of the argument table.  The rows are added in
// ascending g with k_fwd_det's arithmetic, so the result is the same, bit for bit.
static_assert(kMetaChunk == kGroup, "one expert per thread copies the argument table");
template <typename TX, typename TO, int V, int U, bool AL>
__global__ __launch_bounds__(kGroup) void k_fwd_small(const HostTable meta,
                                                      const void* __restrict__ idx, int idx_dtype,
                                                      const void* __restrict__ w, int w_dtype,
                                                      uint32_t N, uint32_t T, uint32_t D,
                                                      uint32_t chunks, TO* __restrict__ out,
                                                      int64_t out_stride, int accumulate,
                                                      int32_t* __restrict__ status) {
  using VX = Vec<TX, V>;
  using VO = Vec<TO, V>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  constexpr int R = AL ? 4 : 1;  // rows per batch of loads (one at a time for element loads)
  __shared__ int tok[kSmallRows];
  __shared__ int win[kWavesPerGroup][2 * kWave];
  __shared__ int off_lds[kMetaChunk + 1];
  __shared__ uint64_t ptr_lds[kMetaChunk];
  __shared__ int invalid;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  if (tid == 0) invalid = 0;
  small_table_to_lds(meta, off_lds, ptr_lds);
  __syncthreads();
  int bad = 0;
  for (uint32_t g = tid; g < N; g += kGroup) {
    const int64_t v = load_index(idx, idx_dtype, g);
    const bool ok = v >= 0 && v < (int64_t)T;
    tok[g] = ok ? (int)v : -1;
    bad += ok ? 0 : 1;
  }
  if (blockIdx.x == 0 && bad) atomicAdd(&invalid, bad);
  __syncthreads();
  if (blockIdx.x == 0 && tid == 0) status[kStatusInvalid] = invalid;

  const uint32_t xrow_bytes = D * (uint32_t)sizeof(TX);
  const int ne = meta.count;
  const uint32_t units = T * chunks;
  for (uint32_t unit = blockIdx.x * kWavesPerGroup + (uint32_t)wave; unit < units;
       unit += gridDim.x * kWavesPerGroup) {
    const uint32_t t = unit / chunks;
    const uint32_t chunk = unit - t * chunks;
    const uint32_t col0 = chunk * CW + (uint32_t)lane * V;
    uint32_t xoff[U], ooff[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xoff[u] = (col0 + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TX);
      ooff[u] = (col0 + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TO);
    }
    const rsrc_t ro = make_rsrc(out + (int64_t)t * out_stride, D * (uint32_t)sizeof(TO));
    float acc[U][V];
    if (accumulate) {
#pragma unroll
      for (int u = 0; u < U; ++u) VO::cvt(VO::ld(ro, ooff[u]), acc[u]);
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < V; ++v) acc[u][v] = 0.f;
    }
    int have = 0;  // rows in the window (wave-uniform)
    int seen = 0;
    for (uint32_t base = 0; base < N; base += kWave) {
      const uint32_t g = base + (uint32_t)lane;
      const bool hit = g < N && tok[g] == (int)t;
      const uint64_t m = __ballot(hit);
      if (hit) win[wave][have + lanes_below(m)] = (int)g;
      have += __builtin_popcountll(m);
      const bool last = base + kWave >= N;
      while (have >= kWave || (last && have > 0)) {
        const int cnt = have < kWave ? have : kWave;
        LaneRecs lr;
        lr.g = lane < cnt ? win[wave][lane] : 0;
        if (lane < cnt) {
          const int e = expert_of_row32(off_lds, ne, lr.g);
          const uint64_t src =
              ptr_lds[e] + (uint64_t)(uint32_t)(lr.g - off_lds[e]) * (uint64_t)xrow_bytes;
          lr.src_lo = (uint32_t)src;
          lr.src_hi = (uint32_t)(src >> 32);
          lr.w_bits = __float_as_uint(load_weight(w, w_dtype, lr.g));
        } else {
          lr.src_lo = lr.src_hi = lr.w_bits = 0;
        }
        const int rest = have - cnt;  // at most 63 rows carried to the window's front
        const int carry = lane < rest ? win[wave][cnt + lane] : 0;
        if (lane < rest) win[wave][lane] = carry;
        have = rest;
        seen += cnt;
        for (int i = 0; i < cnt; i += R) {
          raw_t a[R][U];
          float wr[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int ir = min(i + r, cnt - 1);
            const rsrc_t rx = make_rsrc(lr.src(ir), i + r < cnt ? xrow_bytes : 0u);
            wr[r] = lr.w(ir);
#pragma unroll
            for (int u = 0; u < U; ++u) a[r][u] = load_x<TX, V, AL>(rx, xoff[u]);
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (i + r < cnt) {
#pragma unroll
              for (int u = 0; u < U; ++u) {
                float x[V];
                VX::cvt(a[r][u], x);
#pragma unroll
                for (int v = 0; v < V; ++v) acc[u][v] = acc[u][v] + x[v] * wr[r];
              }
            }
          }
        }
      }
    }
    if (accumulate && seen == 0) continue;  // nothing routed here: out keeps its contents
#pragma unroll
    for (int u = 0; u < U; ++u)  // columns >= D: dropped by range check
      VO::template st<FMOE_OUT_CPOL>(ro, ooff[u], acc[u]);
  }
}

// ---- atomics ---------------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <typename TO, int V> struct AtomicVec;
template <int V> struct AtomicVec<float, V> {
  static __device__ __forceinline__ void add(float* p, const float* f) {
#pragma unroll
    for (int v = 0; v < V; ++v) unsafeAtomicAdd(p + v, f[v]);
  }
};
// 16-bit outputs: packed atomics on element pairs, so the vector path only (V even, rows and
// pairs 4-byte aligned); the host refuses atomic mode with a 16-bit output otherwise.
template <int V> struct AtomicVec<bf16_t, V> {
  static_assert(V % 2 == 0, "packed bf16 atomics need element pairs");
  static __device__ __forceinline__ void add(bf16_t* p, const float* f) {
#pragma unroll
    for (int v = 0; v < V; v += 2) {
      bf16x2_t x;
      x.x = (__bf16)f[v];
      x.y = (__bf16)f[v + 1];
      __builtin_amdgcn_global_atomic_fadd_v2bf16(reinterpret_cast<bf16x2_t*>(p + v), x);
    }
  }
};
template <int V> struct AtomicVec<f16_t, V> {
  static_assert(V % 2 == 0, "packed f16 atomics need element pairs");
  static __device__ __forceinline__ void add(f16_t* p, const float* f) {
#pragma unroll
    for (int v = 0; v < V; v += 2) {
      f16x2_t x;
      x.x = (_Float16)f[v];
      x.y = (_Float16)f[v + 1];
      __builtin_amdgcn_global_atomic_fadd_v2f16(reinterpret_cast<f16x2_t*>(p + v), x);
    }
  }
};

// Lane-interleaved row chunk: every access of the wave covers 64 * EPL consecutive columns (EPL =
// 1 for fp32 outputs, 2 for the packed 16-bit atomics), so the atomics of one instruction land on
// consecutive addresses -- two cache lines per instruction -- rather than on 16-byte lane strides
// spread over eight.  Device-scope float atomics are executed memory-side on MI355X (every L2
// atomic request is forwarded to the memory side), so the request count sets this kernel's speed.
// The chunk width (64 * V * U columns) is the one the host sized the grid with.
template <typename TX, typename TO, int V, int U, bool AL>
__device__ __forceinline__ void fwd_atomic_body(uint64_t src, float wf, TO* __restrict__ orow,
                                                uint32_t D, uint32_t chunk) {
  constexpr int EPL = sizeof(TO) == 4 ? 1 : 2;
  static_assert((V * U) % EPL == 0, "chunk must hold whole element pairs");
  constexpr int A = V * U / EPL;  // accesses per lane per chunk
  using VX = Vec<TX, EPL>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t col0 = chunk * CW + (uint32_t)lane * EPL;
  const rsrc_t rx = make_rsrc(src, D * (uint32_t)sizeof(TX));
  raw_t a[A];
#pragma unroll
  for (int i = 0; i < A; ++i)
    a[i] = load_x<TX, EPL, AL>(rx, (col0 + (uint32_t)i * kWave * EPL) * (uint32_t)sizeof(TX));
#pragma unroll
  for (int i = 0; i < A; ++i) {
    const uint32_t col = col0 + (uint32_t)i * kWave * EPL;
    float x[EPL];
    VX::cvt(a[i], x);
#pragma unroll
    for (int v = 0; v < EPL; ++v) x[v] = x[v] * wf;
    if (col < D) AtomicVec<TO, EPL>::add(orow + col, x);  // D is even for 16-bit outputs
  }
}

template <typename TX, typename TO, int V, int U>
__global__ __launch_bounds__(kGroup) void k_fwd_atomic(
    const int64_t* __restrict__ ptr_table, const int64_t* __restrict__ offsets, int64_t E,
    const void* __restrict__ idx, int idx_dtype, const void* __restrict__ w, int w_dtype,
    TO* __restrict__ out, int64_t out_stride, uint32_t D, uint32_t N, int64_t T, uint32_t chunks,
    int chunk_major) {
  constexpr int EPL = sizeof(TO) == 4 ? 1 : 2;
  const uint32_t unit = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave);
  uint32_t g, chunk;
  if (chunk_major) {  // every row's chunk 0, then every row's chunk 1, ...
    chunk = unit / N;
    if (chunk >= chunks) return;
    g = unit - chunk * N;
  } else {            // a row's chunks side by side
    g = unit / chunks;
    if (g >= N) return;
    chunk = unit - g * chunks;
  }
  const int64_t t = load_index(idx, idx_dtype, g);
  if (t < 0 || t >= T) return;  // out-of-range rows are dropped (the plan counts them)
  const int64_t e = expert_of_row(offsets, E, g);
  const uint64_t src =
      (uint64_t)ptr_table[e] + (uint64_t)((g - offsets[e]) * (int64_t)D) * sizeof(TX);
  const float wf = load_weight(w, w_dtype, g);
  TO* orow = out + t * out_stride;
  if (EPL > 1 && (src % (EPL * sizeof(TX))) != 0)
    fwd_atomic_body<TX, TO, V, U, false>(src, wf, orow, D, chunk);
  else
    fwd_atomic_body<TX, TO, V, U, true>(src, wf, orow, D, chunk);
}

// ---- fp32 accumulator of a 16-bit output, and zero-fill of an overwritten output --------------
// Row-major passes over [T, D]: a thread per 8 consecutive columns of a row, with 16-byte accesses
// when the rows allow them (VEC: D % 8 == 0 and 16-byte aligned rows), element accesses otherwise.
// The accumulator is a contiguous, 16-byte aligned fp32 [T, D] workspace.
constexpr int kAccCols = 8;

template <typename TO, bool VEC>
__global__ __launch_bounds__(kGroup) void k_acc_init(float* __restrict__ acc,
                                                     const TO* __restrict__ out, int64_t out_stride,
                                                     uint32_t D, uint32_t T, int accumulate) {
  const uint32_t groups = (D + kAccCols - 1) / kAccCols;
  const int64_t total = (int64_t)T * groups;
  for (int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kGroup) {
    const uint32_t t = (uint32_t)(i / groups);
    const uint32_t c = (uint32_t)(i - (int64_t)t * groups) * kAccCols;
    const TO* o = out + (int64_t)t * out_stride + c;
    float* a = acc + (int64_t)t * D + c;
    float f[kAccCols];
    if (!accumulate) {
#pragma unroll
      for (int k = 0; k < kAccCols; ++k) f[k] = 0.f;
    } else if constexpr (VEC) {
      Vec<TO, kAccCols>::cvt(*reinterpret_cast<const u32x4*>(o), f);
    } else {
#pragma unroll
      for (int k = 0; k < kAccCols; ++k) f[k] = c + k < D ? ld1(o + k) : 0.f;
    }
    if constexpr (VEC) {
      reinterpret_cast<u32x4*>(a)[0] = u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]),
                                             __float_as_uint(f[2]), __float_as_uint(f[3])};
      reinterpret_cast<u32x4*>(a)[1] = u32x4{__float_as_uint(f[4]), __float_as_uint(f[5]),
                                             __float_as_uint(f[6]), __float_as_uint(f[7])};
    } else {
#pragma unroll
      for (int k = 0; k < kAccCols; ++k)
        if (c + k < D) a[k] = f[k];
    }
  }
}

template <typename TO, bool VEC>
__global__ __launch_bounds__(kGroup) void k_acc_store(const float* __restrict__ acc,
                                                      TO* __restrict__ out, int64_t out_stride,
                                                      uint32_t D, uint32_t T) {
  const uint32_t groups = (D + kAccCols - 1) / kAccCols;
  const int64_t total = (int64_t)T * groups;
  for (int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kGroup) {
    const uint32_t t = (uint32_t)(i / groups);
    const uint32_t c = (uint32_t)(i - (int64_t)t * groups) * kAccCols;
    const float* a = acc + (int64_t)t * D + c;
    TO* o = out + (int64_t)t * out_stride + c;
    if constexpr (VEC) {
      const u32x4 lo = reinterpret_cast<const u32x4*>(a)[0];
      const u32x4 hi = reinterpret_cast<const u32x4*>(a)[1];
      const float f[kAccCols] = {__uint_as_float(lo.x), __uint_as_float(lo.y),
                                 __uint_as_float(lo.z), __uint_as_float(lo.w),
                                 __uint_as_float(hi.x), __uint_as_float(hi.y),
                                 __uint_as_float(hi.z), __uint_as_float(hi.w)};
      *reinterpret_cast<u32x4*>(o) = Vec<TO, kAccCols>::pack(f);
    } else {
#pragma unroll
      for (int k = 0; k < kAccCols; ++k)
        if (c + k < D) st1(o + k, a[k]);
    }
  }
}

// out[t, :] = 0 for every row (an atomic-mode call that overwrites out); 16-byte stores when
// the rows allow them (VEC, as in the accumulator passes).
template <typename TO, bool VEC>
__global__ __launch_bounds__(kGroup) void k_rows_zero(TO* __restrict__ out, int64_t out_stride,
                                                      uint32_t D, uint32_t T) {
  const uint32_t groups = (D + kAccCols - 1) / kAccCols;
  const int64_t total = (int64_t)T * groups;
  for (int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kGroup) {
    const uint32_t t = (uint32_t)(i / groups);
    const uint32_t c = (uint32_t)(i - (int64_t)t * groups) * kAccCols;
    TO* o = out + (int64_t)t * out_stride + c;
    if constexpr (VEC) {
      constexpr int kWords = kAccCols * (int)sizeof(TO) / 16;  // 16-byte words per 8 columns
#pragma unroll
      for (int k = 0; k < kWords; ++k) reinterpret_cast<u32x4*>(o)[k] = u32x4{0u, 0u, 0u, 0u};
    } else {
#pragma unroll
      for (int k = 0; k < kAccCols; ++k)
        if (c + k < D) st1(o + k, 0.f);
    }
  }
}

static unsigned row_pass_blocks(int64_t T, int64_t D) {
  const int64_t threads = T * ((D + kAccCols - 1) / kAccCols);
  return (unsigned)std::min<int64_t>((threads + kGroup - 1) / kGroup, int64_t(1) << 16);
}

template <typename TO>
static int launch_zero(void* out, int64_t stride, int64_t D, int64_t T, hipStream_t s) {
  const bool vec = D % kAccCols == 0 && (uintptr_t)out % 16 == 0 &&
                   (stride * (int64_t)sizeof(TO)) % 16 == 0;
  if (vec)
    hipLaunchKernelGGL((k_rows_zero<TO, true>), dim3(row_pass_blocks(T, D)), dim3(kGroup), 0, s,
                       static_cast<TO*>(out), stride, (uint32_t)D, (uint32_t)T);
  else
    hipLaunchKernelGGL((k_rows_zero<TO, false>), dim3(row_pass_blocks(T, D)), dim3(kGroup), 0, s,
                       static_cast<TO*>(out), stride, (uint32_t)D, (uint32_t)T);
  return fmoe_host::check_launch("fmoe_combine_fwd(zero out)");
}

static int zero_out(void* out, int out_dtype, int64_t stride, int64_t D, int64_t T,
                    hipStream_t s) {
  if (out_dtype == FMOE_F32) return launch_zero<float>(out, stride, D, T, s);
  if (out_dtype == FMOE_BF16) return launch_zero<bf16_t>(out, stride, D, T, s);
  return launch_zero<f16_t>(out, stride, D, T, s);
}

template <typename TO>
static int launch_acc_pass(bool init, float* acc, void* out, int64_t stride, int64_t D, int64_t T,
                           int accumulate, hipStream_t s) {
  const bool vec = D % kAccCols == 0 && (uintptr_t)out % 16 == 0 &&
                   (stride * (int64_t)sizeof(TO)) % 16 == 0;
  const dim3 grid(row_pass_blocks(T, D));
  if (init) {
    if (vec)
      hipLaunchKernelGGL((k_acc_init<TO, true>), grid, dim3(kGroup), 0, s, acc,
                         static_cast<const TO*>(out), stride, (uint32_t)D, (uint32_t)T, accumulate);
    else
      hipLaunchKernelGGL((k_acc_init<TO, false>), grid, dim3(kGroup), 0, s, acc,
                         static_cast<const TO*>(out), stride, (uint32_t)D, (uint32_t)T, accumulate);
  } else {
    if (vec)
      hipLaunchKernelGGL((k_acc_store<TO, true>), grid, dim3(kGroup), 0, s, acc,
                         static_cast<TO*>(out), stride, (uint32_t)D, (uint32_t)T);
    else
      hipLaunchKernelGGL((k_acc_store<TO, false>), grid, dim3(kGroup), 0, s, acc,
                         static_cast<TO*>(out), stride, (uint32_t)D, (uint32_t)T);
  }
  return fmoe_host::check_launch("fmoe_combine_fwd(fp32 accumulator)");
}

// ---- host dispatch ---------------------------------------------------------------------------
// Vectors per lane per row: several 16-byte loads in flight per row, and preferably a chunk
// width that divides D (no tail predication), while small D still spreads over many waves.
static int pick_u(int64_t D, int V) {
  const int forced = (int)fmoe_host::opt(fmoe_host::kOptFwdDetU);
  if (forced == 1 || forced == 2 || forced == 4) return forced;
  for (int u = 4; u >= 1; u >>= 1) {
    const int64_t cw = (int64_t)kWave * V * u;
    if (D % cw == 0 && D / cw >= (u == 1 ? 1 : 2)) return u;
  }
  if (D >= (int64_t)kWave * V * 4 * 2) return 4;
  if (D >= (int64_t)kWave * V * 2) return 2;
  return 1;
}

static int grid_for(int64_t units, const char* who, unsigned* blocks) {
  const int64_t b = (units + kWavesPerGroup - 1) / kWavesPerGroup;
  if (units >= (int64_t(1) << 32) - kWavesPerGroup || b >= (int64_t(1) << 31)) {
    fmoe_host::set_error("%s: grid too large (%lld wave units)", who, (long long)units);
    return FMOE_ERANGE;
  }
  *blocks = (unsigned)b;
  return FMOE_OK;
}

struct FwdArgs {
  int mode;
  const int32_t* status;
  const int32_t* row_ptr;
  const Rec* rec;
  const void* idx;
  int idx_dtype;
  const void* w;
  int w_dtype;
  const int64_t* ptr_table;
  const int64_t* offsets;
  int64_t E, N, T, D;
  void* out;
  int64_t out_stride;
  int accumulate;
  hipStream_t s;
};

template <typename TX, typename TO, int V, int U, int RB>
static int launch_fwd_k(const FwdArgs& a, int64_t chunks) {
  unsigned blocks;
  if (a.mode == FMOE_MODE_DET) {
    if (int rc = grid_for(a.T * chunks, "fmoe_combine_fwd(det)", &blocks)) return rc;
    const int persist = (int)fmoe_host::opt(fmoe_host::kOptFwdGrid);  // 0 = one wave per unit
    if (persist > 0 && (unsigned)persist < blocks) blocks = (unsigned)persist;
    hipLaunchKernelGGL((k_fwd_det<TX, TO, V, U, RB>), dim3(blocks), dim3(kGroup), 0, a.s, a.status,
                       a.row_ptr, a.rec, static_cast<TO*>(a.out), a.out_stride, (uint32_t)a.D,
                       (uint32_t)a.T, (uint32_t)chunks, a.accumulate);
    return fmoe_host::check_launch("fmoe_combine_fwd(det)");
  }
  if constexpr (V == 1 && sizeof(TO) == 2) {
    fmoe_host::set_error(
        "fmoe_combine_fwd(atomic_packed): a 16-bit output needs D %% %d == 0 and %d-byte aligned "
        "output rows (packed atomics on element pairs); use FMOE_MODE_ATOMIC or FMOE_MODE_DET",
        vec16<TX>(), vec16<TX>() * 2);
    return FMOE_EINVAL;
  } else {
    if (int rc = grid_for(a.N * chunks, "fmoe_combine_fwd(atomic)", &blocks)) return rc;
    // Column-chunk-major order keeps each pass over the rows on one column slice of the target.
    // Measured (rocprof, one MI355X, bf16 experts, fp32 accumulator): with a 2 GiB target
    // (T = 32768, D = 16384, top-2) the atomic kernel takes 3332 against 3381 us; with 256 MiB
    // targets (T = 4096, D = 16384, top-8; T = 8192, D = 4096, top-6) it is 1-1.5 % slower, so it
    // is the default from 1 GiB of target.
    const int order = (int)fmoe_host::opt(fmoe_host::kOptAtomicOrder);
    const bool big = a.T * a.D * (int64_t)sizeof(TO) >= (int64_t(1) << 30);
    const int chunk_major = (order == 2 || (order == 0 && big)) ? 1 : 0;
    hipLaunchKernelGGL((k_fwd_atomic<TX, TO, V, U>), dim3(blocks), dim3(kGroup), 0, a.s,
                       a.ptr_table, a.offsets, a.E, a.idx, a.idx_dtype, a.w, a.w_dtype,
                       static_cast<TO*>(a.out), a.out_stride, (uint32_t)a.D, (uint32_t)a.N, a.T,
                       (uint32_t)chunks, chunk_major);
    return fmoe_host::check_launch("fmoe_combine_fwd(atomic)");
  }
}

template <typename TX, typename TO, int V, int U, int RB>
static int launch_fwd_u(const FwdArgs& a) {
  const int64_t CW = (int64_t)kWave * V * U;
  const int64_t chunks = (a.D + CW - 1) / CW;
  return launch_fwd_k<TX, TO, V, U, RB>(a, chunks);
}

// Tile of the deterministic forward by the average rows per token r = N / T.  A batch issues its
// R x U loads whether or not its rows exist (the spare slots read an empty range: no traffic, but
// an issue slot each), so short segments take short batches: r <= 1.5 takes R = 2 (U = 4, with a
// partly empty last chunk if D needs it, when D holds one chunk of 4 vectors per lane), r <= 3
// takes R = 4.  Long segments (r >= 7) whose chunk
// would be 2 vectors per lane take 1 with R = 8.  Measured with HIP events on one MI355X, bf16,
// against the choice by D alone: T=16384, D=7168: k=1 129 -> 75 us, k=2 146 -> 109 us, k=8 355 ->
// 349 us (Zipf) and 361 -> 354 us (top-k); D=5120, 3072, 6144 at k=8 about 2 % faster; D=4096 and
// 16384 at k=2, 6 and 8 unchanged.
static void pick_det_tile(const FwdArgs& a, int V, int* U, int* R) {
  *U = pick_u(a.D, V);
  *R = *U >= 4 ? 4 : 8;
  if (fmoe_host::opt(fmoe_host::kOptFwdDetU) != 0 || a.N == 0) return;  // U forced: keep R by U
  if (2 * a.N <= 3 * a.T && a.D >= (int64_t)kWave * V * 4) {  // r <= 1.5, a whole chunk of 4
    *U = 4;
    *R = 2;
  } else if (a.N <= 3 * a.T) {                                  // r <= 3
    if (*U >= 2) *R = 4;
  } else if (a.N >= 7 * a.T && *U == 2) {                       // r >= 7
    *U = 1;
    *R = 8;
  }
}

// Tile shapes (U vectors per lane per row, R rows per batch).  The "fwd_tile" option <U><R> (e.g.
// 44) overrides the choice for tuning.
template <typename TX, typename TO, int V>
static int launch_fwd_v(const FwdArgs& a) {
  if constexpr (V == 1) {
    return launch_fwd_u<TX, TO, 1, 4, 4>(a);
  } else {
    const int tile = (int)fmoe_host::opt(a.mode == FMOE_MODE_DET ? fmoe_host::kOptFwdTile
                                                                 : fmoe_host::kOptFwdAtomicTile);
    int U = tile / 10, R = tile % 10;
    if (!((U == 4 && (R == 4 || R == 2)) || (U == 2 && (R == 8 || R == 4)) ||
          (U == 1 && R == 8))) {
      if (a.mode == FMOE_MODE_DET) {
        pick_det_tile(a, V, &U, &R);
      } else {
        U = pick_u(a.D, V);
        R = U >= 4 ? 4 : 8;
      }
    }
    if (U == 4 && R == 2) return launch_fwd_u<TX, TO, V, 4, 2>(a);
    if (U == 4) return launch_fwd_u<TX, TO, V, 4, 4>(a);
    if (U == 2 && R == 4) return launch_fwd_u<TX, TO, V, 2, 4>(a);
    if (U == 2) return launch_fwd_u<TX, TO, V, 2, 8>(a);
    return launch_fwd_u<TX, TO, V, 1, 8>(a);
  }
}

template <typename TX, typename TO>
static int launch_fwd_t(const FwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int ob = (int)sizeof(TO) == 4 ? 4 : 2;
  const int64_t vb = (int64_t)V * ob;  // bytes of one output vector
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.out % vb == 0) &&
                      ((a.out_stride * ob) % vb == 0) && fmoe_host::opt(fmoe_host::kOptForceScalar) == 0;
  if (vec_ok) return launch_fwd_v<TX, TO, V>(a);
  return launch_fwd_v<TX, TO, 1>(a);
}

template <typename TX>
static int launch_fwd_x(const FwdArgs& a, int out_dtype) {
  switch (out_dtype) {
    case FMOE_F32: return launch_fwd_t<TX, float>(a);
    case FMOE_BF16: return launch_fwd_t<TX, bf16_t>(a);
    case FMOE_F16: return launch_fwd_t<TX, f16_t>(a);
  }
  fmoe_host::set_error("fmoe_combine_fwd: bad out dtype %d", out_dtype);
  return FMOE_EINVAL;
}


// The small path: a grid of at most kSmallGroups workgroups strides over the (token, chunk) units,
// so that the ids are staged at most that many times.
constexpr unsigned kSmallGroups = 1024;

struct SmallFwdArgs {
  HostTable meta;
  const void* idx;
  int idx_dtype;
  const void* w;
  int w_dtype;
  int64_t N, T, D;
  void* out;
  int64_t out_stride;
  int accumulate;
  int32_t* status;
  bool aligned;
  hipStream_t s;
};

template <typename TX, typename TO, int V, int U, bool AL>
static int launch_small_k(const SmallFwdArgs& a) {
  const int64_t CW = (int64_t)kWave * V * U;
  const int64_t chunks = (a.D + CW - 1) / CW;
  unsigned blocks;
  if (int rc = grid_for(a.T * chunks, "fmoe_combine_fwd_small", &blocks)) return rc;
  blocks = std::min(blocks, kSmallGroups);
  hipLaunchKernelGGL((k_fwd_small<TX, TO, V, U, AL>), dim3(blocks), dim3(kGroup), 0, a.s, a.meta,
                     a.idx, a.idx_dtype, a.w, a.w_dtype, (uint32_t)a.N, (uint32_t)a.T,
                     (uint32_t)a.D, (uint32_t)chunks, static_cast<TO*>(a.out), a.out_stride,
                     a.accumulate, a.status);
  return fmoe_host::check_launch("fmoe_combine_fwd_small");
}

// 16-byte vectors when the output layout allows them (as launch_fwd_t), U by D (pick_u); rows
// that are not 16-byte aligned take element loads one vector per lane.
template <typename TX, typename TO>
static int launch_small_t(const SmallFwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int ob = (int)sizeof(TO) == 4 ? 4 : 2;
  const int64_t vb = (int64_t)V * ob;
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.out % vb == 0) &&
                      ((a.out_stride * ob) % vb == 0) &&
                      fmoe_host::opt(fmoe_host::kOptForceScalar) == 0;
  if (!vec_ok) return launch_small_k<TX, TO, 1, 4, true>(a);
  if (!a.aligned) return launch_small_k<TX, TO, V, 1, false>(a);
  const int U = pick_u(a.D, V);
  if (U == 4) return launch_small_k<TX, TO, V, 4, true>(a);
  if (U == 2) return launch_small_k<TX, TO, V, 2, true>(a);
  return launch_small_k<TX, TO, V, 1, true>(a);
}

template <typename TX>
static int launch_small_x(const SmallFwdArgs& a, int out_dtype) {
  switch (out_dtype) {
    case FMOE_F32: return launch_small_t<TX, float>(a);
    case FMOE_BF16: return launch_small_t<TX, bf16_t>(a);
    case FMOE_F16: return launch_small_t<TX, f16_t>(a);
  }
  fmoe_host::set_error("fmoe_combine_fwd_small: bad out dtype %d", out_dtype);
  return FMOE_EINVAL;
}

}  // namespace fmoe

extern "C" int64_t fmoe_combine_fwd_workspace_bytes(int mode, int64_t num_tokens, int64_t hidden,
                                                    int out_dtype) {
  if (num_tokens < 1 || hidden < 1) return -1;
  if (mode == FMOE_MODE_ATOMIC && (out_dtype == FMOE_BF16 || out_dtype == FMOE_F16))
    return fmoe_host::round_up(num_tokens * hidden * 4, 256);
  return 0;
}

extern "C" int fmoe_combine_fwd(int mode, const void* d_plan, const void* d_indices, int idx_dtype,
                                const void* d_weights, int w_dtype, const int64_t* d_ptr_table,
                                const int64_t* d_offsets, int64_t num_experts, int64_t num_rows,
                                int64_t num_tokens, int64_t hidden, int x_dtype, void* d_out,
                                int out_dtype, int64_t out_row_stride, int accumulate,
                                void* d_workspace, int64_t workspace_bytes, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  FMOE_REQUIRE(mode == FMOE_MODE_DET || mode == FMOE_MODE_ATOMIC || mode == FMOE_MODE_ATOMIC_PACKED,
               "fmoe_combine_fwd: bad mode %d", mode);
  FMOE_REQUIRE(num_rows >= 0 && num_tokens >= 1 && hidden >= 1,
               "fmoe_combine_fwd: bad sizes N=%lld T=%lld D=%lld", (long long)num_rows,
               (long long)num_tokens, (long long)hidden);
  if (num_rows >= (int64_t(1) << 31) || num_tokens >= (int64_t(1) << 30)) {
    fmoe_host::set_error("fmoe_combine_fwd: N/T exceed the 32-bit row counters");
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_float_dtype(x_dtype), "fmoe_combine_fwd: bad x dtype %d", x_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(out_dtype), "fmoe_combine_fwd: bad out dtype %d",
               out_dtype);
  FMOE_REQUIRE(d_out != nullptr, "fmoe_combine_fwd: null out");
  FMOE_REQUIRE(out_row_stride >= hidden, "fmoe_combine_fwd: out row stride %lld < D %lld",
               (long long)out_row_stride, (long long)hidden);
  if (hidden * 4 >= (int64_t(1) << 31)) {
    fmoe_host::set_error("fmoe_combine_fwd: D=%lld exceeds the 2 GiB row limit", (long long)hidden);
    return FMOE_ERANGE;
  }
  FwdArgs a{};
  a.mode = mode;
  a.N = num_rows;
  a.T = num_tokens;
  a.D = hidden;
  a.E = num_experts;
  a.out = d_out;
  a.out_stride = out_row_stride;
  a.accumulate = accumulate ? 1 : 0;
  a.s = static_cast<hipStream_t>(stream);
  if (mode == FMOE_MODE_DET) {
    FMOE_REQUIRE(d_plan != nullptr, "fmoe_combine_fwd(det): null plan");
    FMOE_REQUIRE(((uintptr_t)d_plan & 255) == 0, "fmoe_combine_fwd(det): plan not 256B-aligned");
    const char* ws = static_cast<const char*>(d_plan);
    a.status = reinterpret_cast<const int32_t*>(ws + fmoe_plan_status_offset());
    a.row_ptr = reinterpret_cast<const int32_t*>(ws + fmoe_plan_row_ptr_offset(a.N, a.T));
    a.rec = reinterpret_cast<const Rec*>(ws + fmoe_plan_records_offset(a.N, a.T));
    switch (x_dtype) {
      case FMOE_F32: return launch_fwd_x<float>(a, out_dtype);
      case FMOE_BF16: return launch_fwd_x<bf16_t>(a, out_dtype);
      case FMOE_F16: return launch_fwd_x<f16_t>(a, out_dtype);
    }
    fmoe_host::set_error("fmoe_combine_fwd: bad x dtype %d", x_dtype);
    return FMOE_EINVAL;
  }
  // atomic modes: the fp32 accumulator of a 16-bit output first (its size is checked before any
  // launch)
  const bool acc16 = mode == FMOE_MODE_ATOMIC && out_dtype != FMOE_F32;
  const int64_t need = fmoe_combine_fwd_workspace_bytes(mode, num_tokens, hidden, out_dtype);
  if (acc16)
    FMOE_REQUIRE(d_workspace && workspace_bytes >= need && ((uintptr_t)d_workspace & 15) == 0,
                 "fmoe_combine_fwd(atomic): a 16-bit output needs a 16-byte aligned fp32 "
                 "workspace of %lld bytes (fmoe_combine_fwd_workspace_bytes), got %lld",
                 (long long)need, (long long)workspace_bytes);
  if (num_rows == 0)  // nothing to add: an overwrite still clears out
    return accumulate ? FMOE_OK : zero_out(d_out, out_dtype, out_row_stride, hidden, num_tokens, a.s);
  FMOE_REQUIRE(d_indices && d_weights && d_ptr_table && d_offsets,
               "fmoe_combine_fwd(atomic): null index/weight/metadata pointer");
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype), "fmoe_combine_fwd: bad index dtype %d",
               idx_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "fmoe_combine_fwd: bad weight dtype %d",
               w_dtype);
  FMOE_REQUIRE(num_experts >= 1, "fmoe_combine_fwd: num_experts must be >= 1");
  a.idx = d_indices;
  a.idx_dtype = idx_dtype;
  a.w = d_weights;
  a.w_dtype = w_dtype;
  a.ptr_table = d_ptr_table;
  a.offsets = d_offsets;
  int target_dtype = out_dtype;
  float* acc = static_cast<float*>(d_workspace);
  if (acc16) {
    const int rc = out_dtype == FMOE_BF16
                       ? launch_acc_pass<bf16_t>(true, acc, d_out, out_row_stride, hidden,
                                                 num_tokens, accumulate, a.s)
                       : launch_acc_pass<f16_t>(true, acc, d_out, out_row_stride, hidden,
                                                num_tokens, accumulate, a.s);
    if (rc) return rc;
    a.out = acc;
    a.out_stride = hidden;
    target_dtype = FMOE_F32;
  } else if (!accumulate) {
    if (int rc = zero_out(d_out, out_dtype, out_row_stride, hidden, num_tokens, a.s)) return rc;
  }
  int rc = FMOE_EINVAL;
  switch (x_dtype) {
    case FMOE_F32: rc = launch_fwd_x<float>(a, target_dtype); break;
    case FMOE_BF16: rc = launch_fwd_x<bf16_t>(a, target_dtype); break;
    case FMOE_F16: rc = launch_fwd_x<f16_t>(a, target_dtype); break;
  }
  if (rc || !acc16) return rc;
  return out_dtype == FMOE_BF16
             ? launch_acc_pass<bf16_t>(false, acc, d_out, out_row_stride, hidden, num_tokens, 1,
                                       a.s)
             : launch_acc_pass<f16_t>(false, acc, d_out, out_row_stride, hidden, num_tokens, 1,
                                      a.s);
}

extern "C" int64_t fmoe_combine_small_max_rows(void) { return fmoe::kSmallRows; }

extern "C" int fmoe_combine_fwd_small(const int64_t* host_ptrs, const int64_t* host_rows,
                                      int64_t num_experts, const void* d_indices, int idx_dtype,
                                      const void* d_weights, int w_dtype, int64_t num_tokens,
                                      int64_t hidden, int x_dtype, void* d_out, int out_dtype,
                                      int64_t out_row_stride, int accumulate, int32_t* d_status,
                                      void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  FMOE_REQUIRE(num_tokens >= 1 && hidden >= 1, "fmoe_combine_fwd_small: bad sizes T=%lld D=%lld",
               (long long)num_tokens, (long long)hidden);
  if (num_tokens >= (int64_t(1) << 30) || hidden * 4 >= (int64_t(1) << 31)) {
    fmoe_host::set_error("fmoe_combine_fwd_small: T=%lld / D=%lld exceed the 32-bit counters",
                         (long long)num_tokens, (long long)hidden);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_float_dtype(x_dtype), "fmoe_combine_fwd_small: bad x dtype %d",
               x_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(out_dtype), "fmoe_combine_fwd_small: bad out dtype %d",
               out_dtype);
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype), "fmoe_combine_fwd_small: bad index dtype %d",
               idx_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "fmoe_combine_fwd_small: bad weight dtype %d",
               w_dtype);
  FMOE_REQUIRE(d_out && d_status, "fmoe_combine_fwd_small: null out / status");
  FMOE_REQUIRE(out_row_stride >= hidden, "fmoe_combine_fwd_small: out row stride %lld < D %lld",
               (long long)out_row_stride, (long long)hidden);
  SmallFwdArgs a{};
  const int64_t xb = x_dtype == FMOE_F32 ? 4 : 2;
  int64_t N = 0;
  if (int rc = small_host_table("fmoe_combine_fwd_small", host_ptrs, host_rows, num_experts,
                                hidden * xb, &a.meta, &N, &a.aligned))
    return rc;
  FMOE_REQUIRE(N == 0 || (d_indices && d_weights), "fmoe_combine_fwd_small: null indices/weights");
  a.idx = d_indices;
  a.idx_dtype = idx_dtype;
  a.w = d_weights;
  a.w_dtype = w_dtype;
  a.N = N;
  a.T = num_tokens;
  a.D = hidden;
  a.out = d_out;
  a.out_stride = out_row_stride;
  a.accumulate = accumulate ? 1 : 0;
  a.status = d_status;
  a.s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case FMOE_F32: return launch_small_x<float>(a, out_dtype);
    case FMOE_BF16: return launch_small_x<bf16_t>(a, out_dtype);
    case FMOE_F16: return launch_small_x<f16_t>(a, out_dtype);
  }
  fmoe_host::set_error("fmoe_combine_fwd_small: bad x dtype %d", x_dtype);
  return FMOE_EINVAL;
}
