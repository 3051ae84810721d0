// Backward combine:
//   grad_X[g, :] = round_x(f32(grad_out[t, :]) * w[g])          for every row g routed from token t
//   grad_w[g]    = sum_d grad_out[t, d] * X_e[g - off[e], d]     (fp64 accumulation of fp32
//                  partial sums of 8 exact products -- v_dot2 on 16-bit data -- rounded once)
//
// Replaces GroupedWeightedScatterAdd.backward (src/fastmoe/kernels/ops.py:333-359), which gathers
// grad_out by scatter index, multiplies into an fp32 [N, D] temporary and lets autograd cast it
// back -- three to four passes over [N, D] -- and which returns no gate gradient (:358-359).
//
// Work decomposition (token-grouped whole rows).  A workgroup owns one token's plan segment; its
// waves take the token's rows in turn and each streams a whole row front to back: X[g] read and
// grad_X[g] written with the non-temporal policy, grad_out[t] read with the default policy so the
// rows of a token, running together on one CU, fetch it from HBM once and share it through L2.
// grad_w needs no cross-wave reduction: a wave owns whole rows and reduces its dot product with a
// xor butterfly.  Segment T of the plan (rows whose scatter index was out of range) gets zeros.
//
// Two passes.  When both gradients are wanted the grad_X pass (a write stream) and the grad_w pass
// (read streams only) run as two back-to-back launches rather than one fused kernel: HBM loses
// about a tenth of its throughput when a kernel interleaves this much reading and writing at fine
// grain, which costs more than reading grad_out (T * D, one k-th of X at top-k) a second time.
#include "plan.h"

namespace fmoe {

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) x += __shfl_xor(x, d, kWave);
  return x;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Partial dot product of V elements of X with V elements of grad_out (raw storage).  16-bit
// inputs: v_dot2_f32_{bf16,f16} sums the V exact products in fp32 (3 roundings at most for
// V = 8, i.e. <= 4 * 2^-24 of the partial's absolute sum), the caller accumulates the partials in
// fp64.  fp32 inputs: fp64 fma per element (products exact in fp64).
template <typename TX, int V>
__device__ __forceinline__ double dot_partial(const typename Vec<TX, V>::raw_t& x,
                                              const typename Vec<TX, V>::raw_t& g) {
  using R = typename Vec<TX, V>::R;
  if constexpr (ElemInfo<TX>::kBytes == 2 && V >= 2) {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
      const uint32_t xw = R::word(x, i), gw = R::word(g, i);
      if constexpr (std::is_same<TX, bf16_t>::value)
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, xw),
                                            __builtin_bit_cast(bf16x2_t, gw), d, false);
      else
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, xw), __builtin_bit_cast(f16x2_t, gw),
                                   d, false);
    }
    return (double)d;
  } else {
    float xf[V], gf[V];
    Vec<TX, V>::cvt(x, xf);
    Vec<TX, V>::cvt(g, gf);
    double d = 0.0;
#pragma unroll
    for (int v = 0; v < V; ++v) d = __builtin_fma((double)xf[v], (double)gf[v], d);
    return d;
  }
}

__device__ __forceinline__ void store_gate(void* gw, int dtype, int64_t g, double v) {
  const float f = (float)v;
  if (dtype == FMOE_F32) static_cast<float*>(gw)[g] = f;
  else if (dtype == FMOE_BF16) st1(static_cast<bf16_t*>(gw) + g, f);
  else st1(static_cast<f16_t*>(gw) + g, f);
}

// Zero gradients of a row whose scatter index was out of range.
template <typename TX, int V, bool GX, bool GW>
__device__ __forceinline__ void bwd_zero_row(uint32_t g, TX* __restrict__ gx, void* __restrict__ gw,
                                             int gw_dtype, uint32_t D) {
  const int lane = threadIdx.x & (kWave - 1);
  if constexpr (GX) {
    float z[V];
#pragma unroll
    for (int v = 0; v < V; ++v) z[v] = 0.f;
    const rsrc_t rz = make_rsrc(gx + (int64_t)g * D, D * (uint32_t)sizeof(TX));
    for (uint32_t col = (uint32_t)lane * V; col < D; col += kWave * V)
      Vec<TX, V>::st(rz, col * (uint32_t)sizeof(TX), z);
  }
  if constexpr (GW) {
    if (lane == 0) store_gate(gw, gw_dtype, g, 0.0);
  }
}

// One whole row g of token t: two column steps of 64 * V * U columns per iteration, so 2 * U
// loads of each input stream per lane are in flight; columns past D read 0 and drop their stores
// (buffer range check).
template <typename TX, int V, int U, bool GX, bool GW, bool AL>
__device__ __forceinline__ void bwd_row_body(uint64_t src, float wt, uint32_t t, uint32_t g,
                                             const TX* __restrict__ gout, int64_t gstride,
                                             TX* __restrict__ gx, void* __restrict__ gw,
                                             int gw_dtype, uint32_t D) {
  using VX = Vec<TX, V>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t rowb = D * (uint32_t)sizeof(TX);
  const rsrc_t rg = make_rsrc(gout + (int64_t)t * gstride, rowb);
  const rsrc_t rx = make_rsrc(src, rowb);
  const rsrc_t rgx = make_rsrc(gx + (int64_t)g * D, rowb);
  double part = 0.0;
  for (uint32_t cb = 0; cb < D; cb += 2 * CW) {
    uint32_t off[2][U];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u)
        off[h][u] =
            (cb + h * CW + (uint32_t)lane * V + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TX);
    raw_t gr[2][U];
    raw_t xr[GW ? 2 : 1][U];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u) gr[h][u] = VX::template ld<FMOE_GOUT_CPOL>(rg, off[h][u]);
    if constexpr (GW) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < U; ++u) xr[h][u] = load_x<TX, V, AL>(rx, off[h][u]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (GX) {
          float go[V], y[V];
          VX::cvt(gr[h][u], go);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            y[v] = go[v] * wt;
            // f16: keep the fp32 product in a register.  Otherwise the multiply and the
            // conversion to f16 fuse into v_fma_mixlo_f16, which rounds once where the reference
            // (index_select * w in fp32, then the cast to f16) rounds twice.
            if constexpr (std::is_same<TX, f16_t>::value) __asm__("" : "+v"(y[v]));
          }
          VX::template st<FMOE_GX_CPOL>(rgx, off[h][u], y);
        }
        if constexpr (GW) part += dot_partial<TX, V>(xr[h][u], gr[h][u]);
      }
    }
  }
  if constexpr (GW) {
    const double tot = wave_sum(part);
    if (lane == 0) store_gate(gw, gw_dtype, g, tot);
  }
}

constexpr int kBwdWaves = FMOE_BWD_WAVES;
#ifndef FMOE_GW_STAGE_STEPS
#define FMOE_GW_STAGE_STEPS 4  // column steps of grad_out per LDS slice (one barrier per slice)
#endif

// grad_w pass of a token with at most kBwdWaves rows, grad_out staged in LDS: per slice of
// FMOE_GW_STAGE_STEPS column steps the workgroup reads that part of grad_out[t] once (one 16-byte
// vector per thread per step), and every wave takes it from LDS instead of fetching the same bytes
// from L2 (the per-wave path reads grad_out once per row).  Double-buffered: the next slice's
// loads are in flight while a slice is consumed, and one barrier per slice both publishes a slice
// and frees the other buffer.  The products and their accumulation order are those of
// bwd_row_body, so grad_w is bit-identical to it.
template <typename TX, int V, int U>
__device__ __forceinline__ void bwd_gw_staged(const Rec* __restrict__ rec, int beg, int cnt,
                                              uint32_t t, const TX* __restrict__ gout,
                                              int64_t gstride, void* __restrict__ gw,
                                              int gw_dtype, uint32_t D) {
  using VX = Vec<TX, V>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  constexpr int kStepVecs = 2 * U * kWave;  // 16-byte vectors of grad_out per column step
  static_assert(kStepVecs == kBwdWaves * kWave, "one staging vector per thread per step");
  constexpr int S = FMOE_GW_STAGE_STEPS;  // column steps per slice
  __shared__ raw_t stage[2][S * kStepVecs];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const bool has = wave < cnt;  // wave-uniform
  const uint32_t rowb = D * (uint32_t)sizeof(TX);
  const rsrc_t rg = make_rsrc(gout + (int64_t)t * gstride, rowb);
  Rec r{};
  if (has) r = rec[beg + wave];
  const rsrc_t rx = make_rsrc(has ? r.src : (uint64_t)(uintptr_t)gout, rowb);
  constexpr uint32_t kStepBytes = (uint32_t)kStepVecs * 16;
  constexpr uint32_t kSliceBytes = S * kStepBytes;
  const uint32_t slices = (D + S * 2 * CW - 1) / (S * 2 * CW);
#pragma unroll
  for (int q = 0; q < S; ++q)
    stage[0][q * kStepVecs + tid] =
        VX::template ld<FMOE_GOUT_CPOL>(rg, (uint32_t)(q * kStepVecs + tid) * 16);
  // X of column step q of slice sl, for this wave's row
  auto load_step = [&](uint32_t sl, int q, raw_t (&xr)[2][U]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u)
        xr[h][u] = load_x<TX, V, true>(rx, sl * kSliceBytes + (uint32_t)q * kStepBytes +
                                               (uint32_t)((h * U + u) * kWave + lane) * 16);
  };
  double part = 0.0;
  for (uint32_t sl = 0; sl < slices; ++sl) {
    raw_t xr[S][2][U];
    if (has) load_step(sl, 0, xr[0]);  // in flight across the barrier
    // the next slice (past the row: zeros from the range check, no memory traffic)
    raw_t nxt[S];
#pragma unroll
    for (int q = 0; q < S; ++q)
      nxt[q] = VX::template ld<FMOE_GOUT_CPOL>(
          rg, (sl + 1) * kSliceBytes + (uint32_t)(q * kStepVecs + tid) * 16);
    __syncthreads();  // slice sl is in LDS; every wave is done with the other buffer
#pragma unroll
    for (int q = 0; q < S; ++q) {
      if (has) {
        if (q + 1 < S) load_step(sl, q + 1, xr[(q + 1) % S]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int u = 0; u < U; ++u)
            part += dot_partial<TX, V>(xr[q][h][u],
                                       stage[sl & 1][q * kStepVecs + (h * U + u) * kWave + lane]);
      }
    }
#pragma unroll
    for (int q = 0; q < S; ++q) stage[(sl + 1) & 1][q * kStepVecs + tid] = nxt[q];
  }
  if (has) {
    const double tot = wave_sum(part);
    if (lane == 0) store_gate(gw, gw_dtype, r.g, tot);
  }
}

// Workgroup per plan segment: token t = blockIdx.x; segment T holds the out-of-range rows.
template <typename TX, int V, int U, bool GX, bool GW>
__global__ __launch_bounds__(kBwdWaves * kWave) void k_bwd_tok(const int32_t* __restrict__ status,
                                                               const int32_t* __restrict__ row_ptr,
                                                               const Rec* __restrict__ rec,
                                                               const TX* __restrict__ gout,
                                                               int64_t gstride,
                                                               TX* __restrict__ gx,
                                                               void* __restrict__ gw, int gw_dtype,
                                                               uint32_t D, uint32_t T, int staged) {
  const uint32_t t = blockIdx.x;
  const int wave = uniform(threadIdx.x / kWave);
  const bool al = !(V > 1 && status[kStatusMisaligned] != 0);
  const int beg = row_ptr[t];
  const int end = row_ptr[t + 1];
  if constexpr (GW && !GX && V > 1 && 2 * U == kBwdWaves) {
    if (staged && t < T && al && end - beg <= kBwdWaves) {  // workgroup-uniform
      if (end > beg) bwd_gw_staged<TX, V, U>(rec, beg, end - beg, t, gout, gstride, gw, gw_dtype, D);
      return;
    }
  }
  for (int j = beg + wave; j < end; j += kBwdWaves) {
    const Rec r = rec[j];
    if (t == T) {
      bwd_zero_row<TX, V, GX, GW>((uint32_t)r.g, gx, gw, gw_dtype, D);
    } else if (al) {
      bwd_row_body<TX, V, U, GX, GW, true>(r.src, r.w, t, (uint32_t)r.g, gout, gstride, gx, gw,
                                           gw_dtype, D);
    } else {
      bwd_row_body<TX, V, U, GX, GW, false>(r.src, r.w, t, (uint32_t)r.g, gout, gstride, gx, gw,
                                            gw_dtype, D);
    }
  }
}

// Small inputs (at most kSmallRows rows) without a plan: one wave per packed row g, which
// needs nothing but its own token id, expert and gate -- grad_X[g] = round(grad_out[t] * w[g])
// and grad_w[g] = <X[g], grad_out[t]> with bwd_row_body, both in one launch.  With U chosen as for
// the grad_w pass, both gradients equal the planned passes' bit for bit.
template <typename TX, int V, int U, bool GX, bool GW, bool AL>
__global__ __launch_bounds__(kGroup) void k_bwd_small(const HostTable meta,
                                                      const void* __restrict__ idx, int idx_dtype,
                                                      const void* __restrict__ w, int w_dtype,
                                                      uint32_t N, uint32_t T,
                                                      const TX* __restrict__ gout, int64_t gstride,
                                                      TX* __restrict__ gx, void* __restrict__ gw,
                                                      int gw_dtype, uint32_t D) {
  __shared__ int off_lds[kMetaChunk + 1];
  __shared__ uint64_t ptr_lds[kMetaChunk];
  small_table_to_lds(meta, off_lds, ptr_lds);
  __syncthreads();
  const uint32_t row_bytes = D * (uint32_t)sizeof(TX);
  for (uint32_t g = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave); g < N;
       g += gridDim.x * kWavesPerGroup) {
    const int64_t t = load_index(idx, idx_dtype, g);
    if (t < 0 || t >= (int64_t)T) {  // out of range: zero gradients, as the plan's segment T
      bwd_zero_row<TX, V, GX, GW>(g, gx, gw, gw_dtype, D);
      continue;
    }
    const int e = expert_of_row32(off_lds, meta.count, (int)g);
    const uint64_t src = ptr_lds[e] + (uint64_t)(g - (uint32_t)off_lds[e]) * (uint64_t)row_bytes;
    bwd_row_body<TX, V, U, GX, GW, AL>(src, load_weight(w, w_dtype, g), (uint32_t)t, g, gout,
                                       gstride, gx, gw, gw_dtype, D);
  }
}

struct BwdArgs {
  const int32_t* status;
  const int32_t* row_ptr;
  const Rec* rec;
  const void* gout;
  int64_t gstride;
  void* gx;
  void* gw;
  int gw_dtype;
  int gw_staged;  // grad_w pass: grad_out shared through LDS (option "gw_staged" = 0 turns it off)
  int64_t D, T;
  hipStream_t s;
};

template <typename TX, int V, int U, bool GX, bool GW>
static int launch_bwd_k(const BwdArgs& a) {
  hipLaunchKernelGGL((k_bwd_tok<TX, V, U, GX, GW>), dim3((unsigned)(a.T + 1)),
                     dim3(kBwdWaves * kWave), 0, a.s, a.status, a.row_ptr, a.rec,
                     static_cast<const TX*>(a.gout), a.gstride, static_cast<TX*>(a.gx), a.gw,
                     a.gw_dtype, (uint32_t)a.D, (uint32_t)a.T, a.gw_staged);
  return fmoe_host::check_launch("fmoe_combine_bwd");
}

template <typename TX, int V, bool GX, bool GW>
static int launch_bwd_v(const BwdArgs& a, int U) {
  if (U == 4) return launch_bwd_k<TX, V, 4, GX, GW>(a);
  if (U == 2) return launch_bwd_k<TX, V, 2, GX, GW>(a);
  return launch_bwd_k<TX, V, 1, GX, GW>(a);
}

// U, the 16-byte vectors per lane per column step, is chosen per pass from the row length in
// bytes (option "bwd_u" = 1|2|4 sets both).  grad_X (and the fused pass): 4 from 8 KiB rows, 2
// from 4 KiB, else 1.  grad_w: 4 -- the LDS-staged pass, whose column step is 8 KiB -- only from
// 24 KiB rows, 2 from 4 KiB, else 1.  The staged pass hides its per-step barrier only over several
// steps; at rows of 8 KiB (one step) it takes about twice as long as the per-wave pass at U = 2
// (bf16, T = 4096, top-8, HIP events: 72.9 against 37.6 µs at D = 4096, 104.2 against 82.2 µs at
// D = 7168, 173.6 against 179.5 µs at D = 16384 where it is kept).  The "bwd_fused" option runs
// both gradients in one pass (kept for measurement).
template <typename TX>
static int launch_bwd_x(const BwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int eb = (int)sizeof(TX);
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.gout % 16 == 0) &&
                      ((a.gstride * eb) % 16 == 0) && ((uintptr_t)a.gx % 16 == 0) &&
                      fmoe_host::opt(fmoe_host::kOptForceScalar) == 0;
  const bool fused = fmoe_host::opt(fmoe_host::kOptBwdFused) != 0;
  if (!vec_ok) {
    if (a.gx && a.gw && fused) return launch_bwd_k<TX, 1, 4, true, true>(a);
    if (a.gx)
      if (int rc = launch_bwd_k<TX, 1, 4, true, false>(a)) return rc;
    return a.gw ? launch_bwd_k<TX, 1, 4, false, true>(a) : FMOE_OK;
  }
  const int64_t row_bytes = a.D * eb;
  int ux = (int)fmoe_host::opt(fmoe_host::kOptBwdU);
  int uw = ux;
  if (ux != 1 && ux != 2 && ux != 4) {
    ux = row_bytes >= 8192 ? 4 : (row_bytes >= 4096 ? 2 : 1);
    uw = row_bytes >= 24576 ? 4 : (row_bytes >= 4096 ? 2 : 1);
  }
  if (a.gx && a.gw && fused) return launch_bwd_v<TX, V, true, true>(a, ux);
  if (a.gx)
    if (int rc = launch_bwd_v<TX, V, true, false>(a, ux)) return rc;  // grad_X: write pass
  return a.gw ? launch_bwd_v<TX, V, false, true>(a, uw) : FMOE_OK;    // grad_w: read pass
}

}  // namespace fmoe

extern "C" int fmoe_combine_bwd(const void* d_plan, int64_t num_rows, int64_t num_tokens,
                                int64_t hidden, int x_dtype, const void* d_grad_out,
                                int gout_dtype, int64_t gout_row_stride, void* d_grad_x,
                                void* d_grad_w, int gw_dtype, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  const int64_t N = num_rows, T = num_tokens, D = hidden;
  FMOE_REQUIRE(N >= 0 && T >= 1 && D >= 1, "fmoe_combine_bwd: bad sizes N=%lld T=%lld D=%lld",
               (long long)N, (long long)T, (long long)D);
  if (N >= (int64_t(1) << 31) || T >= (int64_t(1) << 30)) {
    fmoe_host::set_error("fmoe_combine_bwd: N/T exceed the 32-bit row counters");
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_float_dtype(x_dtype), "fmoe_combine_bwd: bad x dtype %d", x_dtype);
  FMOE_REQUIRE(gout_dtype == x_dtype,
               "fmoe_combine_bwd: grad_out dtype %d must equal the expert dtype %d", gout_dtype,
               x_dtype);
  FMOE_REQUIRE(d_plan && d_grad_out, "fmoe_combine_bwd: null plan / grad_out");
  FMOE_REQUIRE(((uintptr_t)d_plan & 255) == 0, "fmoe_combine_bwd: plan not 256B-aligned");
  FMOE_REQUIRE(gout_row_stride >= 0, "fmoe_combine_bwd: negative grad_out row stride");
  if (D * 4 >= (int64_t(1) << 31)) {
    fmoe_host::set_error("fmoe_combine_bwd: D=%lld exceeds the 2 GiB row limit", (long long)D);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(d_grad_w == nullptr || fmoe_host::is_float_dtype(gw_dtype),
               "fmoe_combine_bwd: bad grad_w dtype %d", gw_dtype);
  if (N == 0 || (d_grad_x == nullptr && d_grad_w == nullptr)) return FMOE_OK;
  const char* ws = static_cast<const char*>(d_plan);
  BwdArgs a;
  a.status = reinterpret_cast<const int32_t*>(ws + fmoe_plan_status_offset());
  a.row_ptr = reinterpret_cast<const int32_t*>(ws + fmoe_plan_row_ptr_offset(N, T));
  a.rec = reinterpret_cast<const Rec*>(ws + fmoe_plan_records_offset(N, T));
  a.gout = d_grad_out;
  a.gstride = gout_row_stride;
  a.gx = d_grad_x;
  a.gw = d_grad_w;
  a.gw_dtype = gw_dtype;
  a.gw_staged = fmoe_host::opt(fmoe_host::kOptGwStaged) != 0;
  a.D = D;
  a.T = T;
  a.s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case FMOE_F32: return launch_bwd_x<float>(a);
    case FMOE_BF16: return launch_bwd_x<bf16_t>(a);
    case FMOE_F16: return launch_bwd_x<f16_t>(a);
  }
  fmoe_host::set_error("fmoe_combine_bwd: bad x dtype %d", x_dtype);
  return FMOE_EINVAL;
}

namespace fmoe {
namespace {

struct SmallBwdArgs {
  HostTable meta;
  const void* idx;
  int idx_dtype;
  const void* w;
  int w_dtype;
  int64_t N, T, D;
  const void* gout;
  int64_t gstride;
  void* gx;
  void* gw;
  int gw_dtype;
  bool aligned;
  hipStream_t s;
};

template <typename TX, int V, int U, bool GX, bool GW, bool AL>
int launch_bwd_small_k(const SmallBwdArgs& a) {
  const unsigned blocks = (unsigned)((a.N + kWavesPerGroup - 1) / kWavesPerGroup);
  hipLaunchKernelGGL((k_bwd_small<TX, V, U, GX, GW, AL>), dim3(blocks), dim3(kGroup), 0, a.s,
                     a.meta, a.idx, a.idx_dtype, a.w, a.w_dtype, (uint32_t)a.N, (uint32_t)a.T,
                     static_cast<const TX*>(a.gout), a.gstride, static_cast<TX*>(a.gx), a.gw,
                     a.gw_dtype, (uint32_t)a.D);
  return fmoe_host::check_launch("fmoe_combine_bwd_small");
}

template <typename TX, int V, int U, bool AL>
int launch_bwd_small_g(const SmallBwdArgs& a) {
  if (a.gx && a.gw) return launch_bwd_small_k<TX, V, U, true, true, AL>(a);
  if (a.gx) return launch_bwd_small_k<TX, V, U, true, false, AL>(a);
  return launch_bwd_small_k<TX, V, U, false, true, AL>(a);
}

// The planned passes' vector width and, for grad_w's reduction order, the grad_w pass's U.
template <typename TX>
int launch_bwd_small_x(const SmallBwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int eb = (int)sizeof(TX);
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.gout % 16 == 0) &&
                      ((a.gstride * eb) % 16 == 0) && ((uintptr_t)a.gx % 16 == 0) &&
                      fmoe_host::opt(fmoe_host::kOptForceScalar) == 0;
  if (!vec_ok) return launch_bwd_small_g<TX, 1, 4, true>(a);
  const int64_t row_bytes = a.D * eb;
  int U = (int)fmoe_host::opt(fmoe_host::kOptBwdU);
  if (U != 1 && U != 2 && U != 4) U = row_bytes >= 24576 ? 4 : (row_bytes >= 4096 ? 2 : 1);
  if (!a.aligned) {
    if (U == 4) return launch_bwd_small_g<TX, V, 4, false>(a);
    if (U == 2) return launch_bwd_small_g<TX, V, 2, false>(a);
    return launch_bwd_small_g<TX, V, 1, false>(a);
  }
  if (U == 4) return launch_bwd_small_g<TX, V, 4, true>(a);
  if (U == 2) return launch_bwd_small_g<TX, V, 2, true>(a);
  return launch_bwd_small_g<TX, V, 1, true>(a);
}

}  // namespace
}  // namespace fmoe

extern "C" int fmoe_combine_bwd_small(const int64_t* host_ptrs, const int64_t* host_rows,
                                      int64_t num_experts, const void* d_indices, int idx_dtype,
                                      const void* d_weights, int w_dtype, int64_t num_tokens,
                                      int64_t hidden, int x_dtype, const void* d_grad_out,
                                      int gout_dtype, int64_t gout_row_stride, void* d_grad_x,
                                      void* d_grad_w, int gw_dtype, void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  FMOE_REQUIRE(num_tokens >= 1 && hidden >= 1, "fmoe_combine_bwd_small: bad sizes T=%lld D=%lld",
               (long long)num_tokens, (long long)hidden);
  if (num_tokens >= (int64_t(1) << 30) || hidden * 4 >= (int64_t(1) << 31)) {
    fmoe_host::set_error("fmoe_combine_bwd_small: T=%lld / D=%lld exceed the 32-bit counters",
                         (long long)num_tokens, (long long)hidden);
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_float_dtype(x_dtype), "fmoe_combine_bwd_small: bad x dtype %d",
               x_dtype);
  FMOE_REQUIRE(gout_dtype == x_dtype,
               "fmoe_combine_bwd_small: grad_out dtype %d must equal the expert dtype %d",
               gout_dtype, x_dtype);
  FMOE_REQUIRE(fmoe_host::is_index_dtype(idx_dtype), "fmoe_combine_bwd_small: bad index dtype %d",
               idx_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(w_dtype), "fmoe_combine_bwd_small: bad weight dtype %d",
               w_dtype);
  FMOE_REQUIRE(d_grad_w == nullptr || fmoe_host::is_float_dtype(gw_dtype),
               "fmoe_combine_bwd_small: bad grad_w dtype %d", gw_dtype);
  FMOE_REQUIRE(gout_row_stride >= 0, "fmoe_combine_bwd_small: negative grad_out row stride");
  SmallBwdArgs a{};
  const int64_t xb = x_dtype == FMOE_F32 ? 4 : 2;
  int64_t N = 0;
  if (int rc = small_host_table("fmoe_combine_bwd_small", host_ptrs, host_rows, num_experts,
                                hidden * xb, &a.meta, &N, &a.aligned))
    return rc;
  if (N == 0 || (d_grad_x == nullptr && d_grad_w == nullptr)) return FMOE_OK;
  FMOE_REQUIRE(d_indices && d_weights && d_grad_out,
               "fmoe_combine_bwd_small: null indices / weights / grad_out");
  a.idx = d_indices;
  a.idx_dtype = idx_dtype;
  a.w = d_weights;
  a.w_dtype = w_dtype;
  a.N = N;
  a.T = num_tokens;
  a.D = hidden;
  a.gout = d_grad_out;
  a.gstride = gout_row_stride;
  a.gx = d_grad_x;
  a.gw = d_grad_w;
  a.gw_dtype = gw_dtype;
  a.s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case FMOE_F32: return launch_bwd_small_x<float>(a);
    case FMOE_BF16: return launch_bwd_small_x<bf16_t>(a);
    case FMOE_F16: return launch_bwd_small_x<f16_t>(a);
  }
  fmoe_host::set_error("fmoe_combine_bwd_small: bad x dtype %d", x_dtype);
  return FMOE_EINVAL;
}
