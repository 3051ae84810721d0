// Backward combine, token-major:
//   grad_X[g, :] = round_x(f32(grad_out[t, :]) * w[g])          for every row g routed from token t
//   grad_w[g]    = sum_d grad_out[t, d] * X_e[g - off[e], d]     (fp64 accumulation of fp32
//                  partial sums of 8 exact products -- v_dot2 on 16-bit data -- rounded once)
//
// Replaces GroupedWeightedScatterAdd.backward (src/fastmoe/kernels/ops.py:333-359), which gathers
// grad_out by scatter index, multiplies into an fp32 [N, D] temporary and lets autograd cast it
// back -- three to four passes over [N, D] -- and which returns no gate gradient (:358-359).
//
// A wave owns one token.  It walks the columns in chunks of 64 * V * U; for each chunk it loads
// grad_out[t] once into registers, then for every routed row of the token (plan segment, ascending
// g) writes the grad_X chunk and, when the gate gradient is wanted, loads the X chunk, forms the
// lane's fp64 partial dot product and reduces it across the wave with a xor butterfly (every lane
// ends with the same sum).  Lane j keeps the running dot of the j-th row of the current batch of
// up to 64 rows, so grad_out is read from HBM exactly once for up to 64 rows per token.  Segment T
// of the plan (rows whose index was out of range) is zero-filled.
#include "common.h"

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

// Tile: U 16-byte vectors per lane per column step and batches of R rows whose X loads are in
// flight together and whose dot products are carried across column steps in registers, so each
// row costs one wave reduction.
template <typename TX, int V, int U, int RB, bool GX, bool GW, bool AL>
__device__ __forceinline__ void bwd_body(const int32_t* __restrict__ row_ptr,
                                         const Rec* __restrict__ rec, const TX* __restrict__ gout,
                                         int64_t gstride, TX* __restrict__ gx,
                                         void* __restrict__ gw, int gw_dtype, uint32_t D,
                                         uint32_t t) {
  using VX = Vec<TX, V>;
  using raw_t = typename VX::raw_t;
  constexpr int CW = kWave * V * U;
  constexpr int R = AL ? RB : 1;  // misaligned rows: one at a time (register budget)
  const int lane = threadIdx.x & (kWave - 1);
  const int beg = row_ptr[t];
  const int end = row_ptr[t + 1];
  if (beg == end) return;
  const uint32_t rowb = D * (uint32_t)sizeof(TX);
  const rsrc_t rg = make_rsrc(gout + (int64_t)t * gstride, rowb);

  for (int jb = beg; jb < end; jb += kWave) {
    const int cnt = min(end - jb, kWave);
    LaneRecs lr;
    lr.load(rec, jb, cnt, lane);
    for (int i = 0; i < cnt; i += R) {
      rsrc_t rx[R], rgx[R];
      float wr[R];
      int32_t gr[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int ir = min(i + r, cnt - 1);  // a partial batch repeats its last row (loads only)
        gr[r] = lr.row(ir);
        wr[r] = lr.w(ir);
        rx[r] = make_rsrc(lr.src(ir), rowb);
        if constexpr (GX) rgx[r] = make_rsrc(gx + (int64_t)gr[r] * D, rowb);
      }
      double part[R];
#pragma unroll
      for (int r = 0; r < R; ++r) part[r] = 0.0;
      for (uint32_t cb = 0; cb < D; cb += CW) {
        uint32_t off[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
          off[u] = (cb + (uint32_t)lane * V + (uint32_t)u * kWave * V) * (uint32_t)sizeof(TX);
        raw_t gr_raw[U];
        raw_t xr[GW ? R : 1][U];
#pragma unroll
        for (int u = 0; u < U; ++u) gr_raw[u] = VX::ld(rg, off[u]);  // beyond D: reads 0
        if constexpr (GW) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) xr[r][u] = load_x<TX, V, AL>(rx[r], off[u]);
        }
        float go[U][V];
#pragma unroll
        for (int u = 0; u < U; ++u) VX::cvt(gr_raw[u], go[u]);
        if constexpr (GX) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (i + r < cnt) {
#pragma unroll
              for (int u = 0; u < U; ++u) {
                float y[V];
#pragma unroll
                for (int v = 0; v < V; ++v) y[v] = go[u][v] * wr[r];
                VX::st(rgx[r], off[u], y);  // beyond D: dropped by the range check
              }
            }
          }
        }
        if constexpr (GW) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
              float x[V];
              VX::cvt(xr[r][u], x);
#pragma unroll
              for (int v = 0; v < V; ++v)
                part[r] = __builtin_fma((double)x[v], (double)go[u][v], part[r]);
            }
          }
        }
      }
      if constexpr (GW) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (i + r < cnt) {
            const double tot = wave_sum(part[r]);
            if (lane == 0) store_gate(gw, gw_dtype, gr[r], tot);
          }
        }
      }
    }
  }
}

// ---- packed-row-major variant -------------------------------------------------------------------
// A wave owns one packed row g: it streams X[g] and grad_X[g] front to back (non-temporal) and
// gathers grad_out[idx[g]] with the default cache policy, so the k rows of a token re-read their
// grad_out row from L2 / Infinity Cache rather than HBM.
int64_t plan_row_records_offset(int64_t num_rows, int64_t num_tokens);

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
  for (uint32_t cb = 0; cb < D; cb += 2 * CW) {  // two column steps in flight per iteration
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
      for (int u = 0; u < U; ++u) gr[h][u] = VX::template ld<kCPolCached>(rg, off[h][u]);
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
          for (int v = 0; v < V; ++v) y[v] = go[v] * wt;
          VX::st(rgx, off[h][u], y);  // beyond D: dropped by the range check
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

template <typename TX, int V, int U, bool GX, bool GW>
__global__ __launch_bounds__(kGroup) void k_bwd_rows(const int32_t* __restrict__ status,
                                                     const Rec* __restrict__ row_rec,
                                                     const TX* __restrict__ gout, int64_t gstride,
                                                     TX* __restrict__ gx, void* __restrict__ gw,
                                                     int gw_dtype, uint32_t D, uint32_t N) {
  const uint32_t g = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave);
  if (g >= N) return;
  const Rec r = row_rec[g];
  if (r.g < 0) {  // out-of-range scatter index: zero gradients
    bwd_zero_row<TX, V, GX, GW>(g, gx, gw, gw_dtype, D);
    return;
  }
  if (V > 1 && status[kStatusMisaligned] != 0)
    bwd_row_body<TX, V, U, GX, GW, false>(r.src, r.w, (uint32_t)r.g, g, gout, gstride, gx, gw,
                                          gw_dtype, D);
  else
    bwd_row_body<TX, V, U, GX, GW, true>(r.src, r.w, (uint32_t)r.g, g, gout, gstride, gx, gw,
                                         gw_dtype, D);
}

// ---- token-grouped variant (the default) ------------------------------------------------------
// A workgroup owns one token (plan segment); its 4 waves take the token's rows in turn, each
// streaming a whole row (X read and grad_X write contiguous, non-temporal).  The rows of a token
// run together on one CU, so grad_out[t] is fetched from HBM once and served from L2 to the
// others.  grad_w needs no cross-wave reduction: every wave owns whole rows.
template <typename TX, int V, int U, bool GX, bool GW>
__global__ __launch_bounds__(kGroup) void k_bwd_tok(const int32_t* __restrict__ status,
                                                    const int32_t* __restrict__ row_ptr,
                                                    const Rec* __restrict__ rec,
                                                    const TX* __restrict__ gout, int64_t gstride,
                                                    TX* __restrict__ gx, void* __restrict__ gw,
                                                    int gw_dtype, uint32_t D, uint32_t T) {
  const int wave = uniform(threadIdx.x / kWave);
  const bool al = !(V > 1 && status[kStatusMisaligned] != 0);
  // Segments 0..T (T: out-of-range rows); a grid smaller than T + 1 strides over them.
  for (uint32_t t = blockIdx.x; t <= T; t += gridDim.x) {
    const int beg = row_ptr[t];
    const int end = row_ptr[t + 1];
    for (int j = beg + wave; j < end; j += kWavesPerGroup) {
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
}

template <typename TX, int V, int U, int RB, bool GX, bool GW>
__global__ __launch_bounds__(kGroup) void k_bwd(const int32_t* __restrict__ status,
                                                const int32_t* __restrict__ row_ptr,
                                                const Rec* __restrict__ rec,
                                                const TX* __restrict__ gout, int64_t gstride,
                                                TX* __restrict__ gx, void* __restrict__ gw,
                                                int gw_dtype, uint32_t D, uint32_t T) {
  const uint32_t t = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave);
  if (t > T) return;
  if (t == T) {  // rows with an out-of-range scatter index: zero gradients
    const int lane = threadIdx.x & (kWave - 1);
    const int beg = row_ptr[t];
    const int end = row_ptr[t + 1];
    const uint32_t rowb = D * (uint32_t)sizeof(TX);
    for (int j = beg; j < end; ++j) {
      const int64_t g = rec[j].g;
      if constexpr (GX) {
        float z[V];
#pragma unroll
        for (int v = 0; v < V; ++v) z[v] = 0.f;
        const rsrc_t rz = make_rsrc(gx + g * D, rowb);
        for (uint32_t col = (uint32_t)lane * V; col < D; col += kWave * V)
          Vec<TX, V>::st(rz, col * (uint32_t)sizeof(TX), z);
      }
      if constexpr (GW) {
        if (lane == 0) store_gate(gw, gw_dtype, g, 0.0);
      }
    }
    return;
  }
  if (V > 1 && status[kStatusMisaligned] != 0)
    bwd_body<TX, V, U, RB, GX, GW, false>(row_ptr, rec, gout, gstride, gx, gw, gw_dtype, D, t);
  else
    bwd_body<TX, V, U, RB, GX, GW, true>(row_ptr, rec, gout, gstride, gx, gw, gw_dtype, D, t);
}

static int env_int_b(const char* name, int dflt) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : dflt;
}

struct BwdArgs {
  const int32_t* status;
  const int32_t* row_ptr;
  const Rec* rec;
  const Rec* row_rec;
  int64_t N;
  const void* gout;
  int64_t gstride;
  void* gx;
  void* gw;
  int gw_dtype;
  int64_t D, T;
  hipStream_t s;
};

template <typename TX, int V, int U, int RB, bool GX, bool GW>
static int launch_bwd_k(const BwdArgs& a) {
  const int64_t blocks = (a.T + 1 + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((k_bwd<TX, V, U, RB, GX, GW>), dim3((unsigned)blocks), dim3(kGroup), 0, a.s,
                     a.status, a.row_ptr, a.rec, static_cast<const TX*>(a.gout), a.gstride,
                     static_cast<TX*>(a.gx), a.gw, a.gw_dtype, (uint32_t)a.D, (uint32_t)a.T);
  return fmoe_host::check_launch("fmoe_combine_bwd");
}

template <typename TX, int V, int U, int RB>
static int launch_bwd_u(const BwdArgs& a) {
  if (a.gx && a.gw) return launch_bwd_k<TX, V, U, RB, true, true>(a);
  if (a.gx) return launch_bwd_k<TX, V, U, RB, true, false>(a);
  return launch_bwd_k<TX, V, U, RB, false, true>(a);
}

template <typename TX, int V, int U, bool GX, bool GW>
static int launch_bwd_rows_k(const BwdArgs& a) {
  const int64_t blocks = (a.N + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((k_bwd_rows<TX, V, U, GX, GW>), dim3((unsigned)blocks), dim3(kGroup), 0, a.s,
                     a.status, a.row_rec, static_cast<const TX*>(a.gout), a.gstride,
                     static_cast<TX*>(a.gx), a.gw, a.gw_dtype, (uint32_t)a.D, (uint32_t)a.N);
  return fmoe_host::check_launch("fmoe_combine_bwd(rows)");
}

template <typename TX, int V, int U, bool GX, bool GW>
static int launch_bwd_tok_k(const BwdArgs& a) {
  int64_t grid = a.T + 1;
  const int persist = env_int_b("FMOE_BWD_GRID", 0);  // workgroups; 0 = one per segment
  if (persist > 0 && persist < grid) grid = persist;
  hipLaunchKernelGGL((k_bwd_tok<TX, V, U, GX, GW>), dim3((unsigned)grid), dim3(kGroup), 0, a.s,
                     a.status, a.row_ptr, a.rec, static_cast<const TX*>(a.gout), a.gstride,
                     static_cast<TX*>(a.gx), a.gw, a.gw_dtype, (uint32_t)a.D, (uint32_t)a.T);
  return fmoe_host::check_launch("fmoe_combine_bwd(tok)");
}

template <typename TX, int V, int U>
static int launch_bwd_tok(const BwdArgs& a) {
  if (a.gx && a.gw) return launch_bwd_tok_k<TX, V, U, true, true>(a);
  if (a.gx) return launch_bwd_tok_k<TX, V, U, true, false>(a);
  return launch_bwd_tok_k<TX, V, U, false, true>(a);
}

template <typename TX, int V, int U>
static int launch_bwd_rows(const BwdArgs& a) {
  if (a.gx && a.gw) return launch_bwd_rows_k<TX, V, U, true, true>(a);
  if (a.gx) return launch_bwd_rows_k<TX, V, U, true, false>(a);
  return launch_bwd_rows_k<TX, V, U, false, true>(a);
}

// Tile shapes (U, R); FMOE_BWD_TILE=<U><R> (e.g. "28") overrides the choice for tuning.
template <typename TX>
static int launch_bwd_x(const BwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int eb = (int)sizeof(TX);
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.gout % 16 == 0) &&
                      ((a.gstride * eb) % 16 == 0) && ((uintptr_t)a.gx % 16 == 0) &&
                      env_int_b("FMOE_FORCE_SCALAR", 0) == 0;
  if (!vec_ok) return launch_bwd_u<TX, 1, 4, 4>(a);
  // Token-grouped whole rows by default; FMOE_BWD_ORDER=row / =column select the packed-row-major
  // and the token-major column-tiled kernels (kept for comparison).
  const char* order = getenv("FMOE_BWD_ORDER");
  const int ur = env_int_b("FMOE_BWD_ROWS_U", 2);
  if (!order || order[0] == 't') {
    if (ur == 4) return launch_bwd_tok<TX, V, 4>(a);
    if (ur == 1) return launch_bwd_tok<TX, V, 1>(a);
    return launch_bwd_tok<TX, V, 2>(a);
  }
  if (order[0] == 'r') {
    if (ur == 4) return launch_bwd_rows<TX, V, 4>(a);
    if (ur == 1) return launch_bwd_rows<TX, V, 1>(a);
    return launch_bwd_rows<TX, V, 2>(a);
  }
  const int tile = env_int_b("FMOE_BWD_TILE", 0);
  int U = tile / 10, R = tile % 10;
  if (!((U == 4 && R == 4) || (U == 2 && (R == 8 || R == 4)) || (U == 1 && R == 8))) {
    U = a.D >= (int64_t)kWave * V * 2 ? 2 : 1;
    R = U == 2 ? 4 : 8;
  }
  if (U == 4) return launch_bwd_u<TX, V, 4, 4>(a);
  if (U == 2 && R == 8) return launch_bwd_u<TX, V, 2, 8>(a);
  if (U == 2) return launch_bwd_u<TX, V, 2, 4>(a);
  return launch_bwd_u<TX, V, 1, 8>(a);
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
  a.row_rec = reinterpret_cast<const Rec*>(ws + plan_row_records_offset(N, T));
  a.N = N;
  a.gout = d_grad_out;
  a.gstride = gout_row_stride;
  a.gx = d_grad_x;
  a.gw = d_grad_w;
  a.gw_dtype = gw_dtype;
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
