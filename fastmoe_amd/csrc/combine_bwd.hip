// Backward combine, token-major:
//   grad_X[g, :] = round_x(f32(grad_out[t, :]) * w[g])          for every row g routed from token t
//   grad_w[g]    = sum_d grad_out[t, d] * X_e[g - off[e], d]     (fp64 accumulation, rounded once)
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

__device__ __forceinline__ void store_gate(void* gw, int dtype, int64_t g, double v) {
  const float f = (float)v;
  if (dtype == FMOE_F32) static_cast<float*>(gw)[g] = f;
  else if (dtype == FMOE_BF16) st1(static_cast<bf16_t*>(gw) + g, f);
  else st1(static_cast<f16_t*>(gw) + g, f);
}

template <typename TX, int V, int U, bool FULL, bool GX, bool GW, bool AL>
__device__ __forceinline__ void bwd_body(const int32_t* __restrict__ row_ptr,
                                         const Rec* __restrict__ rec, const TX* __restrict__ gout,
                                         int64_t gstride, TX* __restrict__ gx,
                                         void* __restrict__ gw, int gw_dtype, int64_t D,
                                         uint32_t t) {
  using raw_t = typename Vec<TX, V>::raw_t;
  constexpr int CW = kWave * V * U;
  const int lane = threadIdx.x & (kWave - 1);
  const int beg = row_ptr[t];
  const int end = row_ptr[t + 1];
  if (beg == end) return;
  const TX* grow = gout + (int64_t)t * gstride;

  for (int pb = beg; pb < end; pb += kWave) {
    const int pe = min(end, pb + kWave);
    double mine = 0.0;  // lane j: dot product of row pb + j
    for (int64_t cbase = 0; cbase < D; cbase += CW) {
      int64_t col[U], cl[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        col[u] = cbase + (int64_t)lane * V + (int64_t)u * kWave * V;
        ok[u] = FULL || col[u] < D;
        cl[u] = ok[u] ? col[u] : D - V;
      }
      float go[U][V];
      {
        raw_t r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = Vec<TX, V>::ld(grow + cl[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          Vec<TX, V>::cvt(r[u], go[u]);
          if (!FULL && !ok[u]) {
#pragma unroll
            for (int v = 0; v < V; ++v) go[u][v] = 0.f;
          }
        }
      }
      int j = pb;
      // Two rows per iteration: their X loads are in flight together.
      for (; j + 2 <= pe; j += 2) {
        const Rec r0 = rec[j];
        const Rec r1 = rec[j + 1];
        raw_t a[U], b[U];
        if constexpr (GW) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            a[u] = load_x<TX, V, AL>(r0.src, cl[u]);
            b[u] = load_x<TX, V, AL>(r1.src, cl[u]);
          }
        }
        if constexpr (GX) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (ok[u]) {
              float y[V];
#pragma unroll
              for (int v = 0; v < V; ++v) y[v] = go[u][v] * r0.w;
              Vec<TX, V>::st(gx + (int64_t)r0.g * D + col[u], y);
#pragma unroll
              for (int v = 0; v < V; ++v) y[v] = go[u][v] * r1.w;
              Vec<TX, V>::st(gx + (int64_t)r1.g * D + col[u], y);
            }
          }
        }
        if constexpr (GW) {
          double d0 = 0.0, d1 = 0.0;
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float x[V];
            Vec<TX, V>::cvt(a[u], x);
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float xv = (FULL || ok[u]) ? x[v] : 0.f;
              d0 = __builtin_fma((double)xv, (double)go[u][v], d0);
            }
            Vec<TX, V>::cvt(b[u], x);
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float xv = (FULL || ok[u]) ? x[v] : 0.f;
              d1 = __builtin_fma((double)xv, (double)go[u][v], d1);
            }
          }
          d0 = wave_sum(d0);
          d1 = wave_sum(d1);
          if (lane == j - pb) mine += d0;
          if (lane == j + 1 - pb) mine += d1;
        }
      }
      if (j < pe) {
        const Rec r0 = rec[j];
        raw_t a[U];
        if constexpr (GW) {
#pragma unroll
          for (int u = 0; u < U; ++u) a[u] = load_x<TX, V, AL>(r0.src, cl[u]);
        }
        if constexpr (GX) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (ok[u]) {
              float y[V];
#pragma unroll
              for (int v = 0; v < V; ++v) y[v] = go[u][v] * r0.w;
              Vec<TX, V>::st(gx + (int64_t)r0.g * D + col[u], y);
            }
          }
        }
        if constexpr (GW) {
          double d0 = 0.0;
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float x[V];
            Vec<TX, V>::cvt(a[u], x);
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float xv = (FULL || ok[u]) ? x[v] : 0.f;
              d0 = __builtin_fma((double)xv, (double)go[u][v], d0);
            }
          }
          d0 = wave_sum(d0);
          if (lane == j - pb) mine += d0;
        }
      }
    }
    if constexpr (GW) {
      if (lane < pe - pb) store_gate(gw, gw_dtype, rec[pb + lane].g, mine);
    }
  }
}

template <typename TX, int V, int U, bool FULL, bool GX, bool GW>
__global__ __launch_bounds__(kGroup) void k_bwd(const int32_t* __restrict__ status,
                                                const int32_t* __restrict__ row_ptr,
                                                const Rec* __restrict__ rec,
                                                const TX* __restrict__ gout, int64_t gstride,
                                                TX* __restrict__ gx, void* __restrict__ gw,
                                                int gw_dtype, int64_t D, uint32_t T) {
  const uint32_t t = blockIdx.x * kWavesPerGroup + (uint32_t)uniform(threadIdx.x / kWave);
  if (t > T) return;
  if (t == T) {  // rows with an out-of-range scatter index: zero gradients
    const int lane = threadIdx.x & (kWave - 1);
    const int beg = row_ptr[t];
    const int end = row_ptr[t + 1];
    for (int j = beg; j < end; ++j) {
      const int64_t g = rec[j].g;
      if constexpr (GX) {
        float z[V];
#pragma unroll
        for (int v = 0; v < V; ++v) z[v] = 0.f;
        for (int64_t col = (int64_t)lane * V; col < D; col += (int64_t)kWave * V)
          Vec<TX, V>::st(gx + g * D + col, z);
      }
      if constexpr (GW) {
        if (lane == 0) store_gate(gw, gw_dtype, g, 0.0);
      }
    }
    return;
  }
  if (V > 1 && status[kStatusMisaligned] != 0)
    bwd_body<TX, V, U, FULL, GX, GW, false>(row_ptr, rec, gout, gstride, gx, gw, gw_dtype, D, t);
  else
    bwd_body<TX, V, U, FULL, GX, GW, true>(row_ptr, rec, gout, gstride, gx, gw, gw_dtype, D, t);
}

static int env_int_b(const char* name, int dflt) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : dflt;
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
  int64_t D, T;
  hipStream_t s;
};

template <typename TX, int V, int U, bool FULL, bool GX, bool GW>
static int launch_bwd_k(const BwdArgs& a) {
  const int64_t blocks = (a.T + 1 + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((k_bwd<TX, V, U, FULL, GX, GW>), dim3((unsigned)blocks), dim3(kGroup), 0, a.s,
                     a.status, a.row_ptr, a.rec, static_cast<const TX*>(a.gout), a.gstride,
                     static_cast<TX*>(a.gx), a.gw, a.gw_dtype, a.D, (uint32_t)a.T);
  return fmoe_host::check_launch("fmoe_combine_bwd");
}

template <typename TX, int V, int U, bool FULL>
static int launch_bwd_f(const BwdArgs& a) {
  if (a.gx && a.gw) return launch_bwd_k<TX, V, U, FULL, true, true>(a);
  if (a.gx) return launch_bwd_k<TX, V, U, FULL, true, false>(a);
  return launch_bwd_k<TX, V, U, FULL, false, true>(a);
}

template <typename TX, int V, int U>
static int launch_bwd_u(const BwdArgs& a) {
  if constexpr (V > 1) {
    if (a.D % ((int64_t)kWave * V * U) == 0) return launch_bwd_f<TX, V, U, true>(a);
  }
  return launch_bwd_f<TX, V, U, false>(a);
}

template <typename TX>
static int launch_bwd_x(const BwdArgs& a) {
  constexpr int V = vec16<TX>();
  const int eb = (int)sizeof(TX);
  const bool vec_ok = (a.D % V == 0) && ((uintptr_t)a.gout % 16 == 0) &&
                      ((a.gstride * eb) % 16 == 0) && ((uintptr_t)a.gx % 16 == 0) &&
                      env_int_b("FMOE_FORCE_SCALAR", 0) == 0;
  if (!vec_ok) return launch_bwd_u<TX, 1, 4>(a);
  int U = env_int_b("FMOE_BWD_U", 0);
  if (U != 1 && U != 2 && U != 4) {
    U = 1;
    for (int u = 4; u >= 1; u >>= 1)
      if (a.D % ((int64_t)kWave * V * u) == 0) { U = u; break; }
  }
  if (U == 4) return launch_bwd_u<TX, V, 4>(a);
  if (U == 2) return launch_bwd_u<TX, V, 2>(a);
  return launch_bwd_u<TX, V, 1>(a);
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
  FMOE_REQUIRE(gout_row_stride >= D, "fmoe_combine_bwd: grad_out row stride < D");
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
