/*
 * CPU oracle of the grouped weighted scatter-add (MoE combine) -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this; the product
 * path (fastmoe_amd) never does.  It is a scalar restatement of the reference's CPU algorithm:
 *
 *   forward  : src/fastmoe/kernels/ops.py:373-384 -- for each expert e in order, for each of its
 *              rows r in order (packed row g = off[e] + r), out[idx[g], :] += X_e[r, :] * w[g],
 *              where the product is computed and rounded in fp32 first (torch's `t * w[:, None]`
 *              promotes to fp32) and then added (torch's index_add_, ascending index order).
 *              Also the same order as run_on_cloud.py:17-20 (cat -> * w -> index_add_).
 *   backward : ops.py:344-353 -- grad_X[g, :] = round_x(f32(grad_out[idx[g], :]) * w[g]);
 *              the gate gradient (absent at ops.py:358-359) as the autograd of the same forward:
 *              grad_w[g] = sum_d grad_out[idx[g], d] * X[g, d], accumulated here in double.
 *   metadata : ops.py:233-256,268 -- offsets = exclusive cumsum of the row counts, max_rows.
 *   plan     : the token-major inverse of idx (CSR, ascending g per token, invalid rows last).
 *   permute  : src/fastmoe/models/tiny_model.py:108-138 -- slots i = t*k + j sorted by expert id
 *              (stable: a counting sort in ascending slot order, as torch.argsort(stable=True)),
 *              the reverse map rev[pos] = i / k (:121-125), counts = bincount (:138); ids outside
 *              [0, E) form one extra bucket after every expert.
 *
 * Element codes follow include/fastmoe_amd.h: 0 = f32, 1 = bf16, 2 = f16.  Out-of-range indices
 * are skipped and counted (the product drops them the same way).
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off (oracle/build.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- element conversions (round to nearest even, as torch's CPU casts) ---------------------- */
static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float oracle_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 (exact in fp32) */
    const float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  const uint32_t u = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (a < 0x38800000u) {
    /* result is subnormal or zero: round a * 2^24 to an integer, ties to even */
    const double v = (double)bits_to_f32(a) * 16777216.0; /* exact */
    double r = floor(v);
    const double frac = v - r;
    if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) != 0.0)) r += 1.0;
    return (uint16_t)(sign | (uint16_t)r); /* r may reach 0x400: smallest normal, still right */
  }
  /* normal: keep 10 mantissa bits of 23, round to nearest even on the 13 dropped bits */
  uint32_t m = a + 0xfffu + ((a >> 13) & 1u);
  m -= 0x38000000u; /* rebias exponent 127 -> 15 */
  return (uint16_t)(sign | (m >> 13));
}

static float load_f32(const void* base, int dtype, int64_t i) {
  if (dtype == 0) return ((const float*)base)[i];
  if (dtype == 1) return oracle_bf16_to_f32(((const uint16_t*)base)[i]);
  return oracle_f16_to_f32(((const uint16_t*)base)[i]);
}

static void store_f32(void* base, int dtype, int64_t i, float v) {
  if (dtype == 0) ((float*)base)[i] = v;
  else if (dtype == 1) ((uint16_t*)base)[i] = oracle_f32_to_bf16(v);
  else ((uint16_t*)base)[i] = oracle_f32_to_f16(v);
}

/* Round an fp32 array to `dtype` in place semantics: dst[i] = round(src[i]). */
void oracle_round_f32(const float* src, int64_t n, int dtype, void* dst) {
  for (int64_t i = 0; i < n; ++i) store_f32(dst, dtype, i, src[i]);
}

/* Widen any element type to fp32. */
void oracle_widen_f32(const void* src, int64_t n, int dtype, float* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = load_f32(src, dtype, i);
}

/* ---- metadata (ops.py:233-256, 268) ------------------------------------------------------- */
int64_t oracle_metadata(const int64_t* rows, int64_t E, int64_t* offsets, int64_t* max_rows) {
  int64_t acc = 0, mx = 0;
  for (int64_t e = 0; e < E; ++e) {
    offsets[e] = acc;
    acc += rows[e];
    if (rows[e] > mx) mx = rows[e];
  }
  offsets[E] = acc;
  *max_rows = mx;
  return acc;
}

/* ---- forward (ops.py:373-384) -------------------------------------------------------------
 * acc[T * D] (fp32) is accumulated in place: pass zeros for the reference's fresh output, or the
 * widened existing out for the in-place (accumulate) contract.  Returns the number of skipped
 * (out-of-range) rows. */
int64_t oracle_combine_fwd(const void* const* xs, const int64_t* rows, int64_t E, int x_dtype,
                           const int64_t* idx, const float* w, int64_t T, int64_t D, float* acc) {
  int64_t g = 0, bad = 0;
  for (int64_t e = 0; e < E; ++e) {
    for (int64_t r = 0; r < rows[e]; ++r, ++g) {
      const int64_t t = idx[g];
      if (t < 0 || t >= T) {
        ++bad;
        continue;
      }
      const float wg = w[g];
      float* o = acc + t * D;
      for (int64_t d = 0; d < D; ++d) {
        const float p = load_f32(xs[e], x_dtype, r * D + d) * wg; /* rounded fp32 product */
        o[d] = o[d] + p;
      }
    }
  }
  return bad;
}

/* ---- backward (ops.py:344-353 + the gate gradient) ----------------------------------------
 * grad_out is [T, D] in x_dtype.  grad_x ([N, D], x_dtype) and grad_w ([N], double) may be NULL.
 * Rows with an out-of-range index get zero gradients. */
void oracle_combine_bwd(const void* const* xs, const int64_t* rows, int64_t E, int x_dtype,
                        const int64_t* idx, const float* w, int64_t T, int64_t D,
                        const void* grad_out, void* grad_x, double* grad_w) {
  int64_t g = 0;
  for (int64_t e = 0; e < E; ++e) {
    for (int64_t r = 0; r < rows[e]; ++r, ++g) {
      const int64_t t = idx[g];
      const int valid = t >= 0 && t < T;
      double dot = 0.0;
      for (int64_t d = 0; d < D; ++d) {
        const float go = valid ? load_f32(grad_out, x_dtype, t * D + d) : 0.0f;
        /* an out-of-range row's gradient is +0, whatever the sign of its gate */
        if (grad_x) store_f32(grad_x, x_dtype, g * D + d, valid ? go * w[g] : 0.0f);
        if (grad_w && valid) dot += (double)go * (double)load_f32(xs[e], x_dtype, r * D + d);
      }
      if (grad_w) grad_w[g] = dot;
    }
  }
}

/* ---- plan: token-major inverse of idx ----------------------------------------------------
 * row_ptr[T + 2]: segment b = [row_ptr[b], row_ptr[b+1]) lists the packed rows g with idx[g] == b
 * in ascending g; segment T lists the rows with an out-of-range index.  g_list[N]. */
void oracle_plan(const int64_t* idx, int64_t N, int64_t T, int32_t* row_ptr, int32_t* g_list) {
  int64_t* cnt = (int64_t*)calloc((size_t)(T + 1), sizeof(int64_t));
  for (int64_t g = 0; g < N; ++g) {
    const int64_t t = idx[g];
    cnt[(t >= 0 && t < T) ? t : T] += 1;
  }
  int64_t run = 0;
  for (int64_t b = 0; b <= T; ++b) {
    row_ptr[b] = (int32_t)run;
    const int64_t c = cnt[b];
    cnt[b] = run; /* becomes the fill cursor */
    run += c;
  }
  row_ptr[T + 1] = (int32_t)run;
  for (int64_t g = 0; g < N; ++g) { /* ascending g: each segment comes out sorted */
    const int64_t t = idx[g];
    const int64_t b = (t >= 0 && t < T) ? t : T;
    g_list[cnt[b]++] = (int32_t)g;
  }
  free(cnt);
}

/* ---- dispatch permutation (tiny_model.py:108-138) ------------------------------------------
 * ids[T * k] -> counts[E], offsets[E + 1] (offsets[E] = valid slots), rev[N] (token of each packed
 * row), slot_pos[N] (packed row of each slot).  Returns the number of slots whose id lies outside
 * [0, E). */
int64_t oracle_permute(const int64_t* ids, int64_t T, int64_t k, int64_t E, int64_t* counts,
                       int64_t* offsets, int64_t* rev, int32_t* slot_pos) {
  const int64_t N = T * k;
  int64_t* cur = (int64_t*)calloc((size_t)(E + 1), sizeof(int64_t));
  for (int64_t i = 0; i < N; ++i) {
    const int64_t e = ids[i];
    cur[(e >= 0 && e < E) ? e : E] += 1;
  }
  int64_t run = 0;
  for (int64_t e = 0; e <= E; ++e) {
    const int64_t c = cur[e];
    if (e < E) {
      counts[e] = c;
      offsets[e] = run;
    } else {
      offsets[E] = run;
    }
    cur[e] = run;
    run += c;
  }
  const int64_t bad = N - offsets[E];
  for (int64_t i = 0; i < N; ++i) { /* ascending slot order: a stable sort */
    const int64_t e = ids[i];
    const int64_t pos = cur[(e >= 0 && e < E) ? e : E]++;
    rev[pos] = i / k;
    slot_pos[i] = (int32_t)pos;
  }
  free(cur);
  return bad;
}
