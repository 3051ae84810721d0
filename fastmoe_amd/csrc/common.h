// Shared device helpers and host-side error plumbing for the gfx950 combine kernels.
//
// Element conversion rules (all round-to-nearest-even, matching torch's CPU casts):
//   bf16 -> f32 : exact (bits << 16)
//   f16  -> f32 : exact (v_cvt_f32_f16)
//   f32  -> bf16: v_cvt_pk_bf16_f32 (gfx950 hardware RNE)
//   f32  -> f16 : v_cvt_f16_f32 (RNE)
// Floating-point contraction is disabled for every kernel (-ffp-contract=off plus the pragma
// below): the forward multiplies x*w in fp32, rounds, then adds, exactly like torch's CPU
// `t * w` followed by `index_add_`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/fastmoe_amd.h"

#pragma clang fp contract(off)

namespace fmoe {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kWavesPerGroup = 4;  // every kernel here runs 256-thread workgroups of 4 waves
constexpr int kGroup = kWave * kWavesPerGroup;

// One routed row in token-major order: where its expert row lives, its gate (converted to fp32)
// and its packed-row number g.  16 bytes so that a wave fetches it with one scalar load.
struct __attribute__((aligned(16))) Rec {
  uint64_t src;  // device address of X_e[g - off[e], 0]
  float w;       // gate weight, fp32
  int32_t g;     // packed row number
};
static_assert(sizeof(Rec) == 16, "Rec must be 16 bytes");

// Storage tags for 16-bit floats (plain uint16 payloads).
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename T> struct ElemInfo;
template <> struct ElemInfo<float> { static constexpr int kBytes = 4; };
template <> struct ElemInfo<bf16_t> { static constexpr int kBytes = 2; };
template <> struct ElemInfo<f16_t> { static constexpr int kBytes = 2; };

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float f16_lo(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// ---- scalar element access -------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ld1(const T* p);
template <> __device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld1<bf16_t>(const bf16_t* p) {
  return __uint_as_float((uint32_t)p->bits << 16);
}
template <> __device__ __forceinline__ float ld1<f16_t>(const f16_t* p) {
  return (float)__builtin_bit_cast(_Float16, p->bits);
}
template <typename T> __device__ __forceinline__ void st1(T* p, float v);
template <> __device__ __forceinline__ void st1<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void st1<bf16_t>(bf16_t* p, float v) {
  p->bits = f32_to_bf16_bits(v);
}
template <> __device__ __forceinline__ void st1<f16_t>(f16_t* p, float v) {
  p->bits = f32_to_f16_bits(v);
}

// ---- vector access: V elements starting at p ------------------------------------------------
// ld() issues one global load of the raw storage (16 bytes per lane for V == 16/sizeof(T)),
// cvt() widens it to fp32 later, so that many loads can be in flight before the first use.
// V == 1 is the unaligned scalar path.
#define FMOE_GLOBAL __attribute__((address_space(1)))

// Native clang vector types: they load/store through address-space-1 pointers directly.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename R, typename T>
__device__ __forceinline__ R gload(const T* p) {
  return *(const FMOE_GLOBAL R*)(p);
}
template <typename R, typename T>
__device__ __forceinline__ void gstore(T* p, R v) {
  *(FMOE_GLOBAL R*)(p) = v;
}

template <typename T, int V> struct Vec;

template <> struct Vec<float, 1> {
  using raw_t = float;
  static __device__ __forceinline__ raw_t ld(const float* p) { return gload<float>(p); }
  static __device__ __forceinline__ void cvt(raw_t r, float* f) { f[0] = r; }
  static __device__ __forceinline__ void st(float* p, const float* f) { gstore<float>(p, f[0]); }
};
template <> struct Vec<bf16_t, 1> {
  using raw_t = uint16_t;
  static __device__ __forceinline__ raw_t ld(const bf16_t* p) { return gload<uint16_t>(p); }
  static __device__ __forceinline__ void cvt(raw_t r, float* f) {
    f[0] = __uint_as_float((uint32_t)r << 16);
  }
  static __device__ __forceinline__ void st(bf16_t* p, const float* f) {
    gstore<uint16_t>(p, f32_to_bf16_bits(f[0]));
  }
};
template <> struct Vec<f16_t, 1> {
  using raw_t = uint16_t;
  static __device__ __forceinline__ raw_t ld(const f16_t* p) { return gload<uint16_t>(p); }
  static __device__ __forceinline__ void cvt(raw_t r, float* f) {
    f[0] = (float)__builtin_bit_cast(_Float16, r);
  }
  static __device__ __forceinline__ void st(f16_t* p, const float* f) {
    gstore<uint16_t>(p, f32_to_f16_bits(f[0]));
  }
};

template <> struct Vec<float, 4> {
  using raw_t = f32x4;
  static __device__ __forceinline__ raw_t ld(const float* p) { return gload<f32x4>(p); }
  static __device__ __forceinline__ void cvt(const raw_t& v, float* f) {
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
  static __device__ __forceinline__ void st(float* p, const float* f) {
    gstore<f32x4>(p, f32x4{f[0], f[1], f[2], f[3]});
  }
};
template <> struct Vec<float, 8> {  // output side only (8 fp32 results of one 16-bit input vector)
  static __device__ __forceinline__ void ld_cvt(const float* p, float* f) {
    Vec<float, 4>::cvt(Vec<float, 4>::ld(p), f);
    Vec<float, 4>::cvt(Vec<float, 4>::ld(p + 4), f + 4);
  }
  static __device__ __forceinline__ void st(float* p, const float* f) {
    Vec<float, 4>::st(p, f);
    Vec<float, 4>::st(p + 4, f + 4);
  }
};
template <> struct Vec<bf16_t, 8> {
  using raw_t = u32x4;
  static __device__ __forceinline__ raw_t ld(const bf16_t* p) { return gload<u32x4>(p); }
  static __device__ __forceinline__ void cvt(const raw_t& v, float* f) {
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
  }
  static __device__ __forceinline__ void st(bf16_t* p, const float* f) {
    u32x4 v;
    v.x = pack_bf16x2(f[0], f[1]); v.y = pack_bf16x2(f[2], f[3]);
    v.z = pack_bf16x2(f[4], f[5]); v.w = pack_bf16x2(f[6], f[7]);
    gstore<u32x4>(p, v);
  }
};
template <> struct Vec<bf16_t, 4> {  // output side of a 4-wide fp32 input vector
  static __device__ __forceinline__ void ld_cvt(const bf16_t* p, float* f) {
    const u32x2 v = gload<u32x2>(p);
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  }
  static __device__ __forceinline__ void st(bf16_t* p, const float* f) {
    u32x2 v;
    v.x = pack_bf16x2(f[0], f[1]); v.y = pack_bf16x2(f[2], f[3]);
    gstore<u32x2>(p, v);
  }
};
template <> struct Vec<f16_t, 8> {
  using raw_t = u32x4;
  static __device__ __forceinline__ raw_t ld(const f16_t* p) { return gload<u32x4>(p); }
  static __device__ __forceinline__ void cvt(const raw_t& v, float* f) {
    f[0] = f16_lo(v.x); f[1] = f16_hi(v.x); f[2] = f16_lo(v.y); f[3] = f16_hi(v.y);
    f[4] = f16_lo(v.z); f[5] = f16_hi(v.z); f[6] = f16_lo(v.w); f[7] = f16_hi(v.w);
  }
  static __device__ __forceinline__ void st(f16_t* p, const float* f) {
    u32x4 v;
    v.x = pack_f16x2(f[0], f[1]); v.y = pack_f16x2(f[2], f[3]);
    v.z = pack_f16x2(f[4], f[5]); v.w = pack_f16x2(f[6], f[7]);
    gstore<u32x4>(p, v);
  }
};
template <> struct Vec<f16_t, 4> {
  static __device__ __forceinline__ void ld_cvt(const f16_t* p, float* f) {
    const u32x2 v = gload<u32x2>(p);
    f[0] = f16_lo(v.x); f[1] = f16_hi(v.x); f[2] = f16_lo(v.y); f[3] = f16_hi(v.y);
  }
  static __device__ __forceinline__ void st(f16_t* p, const float* f) {
    u32x2 v;
    v.x = pack_f16x2(f[0], f[1]); v.y = pack_f16x2(f[2], f[3]);
    gstore<u32x2>(p, v);
  }
};

// Output-side load of V elements widened to fp32 (for accumulate-into-out).
template <typename T, int V>
__device__ __forceinline__ void ld_cvt_out(const T* p, float* f) {
  if constexpr (V == 1 || (V == 4 && sizeof(T) == 4) || (V == 8 && sizeof(T) == 2)) {
    Vec<T, V>::cvt(Vec<T, V>::ld(p), f);
  } else {
    Vec<T, V>::ld_cvt(p, f);
  }
}

// Raw load of V elements of an expert row.  AL: the row address is 16-byte aligned (vector
// load); otherwise V element loads packed into the same raw layout, so cvt() serves both.
template <typename TX, int V, bool AL>
__device__ __forceinline__ typename Vec<TX, V>::raw_t load_x(uint64_t src, int64_t col) {
  const TX* p = reinterpret_cast<const TX*>(src) + col;
  if constexpr (AL || V == 1) {
    return Vec<TX, V>::ld(p);
  } else if constexpr (sizeof(TX) == 4) {
    f32x4 r;
    r.x = gload<float>(p); r.y = gload<float>(p + 1);
    r.z = gload<float>(p + 2); r.w = gload<float>(p + 3);
    return r;
  } else {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    u32x4 r;
    r.x = (uint32_t)gload<uint16_t>(q + 0) | ((uint32_t)gload<uint16_t>(q + 1) << 16);
    r.y = (uint32_t)gload<uint16_t>(q + 2) | ((uint32_t)gload<uint16_t>(q + 3) << 16);
    r.z = (uint32_t)gload<uint16_t>(q + 4) | ((uint32_t)gload<uint16_t>(q + 5) << 16);
    r.w = (uint32_t)gload<uint16_t>(q + 6) | ((uint32_t)gload<uint16_t>(q + 7) << 16);
    return r;
  }
}

// Plan status words (int32, at the start of the plan workspace).
constexpr int kStatusInvalid = 0;    // rows whose scatter index is outside [0, T)
constexpr int kStatusMisaligned = 1; // nonzero if any source row is not 16-byte aligned

// Elements per 16-byte load of T.
template <typename T> constexpr int vec16() { return 16 / ElemInfo<T>::kBytes; }

// Wave-uniform value: forces an SGPR so that dependent loads become scalar loads.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Runtime-typed loads of the small per-row arrays (wave-uniform dtype switch).
__device__ __forceinline__ float load_weight(const void* w, int dtype, int64_t i) {
  if (dtype == FMOE_F32) return static_cast<const float*>(w)[i];
  if (dtype == FMOE_BF16) return ld1(static_cast<const bf16_t*>(w) + i);
  return ld1(static_cast<const f16_t*>(w) + i);
}
__device__ __forceinline__ int64_t load_index(const void* idx, int dtype, int64_t i) {
  if (dtype == FMOE_I64) return static_cast<const int64_t*>(idx)[i];
  return (int64_t) static_cast<const int32_t*>(idx)[i];
}

// Largest e in [0, E) with off[e] <= g, given off[0] == 0 <= g < off[E].  Empty experts share
// their offset with the next expert, so the result is always a non-empty expert.
__device__ __forceinline__ int64_t expert_of_row(const int64_t* __restrict__ off, int64_t E,
                                                 int64_t g) {
  int64_t lo = 0, hi = E;  // invariant: off[lo] <= g < off[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (off[mid] <= g) lo = mid; else hi = mid;
  }
  return lo;
}

}  // namespace fmoe

// ---- host-side error plumbing ---------------------------------------------------------------
namespace fmoe_host {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

inline int dtype_bytes(int dt) {
  switch (dt) {
    case FMOE_F32: return 4;
    case FMOE_BF16: return 2;
    case FMOE_F16: return 2;
    case FMOE_I64: return 8;
    case FMOE_I32: return 4;
    default: return 0;
  }
}
inline bool is_float_dtype(int dt) { return dt == FMOE_F32 || dt == FMOE_BF16 || dt == FMOE_F16; }
inline bool is_index_dtype(int dt) { return dt == FMOE_I64 || dt == FMOE_I32; }

// Check the launch that was just enqueued.
inline int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return FMOE_EHIP;
  }
  return FMOE_OK;
}

inline int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

}  // namespace fmoe_host

#define FMOE_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      fmoe_host::set_error(__VA_ARGS__); \
      return FMOE_EINVAL;                \
    }                                    \
  } while (0)
