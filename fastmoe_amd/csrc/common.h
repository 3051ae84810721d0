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
#include <type_traits>

#include "../../include/fastmoe_amd.h"
#include "options.h"

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

// Native clang vector types.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
#define FMOE_GLOBAL __attribute__((address_space(1)))

// ---- row access through buffer descriptors ---------------------------------------------------
// Every streamed row (an expert row, a grad_out / out / grad_X row) is addressed through a buffer
// resource whose base is the row start and whose num_records is the row length in bytes.  Lanes
// then use 32-bit byte offsets, the cache policy is an instruction immediate (non-temporal "nt"
// for streaming data: on MI355X ~7.1 TB/s reads and ~6.2 TB/s copies against ~6.4 / ~5.7 TB/s
// for the default policy), and the hardware range check makes tail columns free: loads beyond
// the row return 0 and stores beyond it are dropped, so no lane ever touches memory outside the
// row it was given.
#ifndef FMOE_NT
#define FMOE_NT 1
#endif
constexpr int kCPol = FMOE_NT ? 2 : 0;  // gfx950 cache-policy bit 1 = nt

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}
__device__ __forceinline__ rsrc_t make_rsrc(uint64_t base, uint32_t bytes) {
  return make_rsrc(reinterpret_cast<const void*>(base), bytes);
}

constexpr int kCPolCached = 0;  // default policy: keep in L2 / Infinity Cache (re-read data)

// Cache policies and backward workgroup shape (compile-time knobs; defaults measured best).
#ifndef FMOE_GX_CPOL
#define FMOE_GX_CPOL 2   // grad_X stores: non-temporal
#endif
#ifndef FMOE_GOUT_CPOL
#define FMOE_GOUT_CPOL 0 // grad_out loads: cached, shared by the rows of a token through L2
#endif
#ifndef FMOE_X_CPOL
#define FMOE_X_CPOL 2    // expert-row loads (read once): non-temporal
#endif
#ifndef FMOE_OUT_CPOL
#define FMOE_OUT_CPOL 16 // forward output stores: SC1 (device scope), temporal; the output stream
                         // is one k-th of the input stream, and keeping it out of the non-temporal
                         // path measured ~4% faster than nt at D=16384, top-8
#endif
#ifndef FMOE_BWD_WAVES
#define FMOE_BWD_WAVES 8 // waves per token workgroup of the backward (one row each at top-8)
#endif

template <int BYTES> struct Raw;
template <> struct Raw<32> {  // two 16-byte accesses (8 fp32 results of one 16-bit input vector)
  using type = u32x8;
  template <int CP = kCPol>
  static __device__ __forceinline__ type ld(rsrc_t r, uint32_t off) {
    const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CP));
    const u32x4 b =
        __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off + 16, 0, CP));
    return type{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, type v) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[0], v[1], v[2], v[3]}, r, (int)off, 0, CP);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[4], v[5], v[6], v[7]}, r, (int)off + 16, 0, CP);
  }
  static __device__ __forceinline__ uint32_t word(const type& v, int i) { return v[i]; }
};
template <> struct Raw<16> {
  using type = u32x4;
  template <int CP = kCPol>
  static __device__ __forceinline__ type ld(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(type, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CP));
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, type v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, CP);
  }
  static __device__ __forceinline__ uint32_t word(const type& v, int i) { return v[i]; }
};
template <> struct Raw<8> {
  using type = u32x2;
  template <int CP = kCPol>
  static __device__ __forceinline__ type ld(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(type, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, CP));
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, type v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, CP);
  }
  static __device__ __forceinline__ uint32_t word(const type& v, int i) { return v[i]; }
};
template <> struct Raw<4> {
  using type = uint32_t;
  template <int CP = kCPol>
  static __device__ __forceinline__ type ld(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, CP);
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, type v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, (int)off, 0, CP);
  }
  static __device__ __forceinline__ uint32_t word(const type& v, int) { return v; }
};
template <> struct Raw<2> {
  using type = uint16_t;
  template <int CP = kCPol>
  static __device__ __forceinline__ type ld(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, CP);
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, type v) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, (int)off, 0, CP);
  }
  static __device__ __forceinline__ uint32_t word(const type& v, int) { return v; }
};

// V consecutive elements of T: one buffer access of V * sizeof(T) bytes, widened to fp32 by cvt().
template <typename T, int V> struct Vec {
  static constexpr int kBytes = V * ElemInfo<T>::kBytes;
  using R = Raw<kBytes>;
  using raw_t = typename R::type;
  template <int CP = kCPol>
  static __device__ __forceinline__ raw_t ld(rsrc_t r, uint32_t off) {
    return R::template ld<CP>(r, off);
  }
  static __device__ __forceinline__ void cvt(const raw_t& raw, float* f) {
    if constexpr (ElemInfo<T>::kBytes == 4) {
#pragma unroll
      for (int v = 0; v < V; ++v) f[v] = __uint_as_float(R::word(raw, v));
    } else if constexpr (V == 1) {
      f[0] = std::is_same<T, bf16_t>::value ? __uint_as_float((uint32_t)raw << 16)
                                            : (float)__builtin_bit_cast(_Float16, (uint16_t)raw);
    } else {
#pragma unroll
      for (int v = 0; v < V; v += 2) {
        const uint32_t w = R::word(raw, v / 2);
        if constexpr (std::is_same<T, bf16_t>::value) {
          f[v] = bf16_lo(w);
          f[v + 1] = bf16_hi(w);
        } else {
          f[v] = f16_lo(w);
          f[v + 1] = f16_hi(w);
        }
      }
    }
  }
  static __device__ __forceinline__ raw_t pack(const float* f) {
    raw_t raw;
    if constexpr (ElemInfo<T>::kBytes == 4) {
      if constexpr (V == 1) {
        raw = __float_as_uint(f[0]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) raw[v] = __float_as_uint(f[v]);
      }
    } else if constexpr (V == 1) {
      raw = std::is_same<T, bf16_t>::value ? f32_to_bf16_bits(f[0]) : f32_to_f16_bits(f[0]);
    } else if constexpr (V == 2) {
      raw = std::is_same<T, bf16_t>::value ? pack_bf16x2(f[0], f[1]) : pack_f16x2(f[0], f[1]);
    } else {
#pragma unroll
      for (int v = 0; v < V; v += 2)
        raw[v / 2] = std::is_same<T, bf16_t>::value ? pack_bf16x2(f[v], f[v + 1])
                                                    : pack_f16x2(f[v], f[v + 1]);
    }
    return raw;
  }
  template <int CP = kCPol>
  static __device__ __forceinline__ void st(rsrc_t r, uint32_t off, const float* f) {
    R::template st<CP>(r, off, pack(f));
  }
};

// Elements per 16-byte load of T.
template <typename T> constexpr int vec16() { return 16 / ElemInfo<T>::kBytes; }

// Load of V elements of an expert row.  AL: the row start is 16-byte aligned (one vector
// access); otherwise V element accesses assembled into the same raw layout, so cvt() serves both.
template <typename TX, int V, bool AL>
__device__ __forceinline__ typename Vec<TX, V>::raw_t load_x(rsrc_t r, uint32_t off) {
  using VX = Vec<TX, V>;
  if constexpr (AL || V == 1) {
    return VX::template ld<FMOE_X_CPOL>(r, off);
  } else if constexpr (ElemInfo<TX>::kBytes == 4) {
    typename VX::raw_t raw;
#pragma unroll
    for (int v = 0; v < V; ++v) raw[v] = Raw<4>::ld(r, off + 4 * v);
    return raw;
  } else if constexpr (V == 2) {  // one 32-bit word of two 16-bit elements
    return (uint32_t)Raw<2>::ld(r, off) | ((uint32_t)Raw<2>::ld(r, off + 2) << 16);
  } else {
    typename VX::raw_t raw;
#pragma unroll
    for (int v = 0; v < V; v += 2)
      raw[v / 2] = (uint32_t)Raw<2>::ld(r, off + 2 * v) |
                   ((uint32_t)Raw<2>::ld(r, off + 2 * v + 2) << 16);
    return raw;
  }
}

// The (address, rows) table of up to 256 expert buffers as a kernel argument: the metadata kernel
// and the one-launch metadata + plan kernel read it straight from their arguments, so building
// the metadata needs no host staging buffer and no copy.
constexpr int kMetaChunk = 256;  // experts per launch: 256*8 + 256*4 + 16 bytes of arguments
struct MetaChunk {
  int64_t ptr[kMetaChunk];
  int32_t rows[kMetaChunk];
  int32_t count;  // experts in this chunk
  int32_t base;   // index of the first expert of this chunk
  int32_t scan;   // 1: this launch also scans (only when the whole table fits one chunk)
  int32_t pad;
};
static_assert(sizeof(MetaChunk) <= 3200, "kernel-argument table too large");

// Plan status words (int32, at the start of the plan workspace).
constexpr int kStatusInvalid = 0;    // rows whose scatter index is outside [0, T)
constexpr int kStatusMisaligned = 1; // nonzero if any source row is not 16-byte aligned
constexpr int kStatusLongest = 2;    // rows of the longest token segment


// Wave-uniform value: forces an SGPR so that dependent loads become scalar loads.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A batch of up to 64 plan records held one per lane; row i of the batch is read back as
// wave-uniform (SGPR) values with readlane, so the per-row metadata costs no memory latency.
struct LaneRecs {
  uint32_t src_lo, src_hi, w_bits;
  int32_t g;
  __device__ __forceinline__ void load(const Rec* __restrict__ rec, int first, int count, int lane) {
    if (lane < count) {
      const u32x4 v = *(const FMOE_GLOBAL u32x4*)(rec + first + lane);
      src_lo = v.x; src_hi = v.y; w_bits = v.z; g = (int32_t)v.w;
    } else {
      src_lo = src_hi = w_bits = 0; g = 0;
    }
  }
  __device__ __forceinline__ uint64_t src(int i) const {
    return (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)src_lo, i) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)src_hi, i) << 32);
  }
  __device__ __forceinline__ float w(int i) const {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)w_bits, i));
  }
  __device__ __forceinline__ int32_t row(int i) const { return __builtin_amdgcn_readlane(g, i); }
  // Reorder the `count` records to ascending g: each lane ranks its key against all others
  // (readlane broadcasts) and pushes its record to lane `rank` (ds_permute).  Equal keys (never
  // produced by a consistent plan) are ranked by lane, so the ranks always form a permutation and
  // every destination lane receives exactly one record.
  __device__ __forceinline__ void sort_by_row(int count, int lane) {
    const int key = lane < count ? g : 0x7fffffff;
    int rank = 0;
    for (int m = 0; m < count; ++m) {
      const int km = __builtin_amdgcn_readlane(key, m);
      rank += (km < key || (km == key && m < lane)) ? 1 : 0;
    }
    const int addr = rank * 4;  // lanes >= count all push to lane `count`, which is never read
    src_lo = (uint32_t)__builtin_amdgcn_ds_permute(addr, (int)src_lo);
    src_hi = (uint32_t)__builtin_amdgcn_ds_permute(addr, (int)src_hi);
    w_bits = (uint32_t)__builtin_amdgcn_ds_permute(addr, (int)w_bits);
    g = __builtin_amdgcn_ds_permute(addr, g);
  }
};

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

// ---- host-side error plumbing and kernel-variant options ------------------------------------
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
