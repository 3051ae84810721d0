// Dispatch-side permutation of the MoE layer: routing slots grouped by expert.
//
// Replaces the sort-and-gather half of MoEFeedForward.gate_and_sort
// (src/fastmoe/models/tiny_model.py:108-138): argsort of the flattened top-k expert ids (:112),
// the reverse map of packed row -> token (:121-125), the gates in packed order (:128), the gather
// x_flat[reverse_map_indices] (:133) and the per-expert bincount (:138).  The packed order is the
// stable one: rows of one expert keep ascending slot order (token-major), which is what
// torch.argsort(..., stable=True) gives; the reference's unstable argsort (:112) leaves the order
// of equal ids unspecified.
//
// Slot i = t * k + j is token t's j-th routing choice.  Steps (caller's stream, no host sync):
//   1. rank    one workgroup per block of 1024 slots (256 when E > 1024): each slot's stable rank among the
//              block's slots of the same expert (wave ballots on the key bits give the lanes of
//              a wave with an equal key; per-wave counts in LDS give the waves before it), and
//              the block's count of every expert (row b of blkcnt[nb][E + 1]).
//   2. scan    one 1024-thread workgroup: per expert, exclusive prefix over the blocks (in place,
//              through LDS tiles), then the exclusive prefix over experts of the totals -> offsets.
//   3. fill    one thread per slot: pos = off[e] + blkcnt[b][e] + rank; writes the reverse map,
//              the gate in packed order and the slot -> row map (slot_pos).
//   4. gather  one workgroup per token: its waves copy x[t] into the token's k packed rows (the row
//              is read once from HBM and shared through L2; the copies are streaming stores).
// An expert id outside [0, E) is key E: such slots go to the tail, after every expert's rows, and
// are counted in the status word; counts/offsets cover the valid slots only.
#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace fmoe {

// Slots per ranking block: 1024 (16 waves) while the per-wave expert counters fit in 64 KiB of
// LDS (E <= 1024), else 256 (4 waves).  Bigger blocks keep the block-count table small for the scan.
constexpr int kPermBlockLarge = 1024;
constexpr int kPermBlockSmall = kGroup;
constexpr int kPermMaxExperts = 4096;     // 4 waves x 4097 per-wave counters: 64 KiB of LDS
constexpr int kPermSmallExperts = 1024;   // 16 waves x 1025 per-wave counters: 64 KiB of LDS
constexpr int kPermScanThreads = 1024;
constexpr int kPermGatherWaves = 8;

// Workspace: blkcnt[nb][E + 1] (per-block counts, then per-block prefixes), rank[N] (stable rank
// of each slot inside its block and expert), off[E + 1] (first packed row of each key).
struct PermLayout {
  int64_t blkcnt, rank, off, total;
};

__host__ __device__ inline int perm_block(int64_t E) {
  return E <= kPermSmallExperts ? kPermBlockLarge : kPermBlockSmall;
}

__host__ __device__ inline PermLayout perm_layout(int64_t N, int64_t E) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int blk = perm_block(E);
  const int64_t nb = (N + blk - 1) / blk;
  PermLayout L;
  L.blkcnt = 0;
  L.rank = L.blkcnt + up(nb * (E + 1) * 4);
  L.off = L.rank + up(N * 4);
  L.total = L.off + up((E + 1) * 4);
  return L;
}

// Key of slot i: its expert id, or E when the id lies outside [0, E).
template <typename TI>
__device__ __forceinline__ int slot_key(const TI* __restrict__ ids, int64_t i, int64_t E) {
  const int64_t e = (int64_t)ids[i];
  return (e >= 0 && e < E) ? (int)e : (int)E;
}

template <typename TI, int MAXE, int BLK>
__global__ __launch_bounds__(BLK) void k_perm_rank(const TI* __restrict__ ids, int64_t N,
                                                   int64_t E, int key_bits,
                                                   int32_t* __restrict__ blkcnt,
                                                   int32_t* __restrict__ rank) {
  constexpr int W = BLK / kWave;
  __shared__ int32_t wcnt[W][MAXE + 1];
  const int E1 = (int)E + 1;
  for (int w = 0; w < W; ++w)
    for (int k = threadIdx.x; k < E1; k += BLK) wcnt[w][k] = 0;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int64_t i = (int64_t)blockIdx.x * BLK + threadIdx.x;
  const bool live = i < N;
  const int key = live ? slot_key(ids, i, E) : 0;
  // lanes of this wave holding the same key (dead lanes excluded)
  uint64_t same = __ballot(live);
  for (int bit = 0; bit < key_bits; ++bit) {
    const int set = (key >> bit) & 1;
    const uint64_t m = __ballot(set);
    same &= set ? m : ~m;
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  const int in_wave = __popcll(same & below);
  __syncthreads();
  if (live && in_wave == 0) wcnt[wv][key] = __popcll(same);
  __syncthreads();
  if (live) {
    int before = in_wave;
    for (int w = 0; w < wv; ++w) before += wcnt[w][key];
    rank[i] = before;
  }
  int32_t* row = blkcnt + (int64_t)blockIdx.x * E1;
  for (int k = threadIdx.x; k < E1; k += BLK) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) c += wcnt[w][k];
    row[k] = c;
  }
}

// Per expert, exclusive prefix of blkcnt down the nb blocks (in place); then offsets over experts.
// The table is walked in tiles of whole block rows staged in LDS: a coalesced load of the tile,
// one thread per expert column scanning it in LDS (consecutive threads, consecutive words: no
// bank conflicts) with a carry kept in registers across tiles, and a coalesced store back.
constexpr int kPermTileInts = 32768;                      // 128 KiB of LDS per tile
constexpr int kPermKeysPerThread = (kPermMaxExperts + 1 + kPermScanThreads - 1) / kPermScanThreads;

__global__ __launch_bounds__(kPermScanThreads) void k_perm_scan(
    int32_t* __restrict__ blkcnt, int64_t nb, int64_t E, int32_t* __restrict__ off,
    int64_t* __restrict__ counts, int64_t* __restrict__ offsets, int32_t* __restrict__ status) {
  __shared__ int32_t tile[kPermTileInts];
  __shared__ int32_t tot[kPermMaxExperts + 1];
  const int E1 = (int)E + 1;
  const int rows_per_tile = kPermTileInts / E1;  // >= 7 for E1 <= 4097
  int carry[kPermKeysPerThread];
#pragma unroll
  for (int m = 0; m < kPermKeysPerThread; ++m) carry[m] = 0;
  for (int64_t r0 = 0; r0 < nb; r0 += rows_per_tile) {
    const int rows = (int)std::min<int64_t>(rows_per_tile, nb - r0);
    const int n = rows * E1;
    int32_t* g = blkcnt + r0 * E1;
    constexpr int kBatch = 8;  // independent global loads in flight per thread
    for (int base = 0; base < n; base += kPermScanThreads * kBatch) {
      int v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = base + j * kPermScanThreads + (int)threadIdx.x;
        v[j] = i < n ? g[i] : 0;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = base + j * kPermScanThreads + (int)threadIdx.x;
        if (i < n) tile[i] = v[j];
      }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kPermKeysPerThread; ++m) {
      const int k = (int)threadIdx.x + m * kPermScanThreads;
      if (k < E1) {
        int run = carry[m];
        for (int r = 0; r < rows; ++r) {
          const int v = tile[r * E1 + k];
          tile[r * E1 + k] = run;
          run += v;
        }
        carry[m] = run;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kPermScanThreads) g[i] = tile[i];
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < kPermKeysPerThread; ++m) {
    const int k = (int)threadIdx.x + m * kPermScanThreads;
    if (k < E1) tot[k] = carry[m];
  }
  __syncthreads();
  // exclusive prefix over the E + 1 keys (serial chunks of 1024 with a carried total)
  __shared__ int32_t carry_s;
  __shared__ int32_t wave_tot[kPermScanThreads / kWave];
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  for (int kb = 0; kb < E1; kb += kPermScanThreads) {
    const int k = kb + (int)threadIdx.x;
    const int v = k < E1 ? tot[k] : 0;
    int incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) wave_tot[wv] = incl;
    __syncthreads();
    int before = carry_s, all = 0;
#pragma unroll
    for (int w = 0; w < kPermScanThreads / kWave; ++w) {
      before += (w < wv) ? wave_tot[w] : 0;
      all += wave_tot[w];
    }
    const int excl = before + incl - v;
    if (k < E1) {
      off[k] = excl;
      if (k < (int)E) {
        counts[k] = v;
        offsets[k] = excl;
      } else {
        offsets[E] = excl;                     // rows of valid slots
        status[0] = v;                         // slots with an id outside [0, E)
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) carry_s += all;
    __syncthreads();
  }
}

template <typename TI, typename TG>
__global__ __launch_bounds__(kGroup) void k_perm_fill(const TI* __restrict__ ids,
                                                      const TG* __restrict__ gates, int64_t N,
                                                      int64_t E, int64_t k, int blk,
                                                      const int32_t* __restrict__ blkcnt,
                                                      const int32_t* __restrict__ rank,
                                                      const int32_t* __restrict__ off,
                                                      int64_t* __restrict__ rev,
                                                      TG* __restrict__ sorted_gates,
                                                      int32_t* __restrict__ slot_pos) {
  const int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x;
  if (i >= N) return;
  const int key = slot_key(ids, i, E);
  const int64_t b = i / blk;
  const int pos = off[key] + blkcnt[b * (E + 1) + key] + rank[i];
  if (pos < 0 || pos >= N) return;  // unreachable for a consistent rank/scan; never write outside
  rev[pos] = i / k;
  sorted_gates[pos] = gates[i];
  slot_pos[i] = pos;
}

// Row copy x[t] -> out[slot_pos[t * k + j]] for j < k, VB bytes per lane access.
template <int VB>
__global__ __launch_bounds__(kPermGatherWaves * kWave) void k_perm_gather(
    const int32_t* __restrict__ slot_pos, int64_t k, const uint8_t* __restrict__ x,
    int64_t x_stride_bytes, uint8_t* __restrict__ out, uint32_t row_bytes, int64_t N) {
  constexpr int U = VB == 16 ? 8 : 4;  // accesses in flight per lane
  using R = Raw<VB>;
  using raw_t = typename R::type;
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform(threadIdx.x / kWave);
  const rsrc_t rs = make_rsrc(x + t * x_stride_bytes, row_bytes);
  for (int64_t j = wave; j < k; j += kPermGatherWaves) {
    const int64_t pos = slot_pos[t * k + j];
    if (pos < 0 || pos >= N) continue;  // slot_pos comes from fmoe_permute_build: always in range
    const rsrc_t rd = make_rsrc(out + pos * (int64_t)row_bytes, row_bytes);
    for (uint32_t base = 0; base < row_bytes; base += (uint32_t)(kWave * VB * U)) {
      raw_t v[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        v[u] = R::template ld<kCPolCached>(rs, base + (uint32_t)(u * kWave + lane) * VB);
#pragma unroll
      for (int u = 0; u < U; ++u)  // bytes past the row: dropped by the range check
        R::template st<kCPol>(rd, base + (uint32_t)(u * kWave + lane) * VB, v[u]);
    }
  }
}

// grad_gates[i] = grad_sorted[slot_pos[i]] (element copy, any 2- or 4-byte dtype).
template <typename T>
__global__ __launch_bounds__(kGroup) void k_perm_gate_grad(const int32_t* __restrict__ slot_pos,
                                                           int64_t N, const T* __restrict__ src,
                                                           T* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * kGroup + threadIdx.x;
  if (i >= N) return;
  const int32_t p = slot_pos[i];
  dst[i] = (p >= 0 && p < N) ? src[p] : T{};
}

}  // namespace fmoe

using namespace fmoe;

extern "C" int64_t fmoe_permute_workspace_bytes(int64_t num_slots, int64_t num_experts) {
  if (num_slots < 0 || num_experts < 1) return -1;
  return perm_layout(num_slots, num_experts).total;
}

extern "C" int fmoe_permute_build(const void* d_expert_ids, int id_dtype, const void* d_gates,
                                  int gate_dtype, int64_t num_tokens, int64_t top_k,
                                  int64_t num_experts, int64_t* d_counts, int64_t* d_offsets,
                                  int64_t* d_rev, void* d_sorted_gates, int32_t* d_slot_pos,
                                  int32_t* d_status, void* d_workspace, void* stream) {
  fmoe_host::clear_error();
  const int64_t T = num_tokens, K = top_k, E = num_experts;
  FMOE_REQUIRE(T >= 0 && K >= 1, "fmoe_permute_build: bad sizes T=%lld k=%lld", (long long)T,
               (long long)K);
  FMOE_REQUIRE(E >= 1 && E <= kPermMaxExperts,
               "fmoe_permute_build: num_experts %lld not in [1, %d]", (long long)E,
               kPermMaxExperts);
  if (K >= (int64_t(1) << 31) || (T > 0 && K > ((int64_t(1) << 31) - 1) / T)) {
    fmoe_host::set_error("fmoe_permute_build: T*k exceeds the 32-bit row counters");
    return FMOE_ERANGE;
  }
  const int64_t N = T * K;
  const int blk = perm_block(E);
  const int64_t nb = (N + blk - 1) / blk;
  if (nb * (E + 1) >= (int64_t(1) << 31)) {
    fmoe_host::set_error("fmoe_permute_build: block count table too large");
    return FMOE_ERANGE;
  }
  FMOE_REQUIRE(fmoe_host::is_index_dtype(id_dtype), "fmoe_permute_build: bad id dtype %d",
               id_dtype);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(gate_dtype), "fmoe_permute_build: bad gate dtype %d",
               gate_dtype);
  FMOE_REQUIRE(d_counts && d_offsets && d_status && d_workspace,
               "fmoe_permute_build: null device pointer");
  FMOE_REQUIRE(N == 0 || (d_expert_ids && d_gates && d_rev && d_sorted_gates && d_slot_pos),
               "fmoe_permute_build: null ids/gates/outputs");
  FMOE_REQUIRE(((uintptr_t)d_workspace & 255) == 0,
               "fmoe_permute_build: workspace not 256B-aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const PermLayout L = perm_layout(N, E);
  char* ws = static_cast<char*>(d_workspace);
  int32_t* blkcnt = reinterpret_cast<int32_t*>(ws + L.blkcnt);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* off = reinterpret_cast<int32_t*>(ws + L.off);
  int key_bits = 0;
  while ((int64_t(1) << key_bits) <= E) ++key_bits;  // keys lie in [0, E]
  if (N > 0) {
#define FMOE_PRANK(TI, MAXE, BLK)                                                                  \
  hipLaunchKernelGGL((k_perm_rank<TI, MAXE, BLK>), dim3((unsigned)nb), dim3(BLK), 0, s,            \
                     static_cast<const TI*>(d_expert_ids), N, E, key_bits, blkcnt, rank)
    if (id_dtype == FMOE_I64) {
      if (blk == kPermBlockLarge) FMOE_PRANK(int64_t, kPermSmallExperts, kPermBlockLarge);
      else FMOE_PRANK(int64_t, kPermMaxExperts, kPermBlockSmall);
    } else {
      if (blk == kPermBlockLarge) FMOE_PRANK(int32_t, kPermSmallExperts, kPermBlockLarge);
      else FMOE_PRANK(int32_t, kPermMaxExperts, kPermBlockSmall);
    }
#undef FMOE_PRANK
    if (int rc = fmoe_host::check_launch("fmoe_permute_build(rank)")) return rc;
  }
  hipLaunchKernelGGL(k_perm_scan, dim3(1), dim3(kPermScanThreads), 0, s, blkcnt, nb, E, off,
                     d_counts, d_offsets, d_status);
  if (int rc = fmoe_host::check_launch("fmoe_permute_build(scan)")) return rc;
  if (N == 0) return FMOE_OK;
  const dim3 grid((unsigned)((N + kGroup - 1) / kGroup));
  const bool g4 = fmoe_host::dtype_bytes(gate_dtype) == 4;
#define FMOE_PFILL(TI, TG)                                                                         \
  hipLaunchKernelGGL((k_perm_fill<TI, TG>), grid, dim3(kGroup), 0, s,                              \
                     static_cast<const TI*>(d_expert_ids), static_cast<const TG*>(d_gates), N, E,  \
                     K, blk, blkcnt, rank, off, d_rev, static_cast<TG*>(d_sorted_gates),          \
                     d_slot_pos)
  if (id_dtype == FMOE_I64) {
    if (g4) FMOE_PFILL(int64_t, uint32_t);
    else FMOE_PFILL(int64_t, uint16_t);
  } else {
    if (g4) FMOE_PFILL(int32_t, uint32_t);
    else FMOE_PFILL(int32_t, uint16_t);
  }
#undef FMOE_PFILL
  return fmoe_host::check_launch("fmoe_permute_build(fill)");
}

extern "C" int fmoe_permute_gather(const int32_t* d_slot_pos, int64_t num_tokens, int64_t top_k,
                                   int64_t row_bytes, const void* d_x, int64_t x_row_stride_bytes,
                                   void* d_out, void* stream) {
  fmoe_host::clear_error();
  const int64_t T = num_tokens, K = top_k;
  FMOE_REQUIRE(T >= 0 && K >= 1 && row_bytes >= 1,
               "fmoe_permute_gather: bad sizes T=%lld k=%lld row_bytes=%lld", (long long)T,
               (long long)K, (long long)row_bytes);
  if (row_bytes >= (int64_t(1) << 31) || T >= (int64_t(1) << 31) ||
      (T > 0 && K > ((int64_t(1) << 31) - 1) / T)) {
    fmoe_host::set_error("fmoe_permute_gather: sizes exceed the 32-bit row counters");
    return FMOE_ERANGE;
  }
  if (T == 0) return FMOE_OK;
  FMOE_REQUIRE(d_slot_pos && d_x && d_out, "fmoe_permute_gather: null device pointer");
  FMOE_REQUIRE(x_row_stride_bytes >= row_bytes || T == 1,
               "fmoe_permute_gather: x rows overlap (stride %lld < %lld bytes)",
               (long long)x_row_stride_bytes, (long long)row_bytes);
  FMOE_REQUIRE(row_bytes % 2 == 0 && (uintptr_t)d_x % 2 == 0 && (uintptr_t)d_out % 2 == 0 &&
                   x_row_stride_bytes % 2 == 0,
               "fmoe_permute_gather: rows must be 2-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto aligned = [&](int a) {
    return row_bytes % a == 0 && (uintptr_t)d_x % a == 0 && (uintptr_t)d_out % a == 0 &&
           x_row_stride_bytes % a == 0;
  };
  const dim3 grid((unsigned)T), block(kPermGatherWaves * kWave);
  const uint8_t* x = static_cast<const uint8_t*>(d_x);
  uint8_t* out = static_cast<uint8_t*>(d_out);
  if (aligned(16))
    hipLaunchKernelGGL(k_perm_gather<16>, grid, block, 0, s, d_slot_pos, K, x, x_row_stride_bytes,
                       out, (uint32_t)row_bytes, T * K);
  else if (aligned(4))
    hipLaunchKernelGGL(k_perm_gather<4>, grid, block, 0, s, d_slot_pos, K, x, x_row_stride_bytes,
                       out, (uint32_t)row_bytes, T * K);
  else
    hipLaunchKernelGGL(k_perm_gather<2>, grid, block, 0, s, d_slot_pos, K, x, x_row_stride_bytes,
                       out, (uint32_t)row_bytes, T * K);
  return fmoe_host::check_launch("fmoe_permute_gather");
}

extern "C" int fmoe_permute_gate_grad(const int32_t* d_slot_pos, int64_t num_slots,
                                      const void* d_grad_sorted, int dtype, void* d_grad_gates,
                                      void* stream) {
  fmoe_host::clear_error();
  FMOE_REQUIRE(num_slots >= 0 && num_slots < (int64_t(1) << 31),
               "fmoe_permute_gate_grad: bad slot count %lld", (long long)num_slots);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(dtype), "fmoe_permute_gate_grad: bad dtype %d", dtype);
  if (num_slots == 0) return FMOE_OK;
  FMOE_REQUIRE(d_slot_pos && d_grad_sorted && d_grad_gates,
               "fmoe_permute_gate_grad: null device pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((num_slots + kGroup - 1) / kGroup));
  if (fmoe_host::dtype_bytes(dtype) == 4)
    hipLaunchKernelGGL(k_perm_gate_grad<uint32_t>, grid, dim3(kGroup), 0, s, d_slot_pos, num_slots,
                       static_cast<const uint32_t*>(d_grad_sorted),
                       static_cast<uint32_t*>(d_grad_gates));
  else
    hipLaunchKernelGGL(k_perm_gate_grad<uint16_t>, grid, dim3(kGroup), 0, s, d_slot_pos, num_slots,
                       static_cast<const uint16_t*>(d_grad_sorted),
                       static_cast<uint16_t*>(d_grad_gates));
  return fmoe_host::check_launch("fmoe_permute_gate_grad");
}
