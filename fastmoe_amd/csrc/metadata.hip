// Pointer-table / row-count metadata of the ragged expert buffers, built on the device.
//
// Replaces prepare_grouped_metadata (src/fastmoe/kernels/ops.py:200-271): there the host builds
// two Python lists, copies them with two pageable H2D copies and runs cumsum + cat on the device.
// Here the (address, rows) table rides in the kernel arguments of one launch per 256 experts, and
// the same launch scans the row counts into the exclusive offsets and max_rows.  Nothing is staged
// in host memory, so the call is asynchronous and can be captured in a HIP graph.
#include "common.h"

namespace fmoe {

// Block-wide exclusive scan of one int64 per thread (256 threads); returns the total.
__device__ int64_t block_exclusive_scan_256(int64_t v, int64_t* out_excl) {
  __shared__ int64_t wave_tot[kWavesPerGroup];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  int64_t incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int64_t o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) wave_tot[wv] = incl;
  __syncthreads();
  int64_t before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kWavesPerGroup; ++i) {
    if (i < wv) before += wave_tot[i];
    total += wave_tot[i];
  }
  *out_excl = before + incl - v;
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kGroup) void k_meta_upload(MetaChunk a, int64_t* __restrict__ ptr_table,
                                                        int32_t* __restrict__ chunk_sizes,
                                                        int64_t* __restrict__ offsets,
                                                        int32_t* __restrict__ max_rows) {
  const int i = threadIdx.x;
  int64_t rows = 0;
  if (i < a.count) {
    ptr_table[a.base + i] = a.ptr[i];
    chunk_sizes[a.base + i] = a.rows[i];
    rows = a.rows[i];
  }
  if (!a.scan) return;  // uniform across the block
  int64_t excl;
  const int64_t total = block_exclusive_scan_256(rows, &excl);
  if (i < a.count) offsets[i] = excl;
  if (i == 0) offsets[a.count] = total;
  // max over the chunk
  __shared__ int32_t wave_max[kWavesPerGroup];
  int32_t m = (int32_t)rows;
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) m = max(m, __shfl_xor(m, d, kWave));
  if ((i & (kWave - 1)) == 0) wave_max[i / kWave] = m;
  __syncthreads();
  if (i == 0) {
    int32_t mm = 0;
    for (int w = 0; w < kWavesPerGroup; ++w) mm = max(mm, wave_max[w]);
    *max_rows = mm;
  }
}

// Scan for tables larger than one chunk: one block walks chunk_sizes in steps of 256.
__global__ __launch_bounds__(kGroup) void k_meta_scan(const int32_t* __restrict__ chunk_sizes,
                                                      int64_t E, int64_t* __restrict__ offsets,
                                                      int32_t* __restrict__ max_rows) {
  int64_t carry = 0;
  int32_t m = 0;
  for (int64_t b = 0; b < E; b += kGroup) {
    const int64_t e = b + threadIdx.x;
    const int64_t rows = e < E ? chunk_sizes[e] : 0;
    m = max(m, (int32_t)rows);
    int64_t excl;
    const int64_t total = block_exclusive_scan_256(rows, &excl);
    if (e < E) offsets[e] = carry + excl;
    carry += total;
  }
  if (threadIdx.x == 0) offsets[E] = carry;
  __shared__ int32_t wave_max[kWavesPerGroup];
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) m = max(m, __shfl_xor(m, d, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) wave_max[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t mm = 0;
    for (int w = 0; w < kWavesPerGroup; ++w) mm = max(mm, wave_max[w]);
    *max_rows = mm;
  }
}

}  // namespace fmoe

extern "C" int fmoe_build_metadata(const int64_t* host_ptrs, const int64_t* host_rows,
                                   int64_t num_experts, int64_t* d_ptr_table,
                                   int32_t* d_chunk_sizes, int64_t* d_offsets, int32_t* d_max_rows,
                                   void* stream) {
  using namespace fmoe;
  fmoe_host::clear_error();
  FMOE_REQUIRE(num_experts >= 1, "fmoe_build_metadata: num_experts must be >= 1 (got %lld)",
               (long long)num_experts);
  FMOE_REQUIRE(num_experts < (int64_t(1) << 30), "fmoe_build_metadata: too many experts");
  FMOE_REQUIRE(host_ptrs && host_rows, "fmoe_build_metadata: null host table");
  FMOE_REQUIRE(d_ptr_table && d_chunk_sizes && d_offsets && d_max_rows,
               "fmoe_build_metadata: null device output");
  int64_t total = 0;
  for (int64_t e = 0; e < num_experts; ++e) {
    FMOE_REQUIRE(host_rows[e] >= 0 && host_rows[e] < (int64_t(1) << 31),
                 "fmoe_build_metadata: expert %lld has invalid row count %lld", (long long)e,
                 (long long)host_rows[e]);
    FMOE_REQUIRE(host_rows[e] == 0 || host_ptrs[e] != 0,
                 "fmoe_build_metadata: expert %lld has rows but a null address", (long long)e);
    total += host_rows[e];
  }
  FMOE_REQUIRE(total < (int64_t(1) << 31), "fmoe_build_metadata: %lld rows exceed 2^31-1",
               (long long)total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool single = num_experts <= kMetaChunk;
  for (int64_t b = 0; b < num_experts; b += kMetaChunk) {
    MetaChunk a;
    a.count = (int32_t)std::min<int64_t>(kMetaChunk, num_experts - b);
    a.base = (int32_t)b;
    a.scan = single ? 1 : 0;
    a.pad = 0;
    for (int i = 0; i < kMetaChunk; ++i) {
      a.ptr[i] = i < a.count ? host_ptrs[b + i] : 0;
      a.rows[i] = i < a.count ? (int32_t)host_rows[b + i] : 0;
    }
    hipLaunchKernelGGL(k_meta_upload, dim3(1), dim3(kGroup), 0, s, a, d_ptr_table, d_chunk_sizes,
                       d_offsets, d_max_rows);
    if (int rc = fmoe_host::check_launch("fmoe_build_metadata")) return rc;
  }
  if (!single) {
    hipLaunchKernelGGL(k_meta_scan, dim3(1), dim3(kGroup), 0, s, d_chunk_sizes, num_experts,
                       d_offsets, d_max_rows);
    if (int rc = fmoe_host::check_launch("fmoe_build_metadata(scan)")) return rc;
  }
  return FMOE_OK;
}
