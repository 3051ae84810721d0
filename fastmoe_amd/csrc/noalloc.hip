// Allocation-free forward combine (fmoe_combine_fwd_noalloc).
//
// fmoe_combine_fwd in deterministic mode reads a plan -- the token-major inverse of the scatter
// index -- from a workspace the caller allocates, and the metadata (pointer table, offsets) it is
// built from lives in caller-allocated device arrays too.  Callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc) use
// this entry point instead: the metadata and the plan go into `scratch`, a static device array of
// kScratchBytes that each GPU holds from the library's load until the process ends, and the call
// then runs fmoe_build_metadata_and_plan and fmoe_combine_fwd(det) on it.  The caller passes only
// the inputs and the output.
//
// Host code never passes `scratch` itself to a kernel (on the host that name is only a stand-in
// for the device symbol): the first call on each device looks up the array's device address with
// hipGetSymbolAddress, with that device current, and every later call on that device uses the
// address kept for it.  All calls on one GPU share that GPU's array, so calls that overlap on one
// GPU (two streams, two host threads) race on it; calls on one stream are ordered.  The plan
// kernels write every scratch word they later read, so nothing needs clearing between calls.
#include <mutex>

#include "common.h"

namespace {

constexpr int64_t kScratchBytes = FMOE_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes == (int64_t(16) << 20), "header and library disagree on the size");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Scratch layout: the metadata arrays of up to kMaxExperts experts, then the plan workspace.
constexpr int64_t kMaxExperts = 4096;
constexpr int64_t kPtrTableOff = 0;                                // int64[E]
constexpr int64_t kChunkSizesOff = kPtrTableOff + 8 * kMaxExperts; // int32[E]
constexpr int64_t kOffsetsOff = kChunkSizesOff + 4 * kMaxExperts;  // int64[E + 1]
constexpr int64_t kMaxRowsOff = kOffsetsOff + 8 * (kMaxExperts + 1) + 248;  // int32[1]
constexpr int64_t kPlanOff = 128 * 1024;                           // plan workspace, 256-aligned
static_assert(kMaxRowsOff % 256 == 0 && kMaxRowsOff + 4 <= kPlanOff, "scratch layout");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device (null: not looked up)

// Device address of the current device's `scratch`, looked up on the first call on that device.
// That first call must not be recorded into a HIP graph: the lookup is a runtime query, not a
// stream operation, so a stream under capture is refused until the address is known.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fmoe_host::set_error("fmoe_combine_fwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return FMOE_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fmoe_host::set_error("fmoe_combine_fwd_noalloc: device %d beyond the %d supported", dev,
                         kMaxDevices);
    return FMOE_ERANGE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess || cap != hipStreamCaptureStatusNone) {
      fmoe_host::set_error("fmoe_combine_fwd_noalloc: the first call on device %d must come before "
                           "any graph capture on its stream (it looks up the static buffer's "
                           "address); call it once outside the capture", dev);
      return FMOE_EINVAL;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      fmoe_host::set_error("fmoe_combine_fwd_noalloc: hipGetSymbolAddress(scratch) failed on "
                           "device %d: %s", dev, hipGetErrorString(e));
      return FMOE_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FMOE_OK;
}

}  // namespace

extern "C" int fmoe_combine_fwd_noalloc(const int64_t* host_ptrs, const int64_t* host_rows,
                                        int64_t num_experts, const void* d_indices, int idx_dtype,
                                        const void* d_weights, int w_dtype, int64_t num_tokens,
                                        int64_t hidden, int x_dtype, void* d_out, int out_dtype,
                                        int64_t out_row_stride, int accumulate, void* stream) {
  fmoe_host::clear_error();
  const char* who = "fmoe_combine_fwd_noalloc";
  const int64_t E = num_experts, T = num_tokens;
  FMOE_REQUIRE(E >= 1 && E <= kMaxExperts, "%s: num_experts must be in [1, %lld] (got %lld)", who,
               (long long)kMaxExperts, (long long)E);
  FMOE_REQUIRE(host_ptrs && host_rows, "%s: null host table", who);
  FMOE_REQUIRE(T >= 1 && hidden >= 1, "%s: bad sizes T=%lld D=%lld", who, (long long)T,
               (long long)hidden);
  FMOE_REQUIRE(fmoe_host::is_float_dtype(x_dtype), "%s: bad x dtype %d", who, x_dtype);
  int64_t N = 0;
  for (int64_t e = 0; e < E; ++e) {
    FMOE_REQUIRE(host_rows[e] >= 0 && host_rows[e] < (int64_t(1) << 31),
                 "%s: expert %lld has invalid row count %lld", who, (long long)e,
                 (long long)host_rows[e]);
    N += host_rows[e];
  }
  if (N >= (int64_t(1) << 31) || T >= (int64_t(1) << 30)) {
    fmoe_host::set_error("%s: N=%lld / T=%lld exceed the 32-bit row counters", who, (long long)N,
                         (long long)T);
    return FMOE_ERANGE;
  }
  // Size check before any HIP call: the plan of N rows and T tokens must fit after the metadata.
  const int64_t plan_bytes = fmoe_plan_workspace_bytes(N, T);
  if (plan_bytes < 0 || kPlanOff + plan_bytes > kScratchBytes) {
    fmoe_host::set_error(
        "%s: N=%lld rows and T=%lld tokens need %lld bytes of plan, more than the %lld bytes of "
        "the static scratch buffer hold; build the plan in a caller workspace instead "
        "(fmoe_build_metadata_and_plan + fmoe_combine_fwd)",
        who, (long long)N, (long long)T, (long long)plan_bytes,
        (long long)(kScratchBytes - kPlanOff));
    return FMOE_ERANGE;
  }
  void* base = nullptr;
  if (int rc = scratch_address(static_cast<hipStream_t>(stream), &base)) return rc;
  char* s = static_cast<char*>(base);
  int64_t* ptr_table = reinterpret_cast<int64_t*>(s + kPtrTableOff);
  int32_t* chunk_sizes = reinterpret_cast<int32_t*>(s + kChunkSizesOff);
  int64_t* offsets = reinterpret_cast<int64_t*>(s + kOffsetsOff);
  int32_t* max_rows = reinterpret_cast<int32_t*>(s + kMaxRowsOff);
  void* plan = s + kPlanOff;
  const int64_t row_bytes = hidden * fmoe_host::dtype_bytes(x_dtype);
  if (int rc = fmoe_build_metadata_and_plan(host_ptrs, host_rows, E, ptr_table, chunk_sizes,
                                            offsets, max_rows, d_indices, idx_dtype, d_weights,
                                            w_dtype, T, row_bytes, plan, stream))
    return rc;
  return fmoe_combine_fwd(FMOE_MODE_DET, plan, nullptr, FMOE_I64, nullptr, FMOE_F32, ptr_table,
                          offsets, E, N, T, hidden, x_dtype, d_out, out_dtype, out_row_stride,
                          accumulate, nullptr, 0, stream);
}
