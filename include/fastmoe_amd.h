/*
 * fastmoe_amd.h -- C ABI of the MI355X (gfx950) grouped pointer-indirection MoE combine.
 *
 * The combine adds every routed row g of the ragged per-expert output buffers, scaled by its gate
 * weight, into the token-ordered output:
 *
 *     out[idx[g], :] += w[g] * X_e[g - off[e], :]      for g in [off[e], off[e] + n_e)
 *
 * where X_e is expert e's own [n_e, D] buffer (never concatenated), off[] is the exclusive prefix
 * sum of the row counts n_e, idx[] is the scatter index (token of each packed row) and w[] the gate
 * weight.  The backward gives grad_X[g, :] = grad_out[idx[g], :] * w[g] and
 * grad_w[g] = sum_d grad_out[idx[g], d] * X_e[g - off[e], d].
 *
 * Conventions
 *   - Every pointer named d_* is a device pointer; host_* pointers are host memory.
 *   - Sizes are int64_t.  `stream` is a hipStream_t passed as void* (NULL = null stream).
 *   - Every entry point only enqueues work on `stream`: none allocates memory, none synchronises,
 *     so a caller may capture the calls in a HIP graph.
 *   - Return value: FMOE_OK (0) or a negative fmoe_status; fmoe_last_error() then holds a message
 *     (thread-local, valid until the next failing call on the same thread).
 *   - Rows whose scatter index lies outside [0, T) are never read or written through; they are
 *     counted into the plan's status word (fmoe_plan_status_offset()) and their gradients are
 *     written as zero.
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   fmoe_build_metadata    <- prepare_grouped_metadata        src/fastmoe/kernels/ops.py:200-271
 *   fmoe_combine_fwd       <- _launch_grouped_kernel + Triton  src/fastmoe/kernels/ops.py:277-310
 *                             _grouped_weighted_scatter_add_kernel  ops.py:57-194
 *   fmoe_combine_bwd       <- GroupedWeightedScatterAdd.backward    ops.py:333-359
 *   fmoe_combine_fwd_small / fmoe_combine_bwd_small <- the same three, for at most 4096 rows:
 *                             one launch per direction and no plan
 *   fmoe_build_plan        <- no counterpart: the token-major inverse of the scatter index that the
 *                             deterministic combine and the backward read (ops.py:344 gathers by
 *                             scatter index on the fly instead)
 *   fmoe_invert_scatter_index <- no counterpart either: the same inverse as a bare CSR
 *   fmoe_permute_*         <- the sort-and-gather of MoEFeedForward.gate_and_sort
 *                             src/fastmoe/models/tiny_model.py:108-138 (the combine's producer)
 */
#ifndef FASTMOE_AMD_H
#define FASTMOE_AMD_H

#include <stdint.h>

#if defined(__GNUC__)
#define FMOE_API __attribute__((visibility("default")))
#else
#define FMOE_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FMOE_ABI_VERSION 2

/* Element types. */
enum fmoe_dtype {
  FMOE_F32 = 0,
  FMOE_BF16 = 1,
  FMOE_F16 = 2,
  FMOE_I64 = 3, /* scatter index only */
  FMOE_I32 = 4  /* scatter index only */
};

/* Forward combine modes. */
enum fmoe_mode {
  /* Token-major: every output row is reduced in ascending packed-row order in fp32 registers and
     written once.  Bit-identical run to run; bit-identical to the CPU index_add_ path in fp32. */
  FMOE_MODE_DET = 0,
  /* Packed-row-major like the reference kernel: hardware fp32 atomics (global_atomic_add_f32).
     A bf16/f16 `out` is accumulated in a caller-owned fp32 workspace and rounded once at the end,
     so it is within 1 ulp of the fp32 sum rounded once; the order of the fp32 additions (and so
     the last bits) varies run to run. */
  FMOE_MODE_ATOMIC = 1,
  /* As FMOE_MODE_ATOMIC, but a bf16/f16 `out` takes gfx950's packed 16-bit atomics
     (global_atomic_pk_add_bf16 / _f16) directly: no workspace, half the atomic requests, and a
     rounding to 16 bits at every add (the reference Triton kernel's behaviour with a bf16 out). */
  FMOE_MODE_ATOMIC_PACKED = 2
};

enum fmoe_status {
  FMOE_OK = 0,
  FMOE_EINVAL = -1,   /* bad argument (null pointer, size, dtype, alignment, layout) */
  FMOE_EHIP = -2,     /* a HIP runtime call failed */
  FMOE_ERANGE = -3    /* a size exceeds what the kernels address (e.g. N >= 2^31) */
};

/* Version of this ABI (FMOE_ABI_VERSION). */
FMOE_API int fmoe_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
FMOE_API const char* fmoe_last_error(void);

/*
 * Kernel-variant options (no counterpart in the reference, whose Triton kernel has none).  Every
 * option defaults to the measured-best choice; the environment variable in brackets sets the
 * starting value once, when the library loads.  Launches read the option table, never the
 * environment.  Options select among variants that compute the same results (tests compare them):
 *   "plan"            [FMOE_PLAN]      0 = automatic (the radix plan when the tokens average 64
 *                                      rows or more; else one launch below 2^16 rows, the ranged
 *                                      plan up to 2^22 rows and 2^19 tokens, the radix plan
 *                                      beyond), 1 = radix (a stable radix sort by token),
 *                                      2 = bucketed (two launches; never chosen automatically: a
 *                                      hot token's bucket is ordered by one wave), 3 = one launch,
 *                                      4 = ranged (two launches)
 *   "bwd_fused"       [FMOE_BWD_FUSED] 1 = both backward gradients in one pass
 *   "gw_staged"       [FMOE_GW_STAGED] 0 = grad_w pass reads grad_out per wave, not through LDS
 *   "force_scalar"    [FMOE_FORCE_SCALAR] 1 = element-wise instead of 16-byte accesses
 *   "bwd_u", "fwd_tile", "fwd_atomic_tile", "fwd_det_u", "fwd_grid": tile shapes (0 = by D,
 *                                      and for "fwd_tile" by the rows per token too)
 *   "plan_groups"     [FMOE_PLAN_GROUPS] workgroups of the one-launch plan (0 = by N and T)
 *   "small"           [FMOE_SMALL]     the Python host's use of fmoe_combine_fwd_small /
 *                                      fmoe_combine_bwd_small: 0 = by size, 1 = never, 2 = whenever
 *                                      their limits allow (the library itself does not read it)
 *   "fwd_atomic_order" [FMOE_FWD_ATOMIC_ORDER] grid order of the atomic forward: 0 = by size,
 *                                      1 = a row's column chunks side by side, 2 = column-chunk
 *                                      major (all rows' chunk 0, then chunk 1, ...)
 * fmoe_set_option returns FMOE_EINVAL for an unknown name; *previous (if not NULL) gets the old
 * value.  Not synchronised with launches in flight on other threads.
 */
FMOE_API int fmoe_set_option(const char* name, int64_t value, int64_t* previous);
FMOE_API int fmoe_get_option(const char* name, int64_t* value);

/*
 * Pointer table and row-count metadata of E ragged expert buffers
 * (replaces prepare_grouped_metadata, src/fastmoe/kernels/ops.py:200-271).
 *
 * host_ptrs[e]  : device address of expert e's [n_e, D] row-contiguous buffer (may be 0 if n_e==0)
 * host_rows[e]  : n_e
 * Writes on the device:
 *   d_ptr_table[E]        int64 addresses             (ops.py:221-224)
 *   d_chunk_sizes[E]      int32 row counts            (ops.py:233-234)
 *   d_offsets[E + 1]      int64 exclusive prefix sums, d_offsets[E] = sum n_e   (ops.py:247-256)
 *   d_max_rows[1]         int32 max n_e               (ops.py:268)
 * The table travels inside kernel arguments (no host staging buffer, no H2D copy), up to 256
 * experts per launch.
 */
FMOE_API int fmoe_build_metadata(const int64_t* host_ptrs, const int64_t* host_rows, int64_t num_experts,
                        int64_t* d_ptr_table, int32_t* d_chunk_sizes, int64_t* d_offsets,
                        int32_t* d_max_rows, void* stream);

/*
 * Plan: token-major inverse of the scatter index.  For each token t, the packed rows g with
 * idx[g] == t, each as a 16-byte record {source row address, fp32 gate, g}, in ascending g.  Rows
 * with an out-of-range index form one extra segment (number T).  Time is linear in N + T: one
 * launch below 2^16 rows, two (the ranged plan: partition by token range, then a workgroup per
 * range) up to 2^22 rows and 2^19 tokens, and a stable radix sort of the rows by token (3 launches
 * per 8 bits of T, plus 3 to 5) beyond that or when the tokens average 64 rows or more, whose
 * time does not depend on how the rows spread (option "plan" selects a path, and also offers the
 * bucketed plan: partition by token bucket, then a wave per bucket).
 *
 * Workspace: fmoe_plan_workspace_bytes(N, T) bytes of device memory, 256-byte aligned, owned by the
 * caller; no zero-fill is needed.  Layout (byte offsets from the workspace base):
 *   fmoe_plan_status_offset()     : int32 count of out-of-range scatter indices
 *   fmoe_plan_row_ptr_offset(N,T) : int32 row_ptr[T + 2] (segment t = [row_ptr[t], row_ptr[t+1]))
 *   fmoe_plan_records_offset(N,T) : N 16-byte records, grouped by segment
 *
 * d_indices : [N] scatter index, FMOE_I64 or FMOE_I32
 * d_weights : [N] gate weights, FMOE_F32 / FMOE_BF16 / FMOE_F16
 * d_ptr_table, d_offsets : from fmoe_build_metadata
 * row_bytes : D * sizeof(expert element)
 */
FMOE_API int64_t fmoe_plan_workspace_bytes(int64_t num_rows, int64_t num_tokens);
FMOE_API int64_t fmoe_plan_status_offset(void);
FMOE_API int64_t fmoe_plan_row_ptr_offset(int64_t num_rows, int64_t num_tokens);
FMOE_API int64_t fmoe_plan_records_offset(int64_t num_rows, int64_t num_tokens);
FMOE_API int fmoe_build_plan(const void* d_indices, int idx_dtype, const void* d_weights, int w_dtype,
                    int64_t num_rows, int64_t num_tokens, const int64_t* d_ptr_table,
                    const int64_t* d_offsets, int64_t num_experts, int64_t row_bytes,
                    void* d_workspace, void* stream);

/*
 * The plan builder fmoe_build_plan / fmoe_build_metadata_and_plan take for N rows, T tokens and E
 * experts under the current "plan" option: 1 radix, 2 bucketed, 3 one launch, 4 ranged (the
 * option's own numbering), or -1 for sizes no builder takes.  No counterpart in the reference
 * (its Triton kernel has no plan); for callers and benchmarks that force a path and need to know
 * whether its limits hold.  Host only: no GPU call.
 */
FMOE_API int fmoe_plan_path(int64_t num_rows, int64_t num_tokens, int64_t num_experts);

/*
 * fmoe_build_metadata followed by fmoe_build_plan on the same experts, in one call (no counterpart
 * in the reference, which builds metadata per call in prepare_grouped_metadata, ops.py:200-271,
 * and needs no inverse).  Outputs and workspace exactly as those two calls; num_rows is the sum
 * of host_rows.  With at most 256 experts the plan's own kernels also write the metadata, the
 * (address, rows) table riding in their arguments: one launch below 2^16 rows, two beyond (up to
 * 2^22 tokens); otherwise it makes the two calls.
 */
FMOE_API int fmoe_build_metadata_and_plan(const int64_t* host_ptrs, const int64_t* host_rows,
                                 int64_t num_experts, int64_t* d_ptr_table,
                                 int32_t* d_chunk_sizes, int64_t* d_offsets, int32_t* d_max_rows,
                                 const void* d_indices, int idx_dtype, const void* d_weights,
                                 int w_dtype, int64_t num_tokens, int64_t row_bytes,
                                 void* d_workspace, void* stream);

/*
 * Plan of a combine fed by fmoe_permute_build (no counterpart in the reference; it replaces
 * fmoe_build_plan when the scatter index is that permutation's reverse map): token t's rows are
 * d_slot_pos[t * top_k + j], j < top_k, so the plan is written by one thread per slot with no
 * counting or scanning.  Requires num_rows == num_tokens * top_k (every slot is a row of the
 * combine: all expert ids were in range) and top_k <= 64.  d_weights are the gates in packed-row
 * order (the permutation's sorted gates); d_ptr_table / d_offsets from fmoe_build_metadata over the
 * per-expert buffers.  Same workspace size and layout as fmoe_build_plan(num_rows, num_tokens).
 */
FMOE_API int fmoe_build_plan_from_slots(const int32_t* d_slot_pos, int64_t num_tokens,
                               int64_t top_k, const void* d_weights, int w_dtype,
                               const int64_t* d_ptr_table, const int64_t* d_offsets,
                               int64_t num_experts, int64_t num_rows, int64_t row_bytes,
                               void* d_workspace, void* stream);

/*
 * fmoe_build_metadata followed by fmoe_build_plan_from_slots on the same experts, in one call (no
 * counterpart in the reference).  Outputs and workspace exactly as those two calls; num_rows is the
 * sum of host_rows.  With at most 256 experts a single kernel launch writes both, the (address,
 * rows) table riding in its arguments; otherwise it makes the two calls.
 */
FMOE_API int fmoe_build_metadata_and_plan_from_slots(
    const int64_t* host_ptrs, const int64_t* host_rows, int64_t num_experts, int64_t* d_ptr_table,
    int32_t* d_chunk_sizes, int64_t* d_offsets, int32_t* d_max_rows, const int32_t* d_slot_pos,
    int64_t num_tokens, int64_t top_k, const void* d_weights, int w_dtype, int64_t row_bytes,
    void* d_workspace, void* stream);

/*
 * The token-major inverse of the scatter index as a bare CSR (no counterpart in the reference,
 * whose backward gathers by scatter index instead, ops.py:344; this is the plan without the
 * records, for callers that want the inverse index itself):
 *   d_row_ptr[T + 2] int32 : token t's rows are d_rows[d_row_ptr[t] .. d_row_ptr[t + 1]); segment T
 *                            holds the rows whose index lies outside [0, T)
 *   d_rows[N]        int32 : row numbers g, ascending within every segment
 * d_indices : [N] scatter index, FMOE_I64 or FMOE_I32.  Workspace: fmoe_plan_workspace_bytes(N, T)
 * bytes, 256-byte aligned, no zero-fill.  The radix plan, or the bucketed plan with option
 * plan=2; linear in N + T either way.
 */
FMOE_API int fmoe_invert_scatter_index(const void* d_indices, int idx_dtype, int64_t num_rows,
                              int64_t num_tokens, int32_t* d_row_ptr, int32_t* d_rows,
                              void* d_workspace, void* stream);

/*
 * Forward combine (replaces _launch_grouped_kernel + _grouped_weighted_scatter_add_kernel,
 * src/fastmoe/kernels/ops.py:277-310 and :57-194).
 *
 * mode == FMOE_MODE_DET     : reads the plan (d_plan from fmoe_build_plan on the same inputs);
 *                             d_indices/d_weights/d_ptr_table/d_offsets may be NULL.
 * mode == FMOE_MODE_ATOMIC[_PACKED] : reads d_indices/d_weights/d_ptr_table/d_offsets; d_plan may
 *                             be NULL.
 * out        : [T, D] with row stride out_row_stride (elements) and unit column stride.
 * accumulate : 1 = add into the existing contents of out (the reference's in-place contract,
 *              ops.py:389-390); 0 = overwrite (rows of tokens without routed rows become 0:
 *              FMOE_MODE_ATOMIC with a 16-bit out starts its fp32 accumulator from zeros, the
 *              other atomic cases clear out first with a fill kernel).
 * x_dtype    : dtype of every expert buffer; out_dtype: dtype of out.
 * d_workspace, workspace_bytes : device memory the caller owns, at least
 *              fmoe_combine_fwd_workspace_bytes(mode, T, D, out_dtype) bytes, 16-byte aligned
 *              (the fp32 accumulator of FMOE_MODE_ATOMIC with a 16-bit out, T * D * 4 bytes);
 *              NULL / 0 when that is 0.
 */
FMOE_API int64_t fmoe_combine_fwd_workspace_bytes(int mode, int64_t num_tokens, int64_t hidden,
                                         int out_dtype);
FMOE_API int fmoe_combine_fwd(int mode, const void* d_plan, const void* d_indices, int idx_dtype,
                     const void* d_weights, int w_dtype, const int64_t* d_ptr_table,
                     const int64_t* d_offsets, int64_t num_experts, int64_t num_rows,
                     int64_t num_tokens, int64_t hidden, int x_dtype, void* d_out, int out_dtype,
                     int64_t out_row_stride, int accumulate, void* d_workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * Allocation-free deterministic forward.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  It computes what fmoe_build_metadata_and_plan followed by
 * fmoe_combine_fwd(FMOE_MODE_DET, ...) compute, bit for bit, but the metadata arrays and the plan
 * live in a static device buffer of FMOE_NOALLOC_SCRATCH_BYTES that the library holds on every
 * GPU it runs on until the process ends; the caller passes only inputs and the output, and the
 * call allocates nothing.
 *
 * Limits: 1 <= num_experts <= 4096 and fmoe_plan_workspace_bytes(N, T) <= 16 MiB - 128 KiB, i.e.
 * roughly 32 * N + 8 * T bytes (N = sum of host_rows; e.g. N = 2^18 rows with T = 2^18 tokens).
 * Larger calls return FMOE_ERANGE before touching the GPU.
 * Calls on one GPU share its buffer: calls that overlap on one GPU (two streams, two threads)
 * race; calls on one stream are ordered.  Arguments as in fmoe_build_metadata_and_plan and
 * fmoe_combine_fwd.
 * Graph capture: the first call on a device looks up the buffer's address and must run outside
 * any capture (under one it returns FMOE_EINVAL); later calls can be captured and replayed, each
 * replay rebuilding the metadata and plan in the buffer.
 */
#define FMOE_NOALLOC_SCRATCH_BYTES (16 << 20)
FMOE_API int fmoe_combine_fwd_noalloc(const int64_t* host_ptrs, const int64_t* host_rows,
                             int64_t num_experts, const void* d_indices, int idx_dtype,
                             const void* d_weights, int w_dtype, int64_t num_tokens,
                             int64_t hidden, int x_dtype, void* d_out, int out_dtype,
                             int64_t out_row_stride, int accumulate, void* stream);

/*
 * Backward combine (replaces GroupedWeightedScatterAdd.backward, src/fastmoe/kernels/ops.py:333-359,
 * and adds the gate gradient that the reference leaves out at :358-359).
 *
 * d_grad_out : [T, D] of gout_dtype, row stride gout_row_stride, unit column stride
 * d_grad_x   : [N, D] contiguous of x_dtype (packed-row order; split per expert by the caller), or
 *              NULL to skip it.  grad_X[g] = round_x(f32(grad_out[idx[g]]) * w[g]).
 * d_grad_w   : [N] of gw_dtype, or NULL to skip it (then the expert buffers are not read).
 *              grad_w[g] accumulates the D products in fp64 and rounds once.
 * Given both outputs, the call enqueues two kernels: the grad_X pass, then the grad_w pass.
 */
FMOE_API int fmoe_combine_bwd(const void* d_plan, int64_t num_rows, int64_t num_tokens, int64_t hidden,
                     int x_dtype, const void* d_grad_out, int gout_dtype, int64_t gout_row_stride,
                     void* d_grad_x, void* d_grad_w, int gw_dtype, void* stream);

/*
 * Small inputs: the deterministic forward and the backward of at most
 * fmoe_combine_small_max_rows() rows (4096) over at most 256 experts, one launch each and no plan
 * (they replace the same reference code as fmoe_combine_fwd in FMOE_MODE_DET and
 * fmoe_combine_bwd: src/fastmoe/kernels/ops.py:57-194, :277-310 and :333-359).  Results equal
 * fmoe_build_metadata_and_plan + fmoe_combine_fwd(FMOE_MODE_DET) and fmoe_combine_bwd bit for bit;
 * the saving is the plan's launch, which dominates such calls.
 *
 * host_ptrs / host_rows / num_experts : the experts' (address, rows) pairs, as in
 *              fmoe_build_metadata (read on the host, passed in the kernel arguments).
 * d_indices, d_weights : [N] scatter index (FMOE_I64 / FMOE_I32) and gates (any float dtype).
 * fmoe_combine_fwd_small: out, out_row_stride, accumulate and the dtypes as in fmoe_combine_fwd;
 *              d_status [1] int32 receives the number of rows whose index lies outside [0, T)
 *              (those rows are skipped), written by the launch.
 * fmoe_combine_bwd_small: d_grad_out, d_grad_x, d_grad_w and the dtypes as in fmoe_combine_bwd;
 *              both outputs (or either) come from one kernel.
 * More rows or experts return FMOE_ERANGE / FMOE_EINVAL before touching the GPU.
 */
FMOE_API int64_t fmoe_combine_small_max_rows(void);
FMOE_API int fmoe_combine_fwd_small(const int64_t* host_ptrs, const int64_t* host_rows,
                           int64_t num_experts, const void* d_indices, int idx_dtype,
                           const void* d_weights, int w_dtype, int64_t num_tokens, int64_t hidden,
                           int x_dtype, void* d_out, int out_dtype, int64_t out_row_stride,
                           int accumulate, int32_t* d_status, void* stream);
FMOE_API int fmoe_combine_bwd_small(const int64_t* host_ptrs, const int64_t* host_rows,
                           int64_t num_experts, const void* d_indices, int idx_dtype,
                           const void* d_weights, int w_dtype, int64_t num_tokens, int64_t hidden,
                           int x_dtype, const void* d_grad_out, int gout_dtype,
                           int64_t gout_row_stride, void* d_grad_x, void* d_grad_w, int gw_dtype,
                           void* stream);

/*
 * Dispatch-side permutation: the routing slots of T tokens x top_k choices grouped by expert
 * (replaces the sort-and-gather of MoEFeedForward.gate_and_sort,
 * src/fastmoe/models/tiny_model.py:108-138).  Slot i = t * top_k + j.
 *
 * fmoe_permute_build (tiny_model.py:112 argsort, :121-125 reverse map, :128 sorted gates,
 *                     :138 bincount):
 *   d_expert_ids [T * top_k]  FMOE_I64 / FMOE_I32 expert id of each slot
 *   d_gates      [T * top_k]  gate of each slot (any float dtype; copied bit for bit)
 *   d_counts     [E] int64    rows per expert
 *   d_offsets    [E + 1] int64 exclusive prefix of d_counts; d_offsets[E] = valid slots
 *   d_rev        [T * top_k] int64  token of each packed row (the combine's scatter index)
 *   d_sorted_gates [T * top_k]      gate of each packed row (the combine's gate weight)
 *   d_slot_pos   [T * top_k] int32  packed row of each slot
 *   d_status     [1] int32    slots whose id lies outside [0, E) (they go after every expert's
 *                             rows, in slot order)
 *   Packed order: experts ascending, and within an expert the slots in ascending order (a stable
 *   sort; the reference's argsort is unstable, so its order of equal ids is unspecified).
 *   Workspace: fmoe_permute_workspace_bytes(T * top_k, E) bytes, 256-byte aligned, no zero-fill.
 *   E <= 4096.
 *
 * fmoe_permute_gather (tiny_model.py:133, x_flat[reverse_map_indices]):
 *   out[d_slot_pos[t * top_k + j], :] = x[t, :] for every slot: a byte copy of row_bytes per
 *   row; x rows are x_row_stride_bytes apart, out is packed [T * top_k, row_bytes].
 *
 * fmoe_permute_gate_grad (the backward of :128): grad_gates[i] = grad_sorted[d_slot_pos[i]].
 * The backward of the gather is the deterministic combine with unit gates (fmoe_build_plan +
 * fmoe_combine_fwd with the packed rows as one expert buffer and d_rev as scatter index).
 */
FMOE_API int64_t fmoe_permute_workspace_bytes(int64_t num_slots, int64_t num_experts);
FMOE_API int fmoe_permute_build(const void* d_expert_ids, int id_dtype, const void* d_gates,
                       int gate_dtype, int64_t num_tokens, int64_t top_k, int64_t num_experts,
                       int64_t* d_counts, int64_t* d_offsets, int64_t* d_rev, void* d_sorted_gates,
                       int32_t* d_slot_pos, int32_t* d_status, void* d_workspace, void* stream);
FMOE_API int fmoe_permute_gather(const int32_t* d_slot_pos, int64_t num_tokens, int64_t top_k,
                        int64_t row_bytes, const void* d_x, int64_t x_row_stride_bytes,
                        void* d_out, void* stream);
FMOE_API int fmoe_permute_gate_grad(const int32_t* d_slot_pos, int64_t num_slots,
                           const void* d_grad_sorted, int dtype, void* d_grad_gates, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTMOE_AMD_H */
