// Kernel-variant options of the C ABI (fmoe_set_option / fmoe_get_option), shared by the host
// table (abi.cpp) and the launchers.
#pragma once

#include <cstdint>

namespace fmoe_host {

// Kernel-variant options (fmoe_set_option).  Each starts from its environment variable, read once
// when the library loads, else from the measured-best default; launches read the table, not the
// environment.
enum Opt {
  kOptPlan = 0,      // "plan": 0 automatic, 1 radix, 2 bucketed, 3 one launch, 4 ranged
  kOptBwdFused,      // "bwd_fused": 1 = both gradients in one backward pass
  kOptGwStaged,      // "gw_staged": 0 = grad_w pass reads grad_out per wave instead of via LDS
  kOptForceScalar,   // "force_scalar": 1 = element-wise (unvectorised) kernels
  kOptBwdU,          // "bwd_u": backward vectors per lane per column step (0 = per pass, by D)
  kOptFwdTile,       // "fwd_tile": forward tile <U><R> (0 = by D)
  kOptFwdAtomicTile, // "fwd_atomic_tile"
  kOptFwdDetU,       // "fwd_det_u": forward vectors per lane per row (0 = by D)
  kOptFwdGrid,       // "fwd_grid": forward workgroups (0 = one wave per unit)
  kOptPlanGroups,    // "plan_groups": workgroups of the one-launch plan (0 = by N and T)
  kOptSmall,         // "small": the host's choice of the one-launch small path (0 = by size,
                     // 1 = never, 2 = whenever its limits allow)
  kOptAtomicOrder,   // "fwd_atomic_order": atomic forward's grid order (0 = by size, 1 = row
                     // chunks together, 2 = column-chunk-major)
  kOptCount
};
int64_t opt(int o);

}  // namespace fmoe_host
