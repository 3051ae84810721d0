// Version, thread-local error string and kernel-variant options of the C ABI (host code only).
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/fastmoe_amd.h"
#include "options.h"

namespace fmoe_host {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

// Same order as enum Opt (common.h).
struct OptDef {
  const char* name;
  const char* env;
  int64_t dflt;
};
static const OptDef kOpts[] = {
    {"plan", "FMOE_PLAN", 0},          {"bwd_fused", "FMOE_BWD_FUSED", 0},
    {"gw_staged", "FMOE_GW_STAGED", 1}, {"force_scalar", "FMOE_FORCE_SCALAR", 0},
    {"bwd_u", "FMOE_BWD_U", 0},        {"fwd_tile", "FMOE_FWD_TILE", 0},
    {"fwd_atomic_tile", "FMOE_FWD_ATOMIC_TILE", 0},
    {"fwd_det_u", "FMOE_FWD_DET_U", 0}, {"fwd_grid", "FMOE_FWD_GRID", 0},
    {"plan_groups", "FMOE_PLAN_GROUPS", 0}, {"small", "FMOE_SMALL", 0},
    {"fwd_atomic_order", "FMOE_FWD_ATOMIC_ORDER", 0},
};
constexpr int kNumOpts = (int)(sizeof(kOpts) / sizeof(kOpts[0]));
static_assert(kNumOpts == kOptCount, "one table entry per enum Opt value");

static std::atomic<int64_t> g_opts[kNumOpts];

// Read once when the library is loaded.
static const bool g_opts_loaded = [] {
  for (int i = 0; i < kNumOpts; ++i) {
    const char* s = getenv(kOpts[i].env);
    g_opts[i].store((s && *s) ? (int64_t)atoll(s) : kOpts[i].dflt, std::memory_order_relaxed);
  }
  const char* split = getenv("FMOE_PLAN_SPLIT");  // older name of plan=1
  if (split && *split && atoi(split) != 0) g_opts[0].store(1, std::memory_order_relaxed);
  return true;
}();

int64_t opt(int o) { return g_opts[o].load(std::memory_order_relaxed); }

static int find_opt(const char* name) {
  if (!name) return -1;
  for (int i = 0; i < kNumOpts; ++i)
    if (strcmp(name, kOpts[i].name) == 0) return i;
  return -1;
}

}  // namespace fmoe_host

extern "C" int fmoe_abi_version(void) { return FMOE_ABI_VERSION; }

extern "C" const char* fmoe_last_error(void) { return fmoe_host::g_last_error.c_str(); }

extern "C" int fmoe_set_option(const char* name, int64_t value, int64_t* previous) {
  fmoe_host::clear_error();
  const int i = fmoe_host::find_opt(name);
  if (i < 0) {
    fmoe_host::set_error("fmoe_set_option: unknown option \"%s\"", name ? name : "(null)");
    return FMOE_EINVAL;
  }
  const int64_t old = fmoe_host::g_opts[i].exchange(value, std::memory_order_relaxed);
  if (previous) *previous = old;
  return FMOE_OK;
}

extern "C" int fmoe_get_option(const char* name, int64_t* value) {
  fmoe_host::clear_error();
  const int i = fmoe_host::find_opt(name);
  if (i < 0 || !value) {
    fmoe_host::set_error("fmoe_get_option: unknown option \"%s\" or null output",
                         name ? name : "(null)");
    return FMOE_EINVAL;
  }
  *value = fmoe_host::g_opts[i].load(std::memory_order_relaxed);
  return FMOE_OK;
}
