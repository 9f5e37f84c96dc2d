// Host side of the wide streamed grouped GEMM (the kernel: gemm_wide.hpp): whether a launch fits,
// and the dispatch to the per-mode launchers (gemm_wide_gu.hip, gemm_wide_dn.hip).
#include <algorithm>
#include <atomic>

#include "gemm_wide.hpp"

namespace moe {

// Whether the launch fits: whole units, K <= 3072, and, from the host's upper bound on the groups
// (an expert of n entries has ceil(ceil(n / 16) / nch) <= n / (16 nch) + 1 groups), at most
// kWideMaxGroups groups.
static bool gemm_wide_fits(const GemmArgs &a, int rt, int nch, int n_wg) {
  if (a.d.tiles % rt || a.d.ns > (uint32_t)kGemmNs || a.max_active > kMaxExperts || n_wg % 8 || n_wg <= 0)
    return false;
  const long long gu = a.d.tiles / rt;
  if (gu < 1) return false;
  const long long rg = (gu + kWideCompute - 1) / kWideCompute;
  const long long ng = (long long)(a.n_entries / (kWideCols * nch)) +
                       std::min<long long>(a.max_active, (long long)a.n_entries);
  return ng <= kWideMaxGroups && ng * rg <= INT32_MAX / 2;
}

static int wide_cus() {
  static std::atomic<int> cus[64] = {};  // (threads racing here store the same value)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (!c) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
    c = n / 8 * 8;
    cus[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

// The wide streamed kernel, or hipErrorNotSupported when the launch does not fit it (the caller
// then runs another shape).
hipError_t launch_gemm_wide(GemvMode mode, const GemmArgs &a, hipStream_t s) {
  const int n_wg = wide_cus();
  if (!a.n_entries) return hipSuccess;
  if (a.terms != 1 && a.terms != kGemmTerms) return hipErrorInvalidValue;
  // gate_up reads the tokens' records through entry_src, down the entries' own
  if ((mode == GEMV_GATE_UP) != (a.entry_src != nullptr)) return hipErrorNotSupported;
  if (!gemm_wide_fits(a, mode == GEMV_GATE_UP ? 4 : 2, kWideNch, n_wg)) return hipErrorNotSupported;
  return mode == GEMV_GATE_UP ? launch_wide_gate_up(a, s, n_wg) : launch_wide_down(a, s, n_wg);
}

}  // namespace moe
