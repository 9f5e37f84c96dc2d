// Launcher of the wide streamed grouped GEMM for the down matrix (kernel: gemm_wide.hpp): 2 tiles of 16
// rows per compute wavefront. One translation unit per mode, so the instantiations compile in
// parallel.
#include "gemm_wide.hpp"

namespace moe {

hipError_t launch_wide_down(const GemmArgs &a, hipStream_t s, int n_wg) {
  return a.terms == 1 ? launch_wide_rt<GEMV_DOWN, 2, 1>(a, s, n_wg) : launch_wide_rt<GEMV_DOWN, 2, kGemmTerms>(a, s, n_wg);
}

}  // namespace moe
