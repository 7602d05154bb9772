// Launches of the tiled GEMM with a K-major operand: the input gradient
// dY W (W K-major) and the weight gradient dY^T X (both K-major, or dY^T
// row-major when a producer wrote it), compiled apart from gemm.hip for the
// register-assignment flag described in gemm_kernels.h.
#include "gemm_kernels.h"

namespace zk {
namespace gemm {

namespace {
template <typename T>
void launch_t(bool akm, bool bkm, const GemmArgs& ga, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((ga.M / BM) * (ga.N / BN)));
  if (akm && bkm)
    hipLaunchKernelGGL((gemm_tiled_kernel<T, 0, true, true>), grid, dim3(256), 0, s, ga);
  else if (akm)
    hipLaunchKernelGGL((gemm_tiled_kernel<T, 0, true, false>), grid, dim3(256), 0, s, ga);
  else if (half_tiles(grid.x))
    hipLaunchKernelGGL((gemm_tiled_kernel<T, 0, false, true, 4>), dim3(2 * grid.x), dim3(256), 0,
                       s, ga);
  else
    hipLaunchKernelGGL((gemm_tiled_kernel<T, 0, false, true>), grid, dim3(256), 0, s, ga);
}
}  // namespace

void launch_tiled_kmajor(bool bf16_, bool a_kmajor, bool b_kmajor, const GemmArgs& ga,
                         hipStream_t s) {
  if (bf16_)
    launch_t<bf16>(a_kmajor, b_kmajor, ga, s);
  else
    launch_t<f16>(a_kmajor, b_kmajor, ga, s);
}

}  // namespace gemm
}  // namespace zk
