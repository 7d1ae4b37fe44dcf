// B3 of the sparse MLA backward for int8 G rows (bwd_g_kernel<KS, true>, DSA_BWD_G_INT8), in a
// file of its own so that it alone is compiled with MFMA accumulators in VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form is a whole-file option): its quantisation reads every
// accumulator with VALU instructions, which from AccVGPRs would first take one v_accvgpr_read
// each.  The bf16-row B3 (dsa_sparse_bwd.hip) keeps its accumulators in AccVGPRs.
#include "dsa_bwd_g.h"

namespace dsa {

void launch_bwd_g_i8(const SparseBwdParams& p, hipStream_t stream) {
  const int nks = p.n_heads / 16;
  const dim3 grid(xcd_grid(p.total_q, p.n_xcd));
  if (nks > 4)
    hipLaunchKernelGGL((bwd_g_kernel<8, true>), grid, dim3(256), 0, stream, p);
  else if (nks > 2)
    hipLaunchKernelGGL((bwd_g_kernel<4, true>), grid, dim3(256), 0, stream, p);
  else if (nks > 1)
    hipLaunchKernelGGL((bwd_g_kernel<2, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((bwd_g_kernel<1, true>), grid, dim3(256), 0, stream, p);
}

}  // namespace dsa
