// gemm_g32_affine.hip — the grouped GEMM kernels for group size 32, affine scheme.
#include "prefill_gemm_impl.hpp"

namespace tsg {

template tsg_status routed_gemm_launch<32, false>(const tsg_moe*, hipStream_t, int, const GemmArgs&,
                                              uint32_t);
template tsg_status routed_gemm_fused_launch<32, false>(const tsg_moe*, hipStream_t, GemmArgs, GemmArgs,
                                                    uint32_t);
template tsg_status dense_qmm_launch<32, false>(hipStream_t, const GemmArgs&, uint32_t);

}  // namespace tsg
