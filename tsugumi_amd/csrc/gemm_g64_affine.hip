// gemm_g64_affine.hip — the grouped GEMM kernels for group size 64, affine scheme.
#include "prefill_gemm_impl.hpp"

namespace tsg {

template tsg_status routed_gemm_launch<64, false>(const tsg_moe*, hipStream_t, int, const GemmArgs&,
                                              uint32_t);
template tsg_status routed_gemm_fused_launch<64, false>(const tsg_moe*, hipStream_t, GemmArgs, GemmArgs,
                                                    uint32_t);
template tsg_status dense_qmm_launch<64, false>(hipStream_t, const GemmArgs&, uint32_t);

}  // namespace tsg
