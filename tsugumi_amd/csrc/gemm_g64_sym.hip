// gemm_g64_sym.hip — the grouped GEMM kernels for group size 64, symmetric scheme.
#include "prefill_gemm_impl.hpp"

namespace tsg {

template tsg_status routed_gemm_launch<64, true>(const tsg_moe*, hipStream_t, int, const GemmArgs&,
                                              uint32_t);
template tsg_status routed_gemm_fused_launch<64, true>(const tsg_moe*, hipStream_t, GemmArgs, GemmArgs,
                                                    uint32_t);
template tsg_status dense_qmm_launch<64, true>(hipStream_t, const GemmArgs&, uint32_t);

}  // namespace tsg
