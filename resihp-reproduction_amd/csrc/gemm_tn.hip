// GEMM launchers (and so kernels) of the TN operand layout, every dtype and epilogue; see
// gemm_impl.hpp.  One unit per layout so the builds run in parallel.
#include "gemm_impl.hpp"

namespace rh_gemm_impl {

template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<float, RH_GEMM_TN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_layout<float, RH_GEMM_TN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
template int launch_grouped<RH_GEMM_TN>(const rh_gemm_desc*, int, const GroupPlan&, void*, hipStream_t);

}  // namespace rh_gemm_impl
