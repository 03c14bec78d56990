// Dense GEMM entry points (rh_gemm, rh_gemm_stage, rh_gemm_workspace_bytes, rh_gemm_kernel_name):
// validation, planning and dispatch.  The kernels and their launchers are in gemm_impl.hpp; the
// launchers of each operand layout are compiled in their own unit (gemm_nt.hip, gemm_nn.hip,
// gemm_tn.hip) so the three build in parallel.
#include "gemm_impl.hpp"

namespace rh_gemm_impl {

extern template int launch_layout<bf16_t, RH_GEMM_NT, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NT, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NT, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NT, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NT, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_NN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<bf16_t, RH_GEMM_TN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NT, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NT, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NT, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NT, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NT, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_NN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_TN, RH_EPI_NONE>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU_GRAD>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_TN, RH_EPI_GELU_DERIV>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_layout<float, RH_GEMM_TN, RH_EPI_MUL_AUX>(const rh_gemm_desc*, const Plan&, void*, hipStream_t, int);
extern template int launch_grouped<RH_GEMM_NT>(const rh_gemm_desc*, int, const GroupPlan&, void*, hipStream_t);
extern template int launch_grouped<RH_GEMM_NN>(const rh_gemm_desc*, int, const GroupPlan&, void*, hipStream_t);
extern template int launch_grouped<RH_GEMM_TN>(const rh_gemm_desc*, int, const GroupPlan&, void*, hipStream_t);

template <typename T, int EPI>
int launch_epi(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st, int stage) {
  switch (d->layout) {
    case RH_GEMM_NT: return launch_layout<T, RH_GEMM_NT, EPI>(d, pl, ws, st, stage);
    case RH_GEMM_NN: return launch_layout<T, RH_GEMM_NN, EPI>(d, pl, ws, st, stage);
    default: return launch_layout<T, RH_GEMM_TN, EPI>(d, pl, ws, st, stage);
  }
}

template <typename T>
int launch_dtype(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st, int stage) {
  switch (d->epilogue) {
    case RH_EPI_NONE: return launch_epi<T, RH_EPI_NONE>(d, pl, ws, st, stage);
    case RH_EPI_GELU: return launch_epi<T, RH_EPI_GELU>(d, pl, ws, st, stage);
    case RH_EPI_GELU_GRAD: return launch_epi<T, RH_EPI_GELU_GRAD>(d, pl, ws, st, stage);
    case RH_EPI_GELU_DERIV: return launch_epi<T, RH_EPI_GELU_DERIV>(d, pl, ws, st, stage);
    default: return launch_epi<T, RH_EPI_MUL_AUX>(d, pl, ws, st, stage);
  }
}

// Epilogue-only pass for K == 0 (acc = 0).
template <typename T, int EPI>
int launch_k0(const rh_gemm_desc* d, hipStream_t st) {
  Plan pl{kTf32, 1, 0, 0, 1, 1};
  GemmParams<T> p = make_params<T>(d, pl, nullptr);
  const int64_t total = d->M * d->N;
  int64_t blocks = rh_cdiv(total, 256);
  if (blocks > 4 * 1024) blocks = 4 * 1024;
  hipLaunchKernelGGL((gemm_splitk_reduce<T, EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, 0);
  return rh_check_launch("rh_gemm (K=0)");
}

}  // namespace rh_gemm_impl

using namespace rh_gemm_impl;

extern "C" int rh_gemm_kernel_name(const rh_gemm_desc* desc, char* buf, int64_t len) {
  int rc = validate(desc);
  if (rc) return rc;
  RH_REQUIRE(buf != nullptr && len > 0, "rh_gemm_kernel_name: null or empty buffer");
  if (desc->M == 0 || desc->N == 0) {
    snprintf(buf, (size_t)len, "none");
    return RH_OK;
  }
  if (desc->K == 0) {
    snprintf(buf, (size_t)len, "gemm_splitk_reduce<%s, %d>", desc->dtype == RH_DTYPE_BF16 ? "unsigned short" : "float",
             desc->epilogue);
    return RH_OK;
  }
  const Plan pl = plan_gemm(desc);
  const char* split = pl.splits + pl.tail > 1 ? "true" : "false";
  if (desc->dtype != RH_DTYPE_BF16) {
    snprintf(buf, (size_t)len, "gemm_f32_fma<%d, %d, %s>", desc->layout, pl.splits + pl.tail > 1 ? 0 : desc->epilogue,
             split);
    return RH_OK;
  }
  const GemmParams<bf16_t> p = make_params<bf16_t>(desc, pl, nullptr);
  const bool dma = dma_ok(desc, pl, p);
  const bool w4 = dma && pl.cfg == kT256x256 && four_wave_256(pl.splits > 1) && p.w4;  // as launch_cfg decides
  snprintf(buf, (size_t)len, "%s<%d, %d, %d, %d, %d, %d, %s>", dma ? "gemm_bf16_dma" : "gemm_bf16_mfma",
           kShapes[pl.cfg].bm, kShapes[pl.cfg].bn, kWaves[pl.cfg][0], w4 ? 2 : kWaves[pl.cfg][1], desc->layout,
           pl.splits + pl.tail > 1 ? 0 : desc->epilogue,  // split slices use the RH_EPI_NONE kernels
           split);
  return RH_OK;
}

extern "C" int rh_gemm_workspace_bytes(const rh_gemm_desc* desc, int64_t* bytes) {
  int rc = validate(desc);
  if (rc) return rc;
  RH_REQUIRE(bytes != nullptr, "rh_gemm_workspace_bytes: null output");
  *bytes = (desc->M == 0 || desc->N == 0 || desc->K == 0) ? 0 : plan_gemm(desc).ws_bytes;
  return RH_OK;
}

extern "C" int rh_gemm(const rh_gemm_desc* desc, void* workspace, int64_t workspace_bytes, void* stream) {
  return rh_gemm_stage(desc, workspace, workspace_bytes, RH_GEMM_STAGE_ALL, stream);
}

extern "C" int rh_gemm_stage(const rh_gemm_desc* desc, void* workspace, int64_t workspace_bytes, int stage,
                             void* stream) {
  int rc = validate(desc);
  if (rc) return rc;
  RH_REQUIRE(stage >= RH_GEMM_STAGE_ALL && stage <= RH_GEMM_STAGE_REDUCE, "rh_gemm_stage: unknown stage %d", stage);
  if (desc->M == 0 || desc->N == 0) return RH_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf16 = desc->dtype == RH_DTYPE_BF16;
  if (desc->K == 0) {
    if (stage == RH_GEMM_STAGE_REDUCE) return RH_OK;
    switch (desc->epilogue) {
      case RH_EPI_NONE: return bf16 ? launch_k0<bf16_t, RH_EPI_NONE>(desc, st) : launch_k0<float, RH_EPI_NONE>(desc, st);
      case RH_EPI_GELU: return bf16 ? launch_k0<bf16_t, RH_EPI_GELU>(desc, st) : launch_k0<float, RH_EPI_GELU>(desc, st);
      case RH_EPI_GELU_GRAD:
        return bf16 ? launch_k0<bf16_t, RH_EPI_GELU_GRAD>(desc, st) : launch_k0<float, RH_EPI_GELU_GRAD>(desc, st);
      case RH_EPI_GELU_DERIV:
        return bf16 ? launch_k0<bf16_t, RH_EPI_GELU_DERIV>(desc, st) : launch_k0<float, RH_EPI_GELU_DERIV>(desc, st);
      default: return bf16 ? launch_k0<bf16_t, RH_EPI_MUL_AUX>(desc, st) : launch_k0<float, RH_EPI_MUL_AUX>(desc, st);
    }
  }
  Plan pl = plan_gemm(desc);
  if (pl.splits + pl.tail > 1 && (workspace == nullptr || workspace_bytes < pl.ws_bytes || !rh_aligned(workspace, 16))) {
    pl.splits = 1;
    pl.tail = 0;
    pl.k_main = desc->K;
    pl.k_per_split = rh_cdiv(desc->K, bf16 ? kBK : fBK) * (bf16 ? kBK : fBK);
    pl.ws_bytes = 0;
  }
  return bf16 ? launch_dtype<bf16_t>(desc, pl, workspace, st, stage)
              : launch_dtype<float>(desc, pl, workspace, st, stage);
}

extern "C" int rh_gemm_grouped_workspace_bytes(const rh_gemm_desc* descs, int n, int64_t* bytes) {
  RH_REQUIRE(bytes != nullptr, "rh_gemm_grouped_workspace_bytes: null output");
  RH_REQUIRE(n >= 0 && (n == 0 || descs), "rh_gemm_grouped_workspace_bytes: bad descriptor list");
  int64_t most = 0;
  for (int i = 0; i < n; ++i) {
    int64_t b = 0;
    int rc = rh_gemm_workspace_bytes(&descs[i], &b);
    if (rc) return rc;
    most = std::max(most, b);
  }
  const GroupPlan g = plan_grouped(descs, n);
  *bytes = g.ok ? g.ws_off[n] : most;
  return RH_OK;
}

extern "C" int rh_gemm_grouped(const rh_gemm_desc* descs, int n, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  RH_REQUIRE(n >= 0 && (n == 0 || descs), "rh_gemm_grouped: bad descriptor list");
  for (int i = 0; i < n; ++i) {
    int rc = validate(&descs[i]);
    if (rc) return rc;
  }
  const GroupPlan g = plan_grouped(descs, n);
  const bool room = g.ok && (g.ws_off[n] == 0 || (workspace && workspace_bytes >= g.ws_off[n] && rh_aligned(workspace, 16)));
  if (!room) {  // one call per descriptor (each plans its own split within the same workspace)
    for (int i = 0; i < n; ++i) {
      int rc = rh_gemm(&descs[i], workspace, workspace_bytes, stream);
      if (rc) return rc;
    }
    return RH_OK;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (descs[0].layout) {
    case RH_GEMM_NT: return launch_grouped<RH_GEMM_NT>(descs, n, g, workspace, st);
    case RH_GEMM_NN: return launch_grouped<RH_GEMM_NN>(descs, n, g, workspace, st);
    default: return launch_grouped<RH_GEMM_TN>(descs, n, g, workspace, st);
  }
}

extern "C" int rh_gemm_grouped_kernel_name(const rh_gemm_desc* descs, int n, char* buf, int64_t len) {
  RH_REQUIRE(buf != nullptr && len > 0, "rh_gemm_grouped_kernel_name: null or empty buffer");
  RH_REQUIRE(n >= 0 && (n == 0 || descs), "rh_gemm_grouped_kernel_name: bad descriptor list");
  for (int i = 0; i < n; ++i) {
    int rc = validate(&descs[i]);
    if (rc) return rc;
  }
  const GroupPlan g = plan_grouped(descs, n);
  if (!g.ok) {
    snprintf(buf, (size_t)len, "none");
    return RH_OK;
  }
  bool w4 = four_wave_256(true);
  for (int i = 0; i < n; ++i) w4 = w4 && w4_addressable(&descs[i]);  // as launch_grouped decides
  snprintf(buf, (size_t)len, "gemm_bf16_dma_grouped<256, 256, 2, %d, %d, %s>", w4 ? 2 : 4, descs[0].layout,
           g.splits > 1 ? "true" : "false");
  return RH_OK;
}

extern "C" int rh_gemm_grouped_plan(const rh_gemm_desc* descs, int n, int* splits) {
  RH_REQUIRE(splits != nullptr && n >= 0 && (n == 0 || descs), "rh_gemm_grouped_plan: bad arguments");
  for (int i = 0; i < n; ++i) {
    int rc = validate(&descs[i]);
    if (rc) return rc;
  }
  const GroupPlan g = plan_grouped(descs, n);
  *splits = g.ok ? g.splits : 0;
  return RH_OK;
}
