// Elementwise kernels: GELU forward/backward, residual add, in-place scaling
// by a device scalar, and the SGD / AdamW parameter updates.  Grid-stride
// loops; every value is computed in fp32 and rounded once on store.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
  int64_t b = rh_cdiv(n, kThreads);
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return (unsigned)b;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gelu_fwd_kernel(int64_t n, const T* x, T* y) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    st_f32(y + i, std::is_same<T, bf16_t>::value ? gelu_fast_f(ld_f32(x + i)) : gelu_f(ld_f32(x + i)));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gelu_bwd_kernel(int64_t n, const T* x, const T* dy, T* dx) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    st_f32(dx + i, ld_f32(dy + i) * (std::is_same<T, bf16_t>::value ? gelu_grad_fast_f(ld_f32(x + i)) : gelu_grad_f(ld_f32(x + i))));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void add_kernel(int64_t n, const T* a, const T* b, T* out) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    st_f32(out + i, ld_f32(a + i) + ld_f32(b + i));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void scale_kernel(int64_t rows, int64_t cols, int64_t ld, T* x,
                                                          const float* scalar) {
  const float s = *scalar;
  if (s == 1.0f) return;
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    T* p = x + (i / cols) * ld + (i % cols);
    st_f32(p, ld_f32(p) * s);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void sgd_kernel(int64_t n, T* p, const T* g, float lr, float wd) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const float w = ld_f32(p + i);
    st_f32(p + i, w - lr * (ld_f32(g + i) + wd * w));
  }
}

// torch.optim.AdamW (single-tensor form): decoupled decay, then the moment
// updates, then p -= (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps).
template <typename T>
__global__ __launch_bounds__(kThreads) void adamw_kernel(int64_t n, T* p, const T* g, T* m, T* v, float lr, float b1,
                                                          float b2, float eps, float wd, float bc1, float bc2_sqrt) {
  const float step_size = lr / bc1;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    float w = ld_f32(p + i) * (1.0f - lr * wd);
    const float gr = ld_f32(g + i);
    float mv = ld_f32(m + i);
    mv = mv + (gr - mv) * (1.0f - b1);
    const float vv = ld_f32(v + i) * b2 + (1.0f - b2) * gr * gr;
    st_f32(m + i, mv);
    st_f32(v + i, vv);
    const float mq = ld_f32(m + i), vq = ld_f32(v + i);  // rounded moments, as torch stores them
    const float denom = sqrtf(vq) / bc2_sqrt + eps;
    w = w - step_size * (mq / denom);
    st_f32(p + i, w);
  }
}

int check_dtype(int dtype, const char* who) {
  if (dtype != RH_DTYPE_F32 && dtype != RH_DTYPE_BF16) return rh_set_error(RH_ERR_INVALID, "%s: unknown dtype %d", who, dtype);
  return RH_OK;
}

}  // namespace

extern "C" int rh_gelu_fwd(int dtype, int64_t n, const void* x, void* y, void* stream) {
  int rc = check_dtype(dtype, "rh_gelu_fwd");
  if (rc) return rc;
  RH_REQUIRE(n >= 0, "rh_gelu_fwd: negative n");
  if (n == 0) return RH_OK;
  RH_REQUIRE(x && y, "rh_gelu_fwd: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(gelu_fwd_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const bf16_t*)x, (bf16_t*)y);
  else
    hipLaunchKernelGGL(gelu_fwd_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const float*)x, (float*)y);
  return rh_check_launch("rh_gelu_fwd");
}

extern "C" int rh_gelu_bwd(int dtype, int64_t n, const void* x, const void* dy, void* dx, void* stream) {
  int rc = check_dtype(dtype, "rh_gelu_bwd");
  if (rc) return rc;
  RH_REQUIRE(n >= 0, "rh_gelu_bwd: negative n");
  if (n == 0) return RH_OK;
  RH_REQUIRE(x && dy && dx, "rh_gelu_bwd: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(gelu_bwd_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const bf16_t*)x,
                       (const bf16_t*)dy, (bf16_t*)dx);
  else
    hipLaunchKernelGGL(gelu_bwd_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const float*)x,
                       (const float*)dy, (float*)dx);
  return rh_check_launch("rh_gelu_bwd");
}

extern "C" int rh_add(int dtype, int64_t n, const void* a, const void* b, void* out, void* stream) {
  int rc = check_dtype(dtype, "rh_add");
  if (rc) return rc;
  RH_REQUIRE(n >= 0, "rh_add: negative n");
  if (n == 0) return RH_OK;
  RH_REQUIRE(a && b && out, "rh_add: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(add_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const bf16_t*)a,
                       (const bf16_t*)b, (bf16_t*)out);
  else
    hipLaunchKernelGGL(add_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (const float*)a,
                       (const float*)b, (float*)out);
  return rh_check_launch("rh_add");
}

extern "C" int rh_scale_by(int dtype, int64_t rows, int64_t cols, int64_t ld, void* x, const float* scalar,
                           void* stream) {
  int rc = check_dtype(dtype, "rh_scale_by");
  if (rc) return rc;
  RH_REQUIRE(rows >= 0 && cols >= 0 && ld >= cols, "rh_scale_by: bad extents");
  if (rows == 0 || cols == 0) return RH_OK;
  RH_REQUIRE(x && scalar, "rh_scale_by: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = grid_for(rows * cols);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(scale_kernel<bf16_t>, dim3(g), dim3(kThreads), 0, st, rows, cols, ld, (bf16_t*)x, scalar);
  else
    hipLaunchKernelGGL(scale_kernel<float>, dim3(g), dim3(kThreads), 0, st, rows, cols, ld, (float*)x, scalar);
  return rh_check_launch("rh_scale_by");
}

extern "C" int rh_sgd_step(int dtype, int64_t n, void* param, const void* grad, float lr, float weight_decay,
                           void* stream) {
  int rc = check_dtype(dtype, "rh_sgd_step");
  if (rc) return rc;
  RH_REQUIRE(n >= 0, "rh_sgd_step: negative n");
  if (n == 0) return RH_OK;
  RH_REQUIRE(param && grad, "rh_sgd_step: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(sgd_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (bf16_t*)param,
                       (const bf16_t*)grad, lr, weight_decay);
  else
    hipLaunchKernelGGL(sgd_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (float*)param,
                       (const float*)grad, lr, weight_decay);
  return rh_check_launch("rh_sgd_step");
}

extern "C" int rh_adamw_step(int dtype, int64_t n, void* param, const void* grad, void* exp_avg, void* exp_avg_sq,
                             float lr, float beta1, float beta2, float eps, float weight_decay, float bias_c1,
                             float bias_c2, void* stream) {
  int rc = check_dtype(dtype, "rh_adamw_step");
  if (rc) return rc;
  RH_REQUIRE(n >= 0, "rh_adamw_step: negative n");
  if (n == 0) return RH_OK;
  RH_REQUIRE(param && grad && exp_avg && exp_avg_sq, "rh_adamw_step: null pointer");
  RH_REQUIRE(bias_c1 > 0.f && bias_c2 > 0.f, "rh_adamw_step: bias corrections must be positive");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float bc2s = sqrtf(bias_c2);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(adamw_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (bf16_t*)param,
                       (const bf16_t*)grad, (bf16_t*)exp_avg, (bf16_t*)exp_avg_sq, lr, beta1, beta2, eps,
                       weight_decay, bias_c1, bc2s);
  else
    hipLaunchKernelGGL(adamw_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, n, (float*)param,
                       (const float*)grad, (float*)exp_avg, (float*)exp_avg_sq, lr, beta1, beta2, eps, weight_decay,
                       bias_c1, bc2s);
  return rh_check_launch("rh_adamw_step");
}
