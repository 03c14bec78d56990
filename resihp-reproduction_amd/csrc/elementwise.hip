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

// torch.optim.AdamW over many tensors in one launch.  Every workgroup takes one chunk of one
// tensor (block ranges per tensor in `block_end`), reads the tensor's device step count (already
// incremented by adamw_step_increment) and forms the bias corrections as torch does, in double
// precision, rounding to fp32 where torch's scalar arguments are.
constexpr int kMultiMax = 64;       // tensors per launch (the argument block stays under 4 KB)
constexpr int kMultiChunk = 8192;   // elements per workgroup

template <typename T>
struct AdamMultiArgs {
  T* p[kMultiMax];
  const T* g[kMultiMax];
  T* m[kMultiMax];
  T* v[kMultiMax];
  const float* step[kMultiMax];
  int64_t n[kMultiMax];
  int block_end[kMultiMax];
  int count;
  double lr, b1, b2, eps, wd;
};

__global__ __launch_bounds__(64) void adamw_step_increment(AdamMultiArgs<float> a) {
  if ((int)threadIdx.x < a.count) {
    float* s = const_cast<float*>(a.step[threadIdx.x]);
    *s = *s + 1.0f;
  }
}

// One AdamW update in fp32 of values read from T storage; returns the new param and moments as
// they are stored (the update divides by the stored, i.e. rounded, moments, as torch does).
template <typename T>
__device__ __forceinline__ void adamw_math(float& w, float gr, float& mv, float& vv, float decay, float omb1, float b2f,
                                           float omb2, float step_size, float bc2_sqrt, float eps) {
  w *= decay;
  mv = Storage<T>::to_f32(Storage<T>::from_f32(mv + (gr - mv) * omb1));
  vv = Storage<T>::to_f32(Storage<T>::from_f32(vv * b2f + omb2 * gr * gr));
  w = w - step_size * (mv / (sqrtf(vv) / bc2_sqrt + eps));
}

template <typename T>
__device__ __forceinline__ void adamw_update(T* p, const T* g, T* m, T* v, float decay, float omb1, float b2f,
                                             float omb2, float step_size, float bc2_sqrt, float eps) {
  float w = ld_f32(p), mv = ld_f32(m), vv = ld_f32(v);
  adamw_math<T>(w, ld_f32(g), mv, vv, decay, omb1, b2f, omb2, step_size, bc2_sqrt, eps);
  st_f32(m, mv);
  st_f32(v, vv);
  st_f32(p, w);
}

// Four consecutive elements per thread with one 16-byte (fp32) or 8-byte (bf16) access per array.
template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct Vec4<bf16_t> {
  typedef uint16_t type __attribute__((ext_vector_type(4)));
};
template <typename T>
__device__ __forceinline__ void adamw_update4(T* p, const T* g, T* m, T* v, float decay, float omb1, float b2f,
                                              float omb2, float step_size, float bc2_sqrt, float eps) {
  using V = typename Vec4<T>::type;
  V pv = *reinterpret_cast<const V*>(p), gv = *reinterpret_cast<const V*>(g);
  V mv4 = *reinterpret_cast<const V*>(m), vv4 = *reinterpret_cast<const V*>(v);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float w = Storage<T>::to_f32(pv[j]), mv = Storage<T>::to_f32(mv4[j]), vv = Storage<T>::to_f32(vv4[j]);
    adamw_math<T>(w, Storage<T>::to_f32(gv[j]), mv, vv, decay, omb1, b2f, omb2, step_size, bc2_sqrt, eps);
    pv[j] = Storage<T>::from_f32(w);
    mv4[j] = Storage<T>::from_f32(mv);
    vv4[j] = Storage<T>::from_f32(vv);
  }
  *reinterpret_cast<V*>(m) = mv4;
  *reinterpret_cast<V*>(v) = vv4;
  *reinterpret_cast<V*>(p) = pv;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void adamw_multi_kernel(AdamMultiArgs<T> a) {
  const int b = blockIdx.x;
  int t = 0;
  while (t + 1 < a.count && a.block_end[t] <= b) ++t;
  const int first = t ? a.block_end[t - 1] : 0;
  const int64_t lo = (int64_t)(b - first) * kMultiChunk;
  const int64_t hi = min(a.n[t], lo + kMultiChunk);
  const double s = (double)*a.step[t];
  const float step_size = (float)(a.lr / (1.0 - pow(a.b1, s)));
  const float bc2_sqrt = (float)sqrt(1.0 - pow(a.b2, s));
  const float decay = (float)(1.0 - a.lr * a.wd);
  const float omb1 = (float)(1.0 - a.b1), b2f = (float)a.b2, omb2 = (float)(1.0 - a.b2), eps = (float)a.eps;
  T* p = a.p[t];
  const T* g = a.g[t];
  T* m = a.m[t];
  T* v = a.v[t];
  const uintptr_t al = (uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v;
  int64_t i = lo;
  if (al % (4 * sizeof(T)) == 0) {  // chunk starts are multiples of 4 elements
    for (i = lo + 4 * (int64_t)threadIdx.x; i + 3 < hi; i += 4 * kThreads)
      adamw_update4(p + i, g + i, m + i, v + i, decay, omb1, b2f, omb2, step_size, bc2_sqrt, eps);
    i = lo + (hi - lo) / 4 * 4;  // the last < 4 elements of the chunk
  }
  for (i += threadIdx.x; i < hi; i += kThreads)
    adamw_update(p + i, g + i, m + i, v + i, decay, omb1, b2f, omb2, step_size, bc2_sqrt, eps);
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

extern "C" int rh_adamw_multi(int dtype, int n_tensors, const rh_adamw_tensor* tensors, double lr, double beta1,
                              double beta2, double eps, double weight_decay, void* stream) {
  int rc = check_dtype(dtype, "rh_adamw_multi");
  if (rc) return rc;
  RH_REQUIRE(n_tensors >= 0, "rh_adamw_multi: negative tensor count");
  if (n_tensors == 0) return RH_OK;
  RH_REQUIRE(tensors != nullptr, "rh_adamw_multi: null tensor list");
  RH_REQUIRE(lr >= 0 && eps >= 0 && weight_decay >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1,
             "rh_adamw_multi: invalid hyperparameters");
  for (int i = 0; i < n_tensors; ++i) {
    const rh_adamw_tensor& t = tensors[i];
    RH_REQUIRE(t.numel >= 0, "rh_adamw_multi: tensor %d has a negative size", i);
    RH_REQUIRE(t.numel == 0 || (t.param && t.grad && t.exp_avg && t.exp_avg_sq), "rh_adamw_multi: tensor %d: null pointer", i);
    RH_REQUIRE(t.step, "rh_adamw_multi: tensor %d: null step counter", i);
    for (int j = 0; j < i; ++j)
      RH_REQUIRE(tensors[j].step != t.step, "rh_adamw_multi: tensors %d and %d share a step counter", j, i);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int base = 0; base < n_tensors; base += kMultiMax) {
    const int cnt = min(kMultiMax, n_tensors - base);
    AdamMultiArgs<float> a{};  // pointers are reinterpreted per dtype below; the layout is identical
    int64_t blocks = 0;
    for (int i = 0; i < cnt; ++i) {
      const rh_adamw_tensor& t = tensors[base + i];
      a.p[i] = (float*)t.param;
      a.g[i] = (const float*)t.grad;
      a.m[i] = (float*)t.exp_avg;
      a.v[i] = (float*)t.exp_avg_sq;
      a.step[i] = t.step;
      a.n[i] = t.numel;
      blocks += rh_cdiv(t.numel, kMultiChunk);
      RH_REQUIRE(blocks <= INT32_MAX, "rh_adamw_multi: too many elements in one launch");
      a.block_end[i] = (int)blocks;
    }
    a.count = cnt;
    a.lr = lr;
    a.b1 = beta1;
    a.b2 = beta2;
    a.eps = eps;
    a.wd = weight_decay;
    hipLaunchKernelGGL(adamw_step_increment, dim3(1), dim3(64), 0, st, a);
    rc = rh_check_launch("rh_adamw_multi (step count)");
    if (rc) return rc;
    if (blocks == 0) continue;
    if (dtype == RH_DTYPE_BF16) {
      AdamMultiArgs<bf16_t> ab;
      static_assert(sizeof(ab) == sizeof(a), "argument layouts must match");
      __builtin_memcpy(&ab, &a, sizeof(a));
      hipLaunchKernelGGL(adamw_multi_kernel<bf16_t>, dim3((unsigned)blocks), dim3(kThreads), 0, st, ab);
    } else {
      hipLaunchKernelGGL(adamw_multi_kernel<float>, dim3((unsigned)blocks), dim3(kThreads), 0, st, a);
    }
    rc = rh_check_launch("rh_adamw_multi");
    if (rc) return rc;
  }
  return RH_OK;
}
