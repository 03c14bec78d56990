// Next-token softmax cross-entropy over [batch, seq, vocab] logits, forward and
// backward, without materialising logits[:, :-1] or a one-hot matrix.
//
// One 256-thread block per logits row.  Pass 1 streams the row once with
// 16-byte loads and keeps a per-thread online (max, sum-exp) pair, merged
// across the block.  When the gradient is wanted in the same call, pass 2
// re-reads the row and writes
//   dlogits = (exp(x - lse) - [j == target]) / N.
// bf16 rows of up to 65536 aligned logits take xent_fwd_grad_reg_kernel instead,
// which holds the row in registers between the two passes, so the fused
// forward+backward moves 2 bytes in and 2 bytes out per logit.  Row losses are reduced to the mean by a single block in a fixed
// order (deterministic).
#include "common.hpp"

namespace {

constexpr int kT = 256;

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    const u16x8_t u = *reinterpret_cast<const u16x8_t*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = bf16_to_f32(u[j]);
  } else {
    const floatx4_t a = *reinterpret_cast<const floatx4_t*>(p);
    const floatx4_t b = *reinterpret_cast<const floatx4_t*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    u16x8_t u;
#pragma unroll
    for (int j = 0; j < 8; ++j) u[j] = f32_to_bf16(v[j]);
    *reinterpret_cast<u16x8_t*>(p) = u;
  } else {
    floatx4_t a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) { a[j] = v[j]; b[j] = v[4 + j]; }
    *reinterpret_cast<floatx4_t*>(p) = a;
    *reinterpret_cast<floatx4_t*>(p + 4) = b;
  }
}

// Row log-sum-exp.  VEC: row start 16-byte aligned -> 8-wide loads.
// exp(x) as the hardware base-2 exponential of x*log2(e) (v_exp_f32, ~1 ulp): the online
// log-sum-exp below runs in base-2 units (m2 = max * log2 e), one FMA + one v_exp per logit.
constexpr float kLog2eX = 1.4426950408889634074f;
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T, bool VEC>
__device__ float row_lse(const T* x, int64_t V, float* scratch) {
  float m = -INFINITY, s = 0.f;  // m: running max in base-2 units; s: sum of 2^(x*log2e - m)
  auto add = [&](float cm2, const float* v, int n) {
    const float mn = fmaxf(m, cm2);
    float acc = (m == -INFINITY) ? 0.f : s * exp2_hw(m - mn);
    for (int t = 0; t < n; ++t) acc += exp2_hw(fmaf(v[t], kLog2eX, -mn));
    s = acc;
    m = mn;
  };
  if (VEC) {
    const int64_t full = V / 8 * 8;
    int64_t j = (int64_t)threadIdx.x * 8;
    // two 8-element chunks per trip: both loads in flight before the math
    for (; j + kT * 8 < full; j += 2 * kT * 8) {
      float v[8], w[8];
      load8<T>(x + j, v);
      load8<T>(x + j + kT * 8, w);
      float cm = fmaxf(v[0], w[0]);
#pragma unroll
      for (int t = 1; t < 8; ++t) cm = fmaxf(cm, fmaxf(v[t], w[t]));
      const float mn = fmaxf(m, cm * kLog2eX);
      float acc = (m == -INFINITY) ? 0.f : s * exp2_hw(m - mn);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc += exp2_hw(fmaf(v[t], kLog2eX, -mn)) + exp2_hw(fmaf(w[t], kLog2eX, -mn));
      s = acc;
      m = mn;
    }
    for (; j < full; j += kT * 8) {
      float v[8];
      load8<T>(x + j, v);
      float cm = v[0];
#pragma unroll
      for (int t = 1; t < 8; ++t) cm = fmaxf(cm, v[t]);
      add(cm * kLog2eX, v, 8);
    }
    for (int64_t k = full + threadIdx.x; k < V; k += kT) {
      const float v = ld_f32(x + k);
      add(v * kLog2eX, &v, 1);
    }
  } else {
    for (int64_t k = threadIdx.x; k < V; k += kT) {
      const float v = ld_f32(x + k);
      add(v * kLog2eX, &v, 1);
    }
  }
  const float M = block_max(m, scratch);
  const float part = (m == -INFINITY) ? 0.f : s * exp2_hw(m - M);
  const float tot = block_sum(part, scratch + 8);
  return (M + log2f(tot)) * 0.69314718055994530942f;  // natural-log units
}

template <typename T, bool VEC>
__device__ void row_grad(const T* x, T* d, int64_t V, int64_t ld_d, float lse, int64_t tgt, float scale) {
  if (VEC) {
    const int64_t full = V / 8 * 8;
    for (int64_t j = (int64_t)threadIdx.x * 8; j < full; j += kT * 8) {
      float v[8];
      load8<T>(x + j, v);
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = (expf(v[t] - lse) - ((j + t) == tgt ? 1.f : 0.f)) * scale;
      store8<T>(d + j, v);
    }
    for (int64_t j = full + threadIdx.x; j < V; j += kT)
      st_f32(d + j, (expf(ld_f32(x + j) - lse) - (j == tgt ? 1.f : 0.f)) * scale);
  } else {
    for (int64_t j = threadIdx.x; j < V; j += kT)
      st_f32(d + j, (expf(ld_f32(x + j) - lse) - (j == tgt ? 1.f : 0.f)) * scale);
  }
  for (int64_t j = V + threadIdx.x; j < ld_d; j += kT) st_f32(d + j, 0.f);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kT) void xent_fwd_kernel(int S, int64_t V, const T* __restrict__ logits, int64_t ld,
                                                       const int64_t* __restrict__ tokens, float* __restrict__ lse_out,
                                                       float* __restrict__ loss_rows, T* dl, int64_t ld_d,
                                                       float inv_n) {
  __shared__ float scratch[16];
  const int64_t row = blockIdx.x;
  const int64_t s = row % S;
  const T* x = logits + row * ld;
  if (s == S - 1) {
    if (threadIdx.x == 0) {
      loss_rows[row] = 0.f;
      lse_out[row] = 0.f;
    }
    if (dl)
      for (int64_t j = threadIdx.x; j < ld_d; j += kT) st_f32(dl + row * ld_d + j, 0.f);
    return;
  }
  const float lse = row_lse<T, VEC>(x, V, scratch);
  const int64_t tgt = tokens[row + 1];
  if (threadIdx.x == 0) {
    const float xt = (tgt >= 0 && tgt < V) ? ld_f32(x + tgt) : NAN;
    loss_rows[row] = lse - xt;
    lse_out[row] = lse;
  }
  if (dl) row_grad<T, VEC>(x, dl + row * ld_d, V, ld_d, lse, tgt, inv_n);
}

// bf16 rows of up to kRegCols logits with the gradient wanted in the same call: the row is read
// once into registers (512 threads x 16 chunks of 8), its max and sum-exp come from the registers,
// and the gradient is written from them, so the fused forward moves 2 bytes in and 2 bytes out per
// logit with no second read of the row.  16-byte aligned rows (ld % 8 == 0).
constexpr int kRT = 512, kRC = 16;
constexpr int64_t kRegCols = (int64_t)kRT * kRC * 8;
__global__ __launch_bounds__(kRT) void xent_fwd_grad_reg_kernel(int S, int64_t V, const bf16_t* __restrict__ logits,
                                                                int64_t ld, const int64_t* __restrict__ tokens,
                                                                float* __restrict__ lse_out, float* __restrict__ loss_rows,
                                                                bf16_t* __restrict__ dl, int64_t ld_d, float inv_n) {
  __shared__ float scratch[32];
  const int64_t row = blockIdx.x;
  const int64_t s = row % S;
  bf16_t* drow = dl + row * ld_d;
  if (s == S - 1) {
    if (threadIdx.x == 0) {
      loss_rows[row] = 0.f;
      lse_out[row] = 0.f;
    }
    const u16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t j = (int64_t)threadIdx.x * 8; j < ld_d; j += kRT * 8) *reinterpret_cast<u16x8_t*>(drow + j) = z;
    return;
  }
  const bf16_t* x = logits + row * ld;
  const int64_t full = V / 8 * 8;
  // chunk c of this thread: columns (c * kRT + tid) * 8 .. + 7; the last V % 8 columns (one per
  // thread, tid < V % 8) in `tail`
  u16x8_t raw[kRC];
  float cm = -INFINITY;
#pragma unroll
  for (int c = 0; c < kRC; ++c) {
    const int64_t j = ((int64_t)c * kRT + threadIdx.x) * 8;
    raw[c] = u16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
    if (j < full) raw[c] = *reinterpret_cast<const u16x8_t*>(x + j);
  }
  const int64_t jt = full + threadIdx.x;
  const float tail = jt < V ? bf16_to_f32(x[jt]) : -INFINITY;
#pragma unroll
  for (int c = 0; c < kRC; ++c) {
    const int64_t j = ((int64_t)c * kRT + threadIdx.x) * 8;
#pragma unroll
    for (int t = 0; t < 8; ++t) cm = fmaxf(cm, j < full ? bf16_to_f32(raw[c][t]) : -INFINITY);
  }
  cm = fmaxf(cm, tail);
  const float M2 = block_max(cm, scratch) * kLog2eX;  // row max, base-2 units
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < kRC; ++c) {
    const int64_t j = ((int64_t)c * kRT + threadIdx.x) * 8;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float e = exp2_hw(fmaf(bf16_to_f32(raw[c][t]), kLog2eX, -M2));
      sum += j < full ? e : 0.f;
    }
  }
  sum += jt < V ? exp2_hw(fmaf(tail, kLog2eX, -M2)) : 0.f;
  const float tot = block_sum(sum, scratch + 16);
  const float lse2 = M2 + log2f(tot);  // base-2 units
  const float lse = lse2 * 0.69314718055994530942f;
  const int64_t tgt = tokens[row + 1];
  if (threadIdx.x == 0) {
    const float xt = (tgt >= 0 && tgt < V) ? bf16_to_f32(x[tgt]) : NAN;
    loss_rows[row] = lse - xt;
    lse_out[row] = lse;
  }
#pragma unroll
  for (int c = 0; c < kRC; ++c) {
    const int64_t j = ((int64_t)c * kRT + threadIdx.x) * 8;
    if (j >= full) continue;
    u16x8_t o;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float g = exp2_hw(fmaf(bf16_to_f32(raw[c][t]), kLog2eX, -lse2)) - (j + t == tgt ? 1.f : 0.f);
      o[t] = f32_to_bf16(g * inv_n);
    }
    *reinterpret_cast<u16x8_t*>(drow + j) = o;
  }
  if (jt < V) drow[jt] = f32_to_bf16((exp2_hw(fmaf(tail, kLog2eX, -lse2)) - (jt == tgt ? 1.f : 0.f)) * inv_n);
  for (int64_t j = V + threadIdx.x; j < ld_d; j += kRT) drow[j] = f32_to_bf16(0.f);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kT) void xent_bwd_kernel(int S, int64_t V, const T* __restrict__ logits, int64_t ld,
                                                       const int64_t* __restrict__ tokens,
                                                       const float* __restrict__ lse_in, const float* grad_loss,
                                                       T* dl, int64_t ld_d, float inv_n) {
  const int64_t row = blockIdx.x;
  const int64_t s = row % S;
  if (s == S - 1) {
    for (int64_t j = threadIdx.x; j < ld_d; j += kT) st_f32(dl + row * ld_d + j, 0.f);
    return;
  }
  const float scale = inv_n * (grad_loss ? *grad_loss : 1.f);
  row_grad<T, VEC>(logits + row * ld, dl + row * ld_d, V, ld_d, lse_in[row], tokens[row + 1], scale);
}

__global__ __launch_bounds__(1024) void mean_kernel(int64_t n, const float* __restrict__ rows, float inv_n,
                                                    float* __restrict__ out) {
  __shared__ float scratch[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += rows[i];
  const float tot = block_sum(s, scratch);
  if (threadIdx.x == 0) out[0] = tot * inv_n;
}

int check_xent(int dtype, int64_t B, int64_t S, int64_t V, int64_t ld) {
  RH_REQUIRE(dtype == RH_DTYPE_F32 || dtype == RH_DTYPE_BF16, "rh_xent: unknown dtype %d", dtype);
  RH_REQUIRE(B >= 1 && S >= 2, "rh_xent: need batch >= 1 and seq >= 2 (got %lld, %lld)", (long long)B, (long long)S);
  RH_REQUIRE(V >= 1 && ld >= V, "rh_xent: vocab %lld / ld %lld invalid", (long long)V, (long long)ld);
  RH_REQUIRE(B * S <= INT32_MAX, "rh_xent: too many rows");
  return RH_OK;
}

}  // namespace

extern "C" int rh_xent_workspace_bytes(int64_t batch, int64_t seq, int64_t* bytes) {
  RH_REQUIRE(bytes && batch >= 0 && seq >= 0, "rh_xent_workspace_bytes: bad arguments");
  *bytes = batch * seq * (int64_t)sizeof(float);
  return RH_OK;
}

extern "C" int rh_xent_fwd(int dtype, int64_t batch, int64_t seq, int64_t vocab, const void* logits, int64_t ld,
                           const int64_t* tokens, float* row_lse, float* loss, void* dlogits, int64_t ld_d,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_xent(dtype, batch, seq, vocab, ld);
  if (rc) return rc;
  RH_REQUIRE(logits && tokens && row_lse && loss, "rh_xent_fwd: null pointer");
  if (dlogits) RH_REQUIRE(ld_d >= vocab, "rh_xent_fwd: ld_d %lld < vocab", (long long)ld_d);
  RH_REQUIRE(workspace && workspace_bytes >= batch * seq * (int64_t)sizeof(float),
             "rh_xent_fwd: workspace of %lld bytes is too small", (long long)workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* rows = static_cast<float*>(workspace);
  const int64_t nrows = batch * seq;
  const float inv_n = 1.0f / (float)(batch * (seq - 1));
  const bool vec = rh_aligned(logits, 16) && ld % 8 == 0 && (!dlogits || (rh_aligned(dlogits, 16) && ld_d % 8 == 0));
  if (dtype == RH_DTYPE_BF16) {
    if (vec && dlogits && vocab <= kRegCols)
      hipLaunchKernelGGL(xent_fwd_grad_reg_kernel, dim3((unsigned)nrows), dim3(kRT), 0, st, (int)seq, vocab,
                         (const bf16_t*)logits, ld, tokens, row_lse, rows, (bf16_t*)dlogits, ld_d, inv_n);
    else if (vec) hipLaunchKernelGGL((xent_fwd_kernel<bf16_t, true>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                                (const bf16_t*)logits, ld, tokens, row_lse, rows, (bf16_t*)dlogits, ld_d, inv_n);
    else hipLaunchKernelGGL((xent_fwd_kernel<bf16_t, false>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                            (const bf16_t*)logits, ld, tokens, row_lse, rows, (bf16_t*)dlogits, ld_d, inv_n);
  } else {
    if (vec) hipLaunchKernelGGL((xent_fwd_kernel<float, true>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                                (const float*)logits, ld, tokens, row_lse, rows, (float*)dlogits, ld_d, inv_n);
    else hipLaunchKernelGGL((xent_fwd_kernel<float, false>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                            (const float*)logits, ld, tokens, row_lse, rows, (float*)dlogits, ld_d, inv_n);
  }
  rc = rh_check_launch("rh_xent_fwd");
  if (rc) return rc;
  hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(1024), 0, st, nrows, rows, inv_n, loss);
  return rh_check_launch("rh_xent_fwd mean");
}

extern "C" int rh_xent_bwd(int dtype, int64_t batch, int64_t seq, int64_t vocab, const void* logits, int64_t ld,
                           const int64_t* tokens, const float* row_lse, const float* grad_loss, void* dlogits,
                           int64_t ld_d, void* stream) {
  int rc = check_xent(dtype, batch, seq, vocab, ld);
  if (rc) return rc;
  RH_REQUIRE(logits && tokens && row_lse && dlogits, "rh_xent_bwd: null pointer");
  RH_REQUIRE(ld_d >= vocab, "rh_xent_bwd: ld_d %lld < vocab", (long long)ld_d);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nrows = batch * seq;
  const float inv_n = 1.0f / (float)(batch * (seq - 1));
  const bool vec = rh_aligned(logits, 16) && ld % 8 == 0 && rh_aligned(dlogits, 16) && ld_d % 8 == 0;
  if (dtype == RH_DTYPE_BF16) {
    if (vec) hipLaunchKernelGGL((xent_bwd_kernel<bf16_t, true>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                                (const bf16_t*)logits, ld, tokens, row_lse, grad_loss, (bf16_t*)dlogits, ld_d, inv_n);
    else hipLaunchKernelGGL((xent_bwd_kernel<bf16_t, false>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                            (const bf16_t*)logits, ld, tokens, row_lse, grad_loss, (bf16_t*)dlogits, ld_d, inv_n);
  } else {
    if (vec) hipLaunchKernelGGL((xent_bwd_kernel<float, true>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                                (const float*)logits, ld, tokens, row_lse, grad_loss, (float*)dlogits, ld_d, inv_n);
    else hipLaunchKernelGGL((xent_bwd_kernel<float, false>), dim3((unsigned)nrows), dim3(kT), 0, st, (int)seq, vocab,
                            (const float*)logits, ld, tokens, row_lse, grad_loss, (float*)dlogits, ld_d, inv_n);
  }
  return rh_check_launch("rh_xent_bwd");
}
