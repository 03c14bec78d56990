// LayerNorm over the last dimension (eps, biased variance) and its backward,
// as bandwidth-bound kernels: one wavefront per row, the row held in registers,
// shuffle reductions, fp32 statistics.
//
// Forward reads x once and writes y once (plus 8 bytes of stats per row).
// Backward reads dy, x (and the optional residual gradient) once and writes dx
// once; the gamma/beta column sums are accumulated per lane across the rows a
// wave visits, combined across the block's waves in LDS, written as one fp32
// partial row per block, and summed over blocks in block order by a second
// kernel (deterministic, no atomics).
#include <algorithm>

#include "common.hpp"

namespace {

// Row element e of lane l:  V == 8 : column 8*(l + 64*(e/8)) + e%8   (16-byte chunks)
//                           V == 1 : column l + 64*e                  (scalar)
template <int V>
__device__ __forceinline__ int col_of(int lane, int e) {
  return V == 8 ? 8 * (lane + 64 * (e / 8)) + (e % 8) : lane + 64 * e;
}

template <typename T, int V>
__device__ __forceinline__ void load_v(const T* p, float* out) {
  if constexpr (V == 1) {
    out[0] = ld_f32(p);
  } else if constexpr (std::is_same<T, bf16_t>::value) {
    const u16x8_t u = *reinterpret_cast<const u16x8_t*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = bf16_to_f32(u[j]);
  } else {
    const floatx4_t a = *reinterpret_cast<const floatx4_t*>(p);
    const floatx4_t b = *reinterpret_cast<const floatx4_t*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) { out[j] = a[j]; out[4 + j] = b[j]; }
  }
}

template <typename T, int V>
__device__ __forceinline__ void store_v(T* p, const float* in) {
  if constexpr (V == 1) {
    st_f32(p, in[0]);
  } else if constexpr (std::is_same<T, bf16_t>::value) {
    u16x8_t u;
#pragma unroll
    for (int j = 0; j < 8; ++j) u[j] = f32_to_bf16(in[j]);
    *reinterpret_cast<u16x8_t*>(p) = u;
  } else {
    floatx4_t a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) { a[j] = in[j]; b[j] = in[4 + j]; }
    *reinterpret_cast<floatx4_t*>(p) = a;
    *reinterpret_cast<floatx4_t*>(p + 4) = b;
  }
}

// E = register elements per lane (multiple of V).  Elements with column >= dim
// are skipped (loads give 0).
template <typename T, int V, int E>
__global__ __launch_bounds__(256) void ln_fwd_kernel(int64_t rows, int dim, const T* __restrict__ x,
                                                      const T* __restrict__ gamma, const T* __restrict__ beta,
                                                      float eps, T* __restrict__ y, float* __restrict__ mean,
                                                      float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * dim;
  float v[E];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < E; e += V) {
    const int c = col_of<V>(lane, e);
    if (c < dim) load_v<T, V>(xr + c, v + e);
    else
#pragma unroll
      for (int j = 0; j < V; ++j) v[e + j] = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += v[e + j];
  }
  const float mu = wave_sum(s) / (float)dim;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < E; e += V) {
    const int c = col_of<V>(lane, e);
    if (c < dim)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float d = v[e + j] - mu;
        q += d * d;
      }
  }
  const float var = wave_sum(q) / (float)dim;
  const float rs = 1.0f / sqrtf(var + eps);
  T* yr = y + row * dim;
#pragma unroll
  for (int e = 0; e < E; e += V) {
    const int c = col_of<V>(lane, e);
    if (c >= dim) continue;
    float gv[V], bv[V], o[V];
    load_v<T, V>(gamma + c, gv);
    load_v<T, V>(beta + c, bv);
#pragma unroll
    for (int j = 0; j < V; ++j) o[j] = (v[e + j] - mu) * rs * gv[j] + bv[j];
    store_v<T, V>(yr + c, o);
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// bf16 rows, dim % 8 == 0, dim <= 512*C, 16-byte aligned: the fast forward.  A wave walks rows
// blockIdx*4 + wave, + 4*gridDim, ... with the next row's loads in flight while the current one
// is reduced and written, and gamma / beta held in registers across rows.  Same arithmetic, in
// the same order, as ln_fwd_kernel<bf16_t, 8, 8*C> (bit-identical results).
template <int C>
__global__ __launch_bounds__(256) void ln_fwd_bf16_kernel(int64_t rows, int dim, const bf16_t* __restrict__ x,
                                                           const bf16_t* __restrict__ gamma,
                                                           const bf16_t* __restrict__ beta, float eps,
                                                           bf16_t* __restrict__ y, float* __restrict__ mean,
                                                           float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const u16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
  bool ok[C];
  u16x8_t gm[C], bt[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int col = 8 * (lane + 64 * c);
    ok[c] = col < dim;
    gm[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(gamma + col) : z;
    bt[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(beta + col) : z;
  }
  const int64_t stride = (int64_t)gridDim.x * 4;
  auto load = [&](int64_t row, u16x8_t(&v)[C]) {
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(x + row * dim + 8 * (lane + 64 * c)) : z;
  };
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  u16x8_t cur[C];
  if (row < rows) load(row, cur);
  for (; row < rows; row += stride) {
    u16x8_t nxt[C];
    if (row + stride < rows) load(row + stride, nxt);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += bf16_to_f32(cur[c][j]);
    const float mu = wave_sum(s) / (float)dim;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (ok[c])
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float d = bf16_to_f32(cur[c][j]) - mu;
          q += d * d;
        }
    const float var = wave_sum(q) / (float)dim;
    const float rs = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (!ok[c]) continue;
      u16x8_t o;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        o[j] = f32_to_bf16((bf16_to_f32(cur[c][j]) - mu) * rs * bf16_to_f32(gm[c][j]) + bf16_to_f32(bt[c][j]));
      *reinterpret_cast<u16x8_t*>(y + row * dim + 8 * (lane + 64 * c)) = o;
    }
    if (lane == 0) {
      mean[row] = mu;
      rstd[row] = rs;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) cur[c] = nxt[c];
  }
}

template <typename T, int V, int E>
__global__ __launch_bounds__(256) void ln_bwd_kernel(int64_t rows, int dim, const T* __restrict__ dy,
                                                      const T* __restrict__ x, const float* __restrict__ mean,
                                                      const float* __restrict__ rstd, const T* __restrict__ gamma,
                                                      const T* __restrict__ dres, T* __restrict__ dx,
                                                      float* __restrict__ part_g, float* __restrict__ part_b) {
  __shared__ float red[2][4][64 * 8];  // per-wave column partials for one chunk row (reused per e)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float pg[E], pb[E], gmm[E];
#pragma unroll
  for (int e = 0; e < E; e += V) {
    const int c = col_of<V>(lane, e);
    if (c < dim) load_v<T, V>(gamma + c, gmm + e);
    else
#pragma unroll
      for (int j = 0; j < V; ++j) gmm[e + j] = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) { pg[e + j] = 0.f; pb[e + j] = 0.f; }
  }
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < rows; row += (int64_t)gridDim.x * 4) {
    const T* dyr = dy + row * dim;
    const T* xr = x + row * dim;
    const float mu = mean[row], rs = rstd[row];
    float xh[E], g[E];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int e = 0; e < E; e += V) {
      const int c = col_of<V>(lane, e);
      float dv[V], xv[V];
      if (c < dim) {
        load_v<T, V>(dyr + c, dv);
        load_v<T, V>(xr + c, xv);
      } else {
#pragma unroll
        for (int j = 0; j < V; ++j) { dv[j] = 0.f; xv[j] = mu; }
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float h = (xv[j] - mu) * rs;
        xh[e + j] = h;
        g[e + j] = dv[j] * gmm[e + j];
        s1 += g[e + j];
        s2 += g[e + j] * h;
        pg[e + j] += dv[j] * h;
        pb[e + j] += dv[j];
      }
    }
    const float m1 = wave_sum(s1) / (float)dim;
    const float m2 = wave_sum(s2) / (float)dim;
    T* dxr = dx + row * dim;
    const T* drr = dres ? dres + row * dim : nullptr;
#pragma unroll
    for (int e = 0; e < E; e += V) {
      const int c = col_of<V>(lane, e);
      if (c >= dim) continue;
      float o[V], rv[V];
      if (drr) load_v<T, V>(drr + c, rv);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        o[j] = rs * (g[e + j] - m1 - xh[e + j] * m2);
        if (drr) o[j] += rv[j];
      }
      store_v<T, V>(dxr + c, o);
    }
  }
  // combine the 4 waves' column partials, one V-chunk of columns at a time
#pragma unroll
  for (int e = 0; e < E; e += V) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      red[0][wave][lane * V + j] = pg[e + j];
      red[1][wave][lane * V + j] = pb[e + j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * V; i += 256) {
      const int ln = i / V, j = i % V;
      const int col = V == 8 ? 8 * (ln + 64 * (e / 8)) + j : ln + 64 * e;
      if (col < dim) {
        const float sg = red[0][0][i] + red[0][1][i] + red[0][2][i] + red[0][3][i];
        const float sb = red[1][0][i] + red[1][1][i] + red[1][2][i] + red[1][3][i];
        part_g[(int64_t)blockIdx.x * dim + col] = sg;
        part_b[(int64_t)blockIdx.x * dim + col] = sb;
      }
    }
    __syncthreads();
  }
}

// bf16 rows, dim % 8 == 0: the fast backward.  Lane l owns the 16-byte chunks l + 64c
// (c < C) of every row.  All loads of a row (dy, x, residual gradient) are issued together and
// the next row's are in flight while the current one is reduced and written, so each wave
// keeps ~3*C*16 bytes per lane moving; column partials as in ln_bwd_kernel.
template <int C>
__global__ __launch_bounds__(256) void ln_bwd_bf16_kernel(int64_t rows, int dim, const bf16_t* __restrict__ dy,
                                                           const bf16_t* __restrict__ x, const float* __restrict__ mean,
                                                           const float* __restrict__ rstd,
                                                           const bf16_t* __restrict__ gamma,
                                                           const bf16_t* __restrict__ dres, bf16_t* __restrict__ dx,
                                                           float* __restrict__ part_g, float* __restrict__ part_b) {
  __shared__ float red[2][4][64 * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const u16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
  bool ok[C];
  u16x8_t gm[C];
  float pg[C][8], pb[C][8];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    ok[c] = 8 * (lane + 64 * c) < dim;
    gm[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(gamma + 8 * (lane + 64 * c)) : z;
#pragma unroll
    for (int j = 0; j < 8; ++j) pg[c][j] = pb[c][j] = 0.f;
  }
  const int64_t stride = (int64_t)gridDim.x * 4;
  auto load = [&](int64_t row, u16x8_t(&a)[C], u16x8_t(&b)[C], u16x8_t(&r)[C]) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t off = row * dim + 8 * (lane + 64 * c);
      a[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(dy + off) : z;
      b[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(x + off) : z;
      r[c] = (ok[c] && dres) ? *reinterpret_cast<const u16x8_t*>(dres + off) : z;
    }
  };
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  u16x8_t a[C], b[C], r[C];
  if (row < rows) load(row, a, b, r);
  for (; row < rows; row += stride) {
    u16x8_t na[C], nb[C], nr[C];
    if (row + stride < rows) load(row + stride, na, nb, nr);
    const float mu = mean[row], rs = rstd[row];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float dv = bf16_to_f32(a[c][j]);
        const float h = (bf16_to_f32(b[c][j]) - mu) * rs;
        const float g = dv * bf16_to_f32(gm[c][j]);
        s1 += g;
        s2 += g * h;
        pg[c][j] += dv * h;
        pb[c][j] += dv;
      }
    const float m1 = wave_sum(s1) / (float)dim;
    const float m2 = wave_sum(s2) / (float)dim;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (!ok[c]) continue;
      u16x8_t o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float h = (bf16_to_f32(b[c][j]) - mu) * rs;
        const float g = bf16_to_f32(a[c][j]) * bf16_to_f32(gm[c][j]);
        o[j] = f32_to_bf16(rs * (g - m1 - h * m2) + bf16_to_f32(r[c][j]));
      }
      *reinterpret_cast<u16x8_t*>(dx + row * dim + 8 * (lane + 64 * c)) = o;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      a[c] = na[c];
      b[c] = nb[c];
      r[c] = nr[c];
    }
  }
  // combine the 4 waves' column partials, one chunk of columns at a time (wave order)
#pragma unroll
  for (int c = 0; c < C; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      red[0][wave][lane * 8 + j] = pg[c][j];
      red[1][wave][lane * 8 + j] = pb[c][j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 8; i += 256) {
      const int col = 8 * (i / 8 + 64 * c) + i % 8;
      if (col < dim) {
        part_g[(int64_t)blockIdx.x * dim + col] = red[0][0][i] + red[0][1][i] + red[0][2][i] + red[0][3][i];
        part_b[(int64_t)blockIdx.x * dim + col] = red[1][0][i] + red[1][1][i] + red[1][2][i] + red[1][3][i];
      }
    }
    __syncthreads();
  }
}

// bf16 rows of 1024 < dim <= 2048 (dim % 8 == 0): two waves share a row.  Wave p (= wave & 1)
// of a pair owns the 16-byte chunks 64*C*p + lane + 64c (c < C), so each lane holds half the
// row buffers and column partials of the one-wave kernel (registers for three to four waves per
// SIMD instead of one).  The pair's partial row sums meet in LDS and are added part 0 + part 1
// (fixed order); the LDS slot alternates with the iteration parity, so one barrier per row pair.
template <int C>
__global__ __launch_bounds__(256) void ln_bwd_bf16_pair_kernel(int64_t rows, int dim, const bf16_t* __restrict__ dy,
                                                                const bf16_t* __restrict__ x,
                                                                const float* __restrict__ mean,
                                                                const float* __restrict__ rstd,
                                                                const bf16_t* __restrict__ gamma,
                                                                const bf16_t* __restrict__ dres,
                                                                bf16_t* __restrict__ dx, float* __restrict__ part_g,
                                                                float* __restrict__ part_b) {
  __shared__ float rsum[2][4][2];               // [parity][wave][s1, s2]
  __shared__ float red[2][2][2][64 * 8];        // [g/b][part][row slot][column of the chunk]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave & 1, slot = wave >> 1;
  const int cbase = 64 * C * part;
  const u16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
  bool ok[C];
  u16x8_t gm[C];
  float pg[C][8], pb[C][8];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    ok[c] = 8 * (cbase + lane + 64 * c) < dim;
    gm[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(gamma + 8 * (cbase + lane + 64 * c)) : z;
#pragma unroll
    for (int j = 0; j < 8; ++j) pg[c][j] = pb[c][j] = 0.f;
  }
  const int64_t stride = (int64_t)gridDim.x * 2;
  auto load = [&](int64_t row, u16x8_t(&a)[C], u16x8_t(&b)[C], u16x8_t(&r)[C]) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t off = row * dim + 8 * (cbase + lane + 64 * c);
      a[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(dy + off) : z;
      b[c] = ok[c] ? *reinterpret_cast<const u16x8_t*>(x + off) : z;
      r[c] = (ok[c] && dres) ? *reinterpret_cast<const u16x8_t*>(dres + off) : z;
    }
  };
  u16x8_t a[C], b[C], r[C];
  {
    const int64_t row = (int64_t)blockIdx.x * 2 + slot;
    if (row < rows) load(row, a, b, r);
  }
  int parity = 0;
  // every wave of the block runs the same iterations (the barrier); rows past the end idle
  for (int64_t r0 = (int64_t)blockIdx.x * 2; r0 < rows; r0 += stride, parity ^= 1) {
    const int64_t row = r0 + slot;
    const bool valid = row < rows;
    u16x8_t na[C], nb[C], nr[C];
    if (row + stride < rows) load(row + stride, na, nb, nr);
    const float mu = valid ? mean[row] : 0.f, rs = valid ? rstd[row] : 0.f;
    float s1 = 0.f, s2 = 0.f;
    if (valid) {
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float dv = bf16_to_f32(a[c][j]);
          const float h = (bf16_to_f32(b[c][j]) - mu) * rs;
          const float g = dv * bf16_to_f32(gm[c][j]);
          s1 += g;
          s2 += g * h;
          pg[c][j] += dv * h;
          pb[c][j] += dv;
        }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if (lane == 0) {
      rsum[parity][wave][0] = s1;
      rsum[parity][wave][1] = s2;
    }
    __syncthreads();
    const float m1 = (rsum[parity][2 * slot][0] + rsum[parity][2 * slot + 1][0]) / (float)dim;
    const float m2 = (rsum[parity][2 * slot][1] + rsum[parity][2 * slot + 1][1]) / (float)dim;
    if (valid) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (!ok[c]) continue;
        u16x8_t o;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float h = (bf16_to_f32(b[c][j]) - mu) * rs;
          const float g = bf16_to_f32(a[c][j]) * bf16_to_f32(gm[c][j]);
          o[j] = f32_to_bf16(rs * (g - m1 - h * m2) + bf16_to_f32(r[c][j]));
        }
        *reinterpret_cast<u16x8_t*>(dx + row * dim + 8 * (cbase + lane + 64 * c)) = o;
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      a[c] = na[c];
      b[c] = nb[c];
      r[c] = nr[c];
    }
  }
  // column partials: the two row slots of each part are added slot 0 + slot 1
#pragma unroll
  for (int c = 0; c < C; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      red[0][part][slot][lane * 8 + j] = pg[c][j];
      red[1][part][slot][lane * 8 + j] = pb[c][j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * 64 * 8; i += 256) {
      const int pt = i / (64 * 8), k = i % (64 * 8);
      const int col = 8 * (64 * C * pt + k / 8 + 64 * c) + k % 8;
      if (col < dim) {
        part_g[(int64_t)blockIdx.x * dim + col] = red[0][pt][0][k] + red[0][pt][1][k];
        part_b[(int64_t)blockIdx.x * dim + col] = red[1][pt][0][k] + red[1][pt][1][k];
      }
    }
    __syncthreads();
  }
}

// Column sums of the per-block partial rows: a block owns 64 columns; its 16 waves sum
// partial rows w, w+16, ... for their lane's column, and the 16 wave sums are added in wave
// order (fixed order: deterministic).  16 waves x 32 blocks keep enough loads in flight.
template <typename T>
__global__ __launch_bounds__(1024) void ln_colsum_kernel(int nblocks, int dim, const float* __restrict__ part_g,
                                                          const float* __restrict__ part_b, T* dgamma, T* dbeta,
                                                          int accumulate) {
  __shared__ float red[2][16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float sg = 0.f, sb = 0.f;
  if (col < dim) {
#pragma unroll 8
    for (int b = wave; b < nblocks; b += 16) {
      sg += part_g[(int64_t)b * dim + col];
      sb += part_b[(int64_t)b * dim + col];
    }
  }
  red[0][wave][lane] = sg;
  red[1][wave][lane] = sb;
  __syncthreads();
  if (wave == 0 && col < dim) {
    sg = 0.f;
    sb = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      sg += red[0][w][lane];
      sb += red[1][w][lane];
    }
    if (dgamma) st_f32(dgamma + col, accumulate ? ld_f32(dgamma + col) + sg : sg);
    if (dbeta) st_f32(dbeta + col, accumulate ? ld_f32(dbeta + col) + sb : sb);
  }
}

int ln_blocks(int64_t rows) {
  int64_t nb = rh_cdiv(rows, 16);
  if (nb > 512) nb = 512;
  if (nb < 1) nb = 1;
  return (int)nb;
}

// Pick (V, E) for a dimension: vectorised when dim % 8 == 0 and aligned.
template <typename T, template <typename, int, int> class Launcher, typename... Args>
int dispatch_ln(int dim, bool vec, Args... args) {
  if (vec) {
    const int chunks = (dim + 511) / 512;  // 16-byte chunks per lane (8 elements each)
    if (chunks <= 1) return Launcher<T, 8, 8>::run(args...);
    if (chunks <= 2) return Launcher<T, 8, 16>::run(args...);
    if (chunks <= 4) return Launcher<T, 8, 32>::run(args...);
    if (chunks <= 8) return Launcher<T, 8, 64>::run(args...);
    return Launcher<T, 8, 128>::run(args...);
  }
  const int per = (dim + 63) / 64;
  if (per <= 1) return Launcher<T, 1, 1>::run(args...);
  if (per <= 2) return Launcher<T, 1, 2>::run(args...);
  if (per <= 4) return Launcher<T, 1, 4>::run(args...);
  if (per <= 8) return Launcher<T, 1, 8>::run(args...);
  if (per <= 16) return Launcher<T, 1, 16>::run(args...);
  if (per <= 32) return Launcher<T, 1, 32>::run(args...);
  if (per <= 64) return Launcher<T, 1, 64>::run(args...);
  return Launcher<T, 1, 128>::run(args...);
}

template <typename T, int V, int E>
struct FwdLauncher {
  static int run(int64_t rows, int dim, const void* x, const void* g, const void* b, float eps, void* y, float* mean,
                 float* rstd, hipStream_t st) {
    hipLaunchKernelGGL((ln_fwd_kernel<T, V, E>), dim3((unsigned)rh_cdiv(rows, 4)), dim3(256), 0, st, rows, dim,
                       (const T*)x, (const T*)g, (const T*)b, eps, (T*)y, mean, rstd);
    return rh_check_launch("rh_layernorm_fwd");
  }
};

template <typename T, int V, int E>
struct BwdLauncher {
  static int run(int64_t rows, int dim, const void* dy, const void* x, const float* mean, const float* rstd,
                 const void* gamma, const void* dres, void* dx, float* pg, float* pb, int nb, hipStream_t st) {
    hipLaunchKernelGGL((ln_bwd_kernel<T, V, E>), dim3((unsigned)nb), dim3(256), 0, st, rows, dim, (const T*)dy,
                       (const T*)x, mean, rstd, (const T*)gamma, (const T*)dres, (T*)dx, pg, pb);
    return rh_check_launch("rh_layernorm_bwd");
  }
};

int launch_bwd_bf16(int64_t rows, int dim, const void* dy, const void* x, const float* mean, const float* rstd,
                    const void* gamma, const void* dres, void* dx, float* pg, float* pb, int nb, hipStream_t st) {
  const int chunks = (dim + 511) / 512;
#define RH_LN_BWD(CC)                                                                                              \
  hipLaunchKernelGGL((ln_bwd_bf16_kernel<CC>), dim3((unsigned)nb), dim3(256), 0, st, rows, dim, (const bf16_t*)dy, \
                     (const bf16_t*)x, mean, rstd, (const bf16_t*)gamma, (const bf16_t*)dres, (bf16_t*)dx, pg, pb)
  if (chunks <= 1) RH_LN_BWD(1);
  else if (chunks <= 2) RH_LN_BWD(2);
  else  // dim <= 2048: two waves per row
    hipLaunchKernelGGL((ln_bwd_bf16_pair_kernel<2>), dim3((unsigned)nb), dim3(256), 0, st, rows, dim,
                       (const bf16_t*)dy, (const bf16_t*)x, mean, rstd, (const bf16_t*)gamma, (const bf16_t*)dres,
                       (bf16_t*)dx, pg, pb);
#undef RH_LN_BWD
  return rh_check_launch("rh_layernorm_bwd");
}

int check_ln(int dtype, int64_t rows, int64_t dim) {
  RH_REQUIRE(dtype == RH_DTYPE_F32 || dtype == RH_DTYPE_BF16, "rh_layernorm: unknown dtype %d", dtype);
  RH_REQUIRE(rows >= 0, "rh_layernorm: negative rows");
  RH_REQUIRE(dim >= 1 && dim <= 8192, "rh_layernorm: dim %lld outside [1, 8192]", (long long)dim);
  return RH_OK;
}

}  // namespace

extern "C" int rh_layernorm_fwd(int dtype, int64_t rows, int64_t dim, const void* x, const void* gamma,
                                const void* beta, float eps, void* y, float* mean, float* rstd, void* stream) {
  int rc = check_ln(dtype, rows, dim);
  if (rc) return rc;
  if (rows == 0) return RH_OK;
  RH_REQUIRE(x && gamma && beta && y && mean && rstd, "rh_layernorm_fwd: null pointer");
  const bool vec = dim % 8 == 0 && rh_aligned(x, 16) && rh_aligned(y, 16) && rh_aligned(gamma, 16) &&
                   rh_aligned(beta, 16);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RH_DTYPE_BF16 && vec && dim <= 2048) {
    // about four rows per wave
    const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(rh_cdiv(rows, 16), 1024));
#define RH_LN_FWD(CC)                                                                                              \
  hipLaunchKernelGGL((ln_fwd_bf16_kernel<CC>), dim3(blocks), dim3(256), 0, st, rows, (int)dim, (const bf16_t*)x, \
                     (const bf16_t*)gamma, (const bf16_t*)beta, eps, (bf16_t*)y, mean, rstd)
    if (dim <= 512) RH_LN_FWD(1);
    else if (dim <= 1024) RH_LN_FWD(2);
    else RH_LN_FWD(4);
#undef RH_LN_FWD
    return rh_check_launch("rh_layernorm_fwd");
  }
  if (dtype == RH_DTYPE_BF16)
    return dispatch_ln<bf16_t, FwdLauncher>((int)dim, vec, rows, (int)dim, x, gamma, beta, eps, y, mean, rstd, st);
  return dispatch_ln<float, FwdLauncher>((int)dim, vec, rows, (int)dim, x, gamma, beta, eps, y, mean, rstd, st);
}

extern "C" int rh_layernorm_bwd_workspace_bytes(int64_t rows, int64_t dim, int64_t* bytes) {
  RH_REQUIRE(bytes && rows >= 0 && dim >= 0, "rh_layernorm_bwd_workspace_bytes: bad arguments");
  *bytes = 2 * (int64_t)ln_blocks(rows) * dim * (int64_t)sizeof(float);
  return RH_OK;
}

extern "C" int rh_layernorm_bwd(int dtype, int64_t rows, int64_t dim, const void* dy, const void* x,
                                const float* mean, const float* rstd, const void* gamma, const void* dresidual,
                                void* dx, void* dgamma, void* dbeta, int accumulate, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  int rc = check_ln(dtype, rows, dim);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = ln_blocks(rows);
  if (rows == 0) {
    if (!accumulate && (dgamma || dbeta)) {
      // empty batch: the column sums are zero
      const int64_t eb = dtype == RH_DTYPE_BF16 ? 2 : 4;
      if (dgamma && hipMemsetAsync(dgamma, 0, dim * eb, st) != hipSuccess)
        return rh_set_error(RH_ERR_HIP, "rh_layernorm_bwd: memset failed");
      if (dbeta && hipMemsetAsync(dbeta, 0, dim * eb, st) != hipSuccess)
        return rh_set_error(RH_ERR_HIP, "rh_layernorm_bwd: memset failed");
    }
    return RH_OK;
  }
  RH_REQUIRE(dy && x && mean && rstd && gamma && dx, "rh_layernorm_bwd: null pointer");
  RH_REQUIRE(workspace && workspace_bytes >= 2 * (int64_t)nb * dim * (int64_t)sizeof(float),
             "rh_layernorm_bwd: workspace of %lld bytes is too small", (long long)workspace_bytes);
  float* pg = static_cast<float*>(workspace);
  float* pb = pg + (int64_t)nb * dim;
  const bool vec = dim % 8 == 0 && rh_aligned(dy, 16) && rh_aligned(x, 16) && rh_aligned(dx, 16) &&
                   rh_aligned(gamma, 16) && (dresidual == nullptr || rh_aligned(dresidual, 16));
  if (dtype == RH_DTYPE_BF16 && vec && dim <= 2048)
    rc = launch_bwd_bf16(rows, (int)dim, dy, x, mean, rstd, gamma, dresidual, dx, pg, pb, nb, st);
  else if (dtype == RH_DTYPE_BF16)
    rc = dispatch_ln<bf16_t, BwdLauncher>((int)dim, vec, rows, (int)dim, dy, x, mean, rstd, gamma, dresidual, dx, pg,
                                          pb, nb, st);
  else
    rc = dispatch_ln<float, BwdLauncher>((int)dim, vec, rows, (int)dim, dy, x, mean, rstd, gamma, dresidual, dx, pg,
                                         pb, nb, st);
  if (rc) return rc;
  if (dgamma || dbeta) {
    const unsigned blocks = (unsigned)rh_cdiv(dim, 64);
    if (dtype == RH_DTYPE_BF16)
      hipLaunchKernelGGL(ln_colsum_kernel<bf16_t>, dim3(blocks), dim3(1024), 0, st, nb, (int)dim, pg, pb,
                         (bf16_t*)dgamma, (bf16_t*)dbeta, accumulate);
    else
      hipLaunchKernelGGL(ln_colsum_kernel<float>, dim3(blocks), dim3(1024), 0, st, nb, (int)dim, pg, pb,
                         (float*)dgamma, (float*)dbeta, accumulate);
    return rh_check_launch("rh_layernorm_bwd colsum");
  }
  return RH_OK;
}
