// Token (+ learned position) embedding, forward and a deterministic backward.
//
// Forward: one wavefront per token row, 16-byte loads when rows are aligned.
// Ids outside this rank's vocabulary slice give a zero row (vocab-parallel
// lookup).
//
// Backward: the (id, token position) pairs are sorted once in LDS by a
// single-block bitonic sort (keys id<<32 | position, so equal ids keep
// ascending position order), then one wavefront per distinct id sums the
// gradient rows of that id in position order and adds the sum to its
// embedding-gradient row.  No atomics: the result is bit-reproducible.
// The position gradient is a per-(position, column) sum over the batch.
#include "common.hpp"

namespace {

constexpr int kSortMax = 16384;  // tokens per call for the LDS sort (128 KiB of keys)

template <typename T>
__global__ __launch_bounds__(256) void emb_fwd_kernel(int64_t rows, int S, int dim, const int64_t* __restrict__ tok,
                                                       const T* __restrict__ W, int64_t vstart, int64_t vrows,
                                                       const T* __restrict__ P, T* __restrict__ out, int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t local = tok[row] - vstart;
  const bool inside = local >= 0 && local < vrows;
  const int s = (int)(row % S);
  const T* w = W + (inside ? local : 0) * dim;
  const T* p = P ? P + (int64_t)s * dim : nullptr;
  T* o = out + row * dim;
  if (vec && std::is_same<T, bf16_t>::value) {
    for (int c = lane * 8; c < dim; c += 64 * 8) {
      u16x8_t r = {0, 0, 0, 0, 0, 0, 0, 0};
      float v[8];
      if (inside) {
        const u16x8_t u = *reinterpret_cast<const u16x8_t*>(reinterpret_cast<const bf16_t*>(w) + c);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = bf16_to_f32(u[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.f;
      }
      if (p) {
        const u16x8_t u = *reinterpret_cast<const u16x8_t*>(reinterpret_cast<const bf16_t*>(p) + c);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] += bf16_to_f32(u[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = f32_to_bf16(v[j]);
      *reinterpret_cast<u16x8_t*>(reinterpret_cast<bf16_t*>(o) + c) = r;
    }
  } else {
    for (int c = lane; c < dim; c += 64) {
      float v = inside ? ld_f32(w + c) : 0.f;
      if (p) v += ld_f32(p + c);
      st_f32(o + c, v);
    }
  }
}

__global__ __launch_bounds__(1024) void emb_sort_kernel(int64_t n, const int64_t* __restrict__ tok, int64_t vstart,
                                                          int64_t vrows, int N, uint64_t* __restrict__ keys) {
  __shared__ uint64_t sk[kSortMax];
  for (int i = threadIdx.x; i < N; i += 1024) {
    uint64_t key = ~0ull;
    if (i < n) {
      const int64_t local = tok[i] - vstart;
      if (local >= 0 && local < vrows) key = ((uint64_t)local << 32) | (uint64_t)i;
    }
    sk[i] = key;
  }
  __syncthreads();
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < N; i += 1024) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = sk[i], b = sk[ixj];
          const bool up = (i & k) == 0;
          if (up ? (a > b) : (a < b)) {
            sk[i] = b;
            sk[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < n; i += 1024) keys[i] = sk[i];
}

template <typename T>
__global__ __launch_bounds__(256) void fill_zero_kernel(int64_t n, T* p) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) st_f32(p + i, 0.f);
}

template <typename T>
__global__ __launch_bounds__(256) void emb_seg_kernel(int64_t n, int dim, const uint64_t* __restrict__ keys,
                                                       const T* __restrict__ dout, T* __restrict__ dW) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const uint64_t k = keys[i];
  if (k == ~0ull) return;
  const uint64_t id = k >> 32;
  if (i > 0 && (keys[i - 1] >> 32) == id) return;  // not the first row of this id
  T* w = dW + (int64_t)id * dim;
  for (int c = lane; c < dim; c += 64) {
    float acc = 0.f;
    for (int64_t j = i; j < n; ++j) {
      const uint64_t kj = keys[j];
      if ((kj >> 32) != id) break;
      acc += ld_f32(dout + (int64_t)(kj & 0xffffffffu) * dim + c);
    }
    st_f32(w + c, ld_f32(w + c) + acc);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void emb_pos_kernel(int B, int S, int dim, const T* __restrict__ dout,
                                                       T* __restrict__ dP, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)S * dim) return;
  const int64_t s = idx / dim, c = idx % dim;
  float acc = 0.f;
  for (int b = 0; b < B; ++b) acc += ld_f32(dout + ((int64_t)b * S + s) * dim + c);
  st_f32(dP + idx, accumulate ? ld_f32(dP + idx) + acc : acc);
}

int check_emb(int dtype, int64_t B, int64_t S, int64_t dim) {
  RH_REQUIRE(dtype == RH_DTYPE_F32 || dtype == RH_DTYPE_BF16, "rh_embedding: unknown dtype %d", dtype);
  RH_REQUIRE(B >= 0 && S >= 0 && dim >= 1 && dim <= INT32_MAX, "rh_embedding: bad extents");
  return RH_OK;
}

}  // namespace

extern "C" int rh_embedding_fwd(int dtype, int64_t batch, int64_t seq, int64_t dim, const int64_t* tokens,
                                const void* tok, int64_t vocab_start, int64_t vocab_rows, const void* pos, void* out,
                                void* stream) {
  int rc = check_emb(dtype, batch, seq, dim);
  if (rc) return rc;
  const int64_t rows = batch * seq;
  if (rows == 0) return RH_OK;
  RH_REQUIRE(tokens && tok && out, "rh_embedding_fwd: null pointer");
  RH_REQUIRE(vocab_rows >= 1, "rh_embedding_fwd: empty vocabulary slice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vec = dim % 8 == 0 && rh_aligned(tok, 16) && rh_aligned(out, 16) && (!pos || rh_aligned(pos, 16));
  const unsigned grid = (unsigned)rh_cdiv(rows, 4);
  if (dtype == RH_DTYPE_BF16)
    hipLaunchKernelGGL(emb_fwd_kernel<bf16_t>, dim3(grid), dim3(256), 0, st, rows, (int)seq, (int)dim, tokens,
                       (const bf16_t*)tok, vocab_start, vocab_rows, (const bf16_t*)pos, (bf16_t*)out, vec);
  else
    hipLaunchKernelGGL(emb_fwd_kernel<float>, dim3(grid), dim3(256), 0, st, rows, (int)seq, (int)dim, tokens,
                       (const float*)tok, vocab_start, vocab_rows, (const float*)pos, (float*)out, 0);
  return rh_check_launch("rh_embedding_fwd");
}

extern "C" int rh_embedding_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t* bytes) {
  RH_REQUIRE(bytes && batch >= 0 && seq >= 0, "rh_embedding_bwd_workspace_bytes: bad arguments");
  *bytes = batch * seq * (int64_t)sizeof(uint64_t);
  return RH_OK;
}

extern "C" int rh_embedding_bwd(int dtype, int64_t batch, int64_t seq, int64_t dim, const int64_t* tokens,
                                const void* dout, int64_t vocab_start, int64_t vocab_rows, void* dtok, void* dpos,
                                int accumulate, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_emb(dtype, batch, seq, dim);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = batch * seq;
  const bool bf16 = dtype == RH_DTYPE_BF16;
  if (dtok) {
    RH_REQUIRE(vocab_rows >= 1 && vocab_rows < (1ll << 31), "rh_embedding_bwd: vocabulary slice of %lld rows",
               (long long)vocab_rows);
    if (!accumulate) {
      const int64_t n = vocab_rows * dim;
      unsigned g = (unsigned)std::min<int64_t>(rh_cdiv(n, 256), 65536);
      if (bf16) hipLaunchKernelGGL(fill_zero_kernel<bf16_t>, dim3(g), dim3(256), 0, st, n, (bf16_t*)dtok);
      else hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(g), dim3(256), 0, st, n, (float*)dtok);
    }
    if (rows > 0) {
      RH_REQUIRE(tokens && dout, "rh_embedding_bwd: null pointer");
      RH_REQUIRE(rows <= kSortMax, "rh_embedding_bwd: %lld tokens per call exceeds %d", (long long)rows, kSortMax);
      RH_REQUIRE(workspace && workspace_bytes >= rows * (int64_t)sizeof(uint64_t),
                 "rh_embedding_bwd: workspace of %lld bytes is too small", (long long)workspace_bytes);
      int N = 1;
      while (N < rows) N <<= 1;
      uint64_t* keys = static_cast<uint64_t*>(workspace);
      hipLaunchKernelGGL(emb_sort_kernel, dim3(1), dim3(1024), 0, st, rows, tokens, vocab_start, vocab_rows, N, keys);
      const unsigned g = (unsigned)rh_cdiv(rows, 4);
      if (bf16) hipLaunchKernelGGL(emb_seg_kernel<bf16_t>, dim3(g), dim3(256), 0, st, rows, (int)dim, keys,
                                   (const bf16_t*)dout, (bf16_t*)dtok);
      else hipLaunchKernelGGL(emb_seg_kernel<float>, dim3(g), dim3(256), 0, st, rows, (int)dim, keys,
                              (const float*)dout, (float*)dtok);
    }
    rc = rh_check_launch("rh_embedding_bwd (token)");
    if (rc) return rc;
  }
  if (dpos) {
    RH_REQUIRE(rows == 0 || dout, "rh_embedding_bwd: null dout");
    const int64_t n = seq * dim;
    if (n > 0) {
      const unsigned g = (unsigned)rh_cdiv(n, 256);
      if (bf16) hipLaunchKernelGGL(emb_pos_kernel<bf16_t>, dim3(g), dim3(256), 0, st, (int)batch, (int)seq, (int)dim,
                                   (const bf16_t*)dout, (bf16_t*)dpos, accumulate);
      else hipLaunchKernelGGL(emb_pos_kernel<float>, dim3(g), dim3(256), 0, st, (int)batch, (int)seq, (int)dim,
                              (const float*)dout, (float*)dpos, accumulate);
    }
    rc = rh_check_launch("rh_embedding_bwd (position)");
    if (rc) return rc;
  }
  return RH_OK;
}
