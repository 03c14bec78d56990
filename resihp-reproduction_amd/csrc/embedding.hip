// Token (+ learned position) embedding, forward and a deterministic backward.
//
// Forward: one wavefront per token row, 16-byte loads when rows are aligned.
// Ids outside this rank's vocabulary slice give a zero row (vocab-parallel
// lookup).
//
// Backward, for any token count: the (id, token position) pairs are sorted by a
// bitonic network over keys id<<32 | position (so equal ids keep ascending position
// order) -- compare distances below 8192 run inside one workgroup's LDS tile, larger
// ones as global passes -- and the gradient rows are then summed per id in two levels:
//   1. the sorted rows are cut into chunks of 32; each workgroup sums every id's rows
//      inside its chunk in position order.  An id whose rows all lie in the chunk is
//      added to its embedding-gradient row at once; the piece of an id that continues
//      into a neighbouring chunk goes to an fp32 slot of the workspace;
//   2. for every id spanning several chunks, one workgroup adds its pieces in chunk
//      order and adds the sum to the gradient row.
// A heavily repeated id therefore costs one chunk-parallel pass plus a walk over its
// chunk pieces rather than a serial pass over its rows.  No atomics: the summation
// order depends only on the sorted keys, so the result is bit-reproducible.
// The position gradient is a per-(position, column) sum over the batch.
#include "common.hpp"

namespace {

constexpr int kTile = 8192;   // keys per LDS tile of the bitonic sort (64 KiB)
constexpr int kChunk = 32;    // sorted rows per workgroup of the segmented sum
constexpr uint64_t kNoKey = ~0ull;

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

// keys[i] = local id << 32 | i for the n token positions (kNoKey for ids outside the slice and
// for the padding up to the power of two N)
__global__ __launch_bounds__(256) void emb_keys_kernel(int64_t n, int64_t N, const int64_t* __restrict__ tok,
                                                        int64_t vstart, int64_t vrows, uint64_t* __restrict__ keys) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < N; i += (int64_t)gridDim.x * 256) {
    uint64_t key = kNoKey;
    if (i < n) {
      const int64_t local = tok[i] - vstart;
      if (local >= 0 && local < vrows) key = ((uint64_t)local << 32) | (uint64_t)i;
    }
    keys[i] = key;
  }
}

// Bitonic stages k in [k_lo, k_hi] (powers of two), each with every compare distance
// j < min(k, tile), on one LDS tile of `tile` keys per workgroup.  Pair (i, i ^ j) is put in
// ascending order when bit k of the global index i is clear, descending otherwise.
__global__ __launch_bounds__(1024) void emb_bitonic_tile(uint64_t* __restrict__ keys, int tile, int64_t k_lo,
                                                          int64_t k_hi) {
  __shared__ uint64_t sk[kTile];
  const int64_t base = (int64_t)blockIdx.x * tile;
  for (int i = threadIdx.x; i < tile; i += 1024) sk[i] = keys[base + i];
  __syncthreads();
  for (int64_t k = k_lo; k <= k_hi; k <<= 1) {
    for (int j = (int)min<int64_t>(k, tile) >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < tile / 2; t += 1024) {
        const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));  // i has bit j clear (j a power of two); partner i + j
        const uint64_t a = sk[i], b = sk[i + j];
        const bool up = ((base + i) & k) == 0;
        if (up ? (a > b) : (a < b)) {
          sk[i] = b;
          sk[i + j] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < tile; i += 1024) keys[base + i] = sk[i];
}

// One bitonic compare distance j >= tile of stage k, over global memory.
__global__ __launch_bounds__(256) void emb_bitonic_global(uint64_t* __restrict__ keys, int64_t N, int64_t k, int64_t j) {
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < N / 2; t += (int64_t)gridDim.x * 256) {
    const int64_t i = ((t & ~(j - 1)) << 1) | (t & (j - 1));  // j a power of two
    const uint64_t a = keys[i], b = keys[i + j];
    const bool up = (i & k) == 0;
    if (up ? (a > b) : (a < b)) {
      keys[i] = b;
      keys[i + j] = a;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void fill_zero_kernel(int64_t n, T* p) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) st_f32(p + i, 0.f);
}

__device__ __forceinline__ uint64_t key_id(uint64_t k) { return k >> 32; }

// Level 1 of the per-id sum: workgroup (c, y) sums the sorted rows [32c, 32c + 32) per id over
// columns 64y .. 64y+63, one column per lane (all 32 row loads issued before the sums, then all
// gradient-row loads of the pieces that go straight into dW); one wave per workgroup and one
// workgroup per (chunk, 64 columns), so the chip has enough loads in flight.  Piece
// slots: head[c] holds the chunk's first piece when that id began in an earlier chunk; tail[c]
// its last piece when that id continues into the next chunk and began in this one.  Pieces
// closed on both sides go straight into dW.
template <typename T>
__global__ __launch_bounds__(64) void emb_chunk_sum(int64_t n, int dim, const uint64_t* __restrict__ keys,
                                                      const T* __restrict__ dout, T* __restrict__ dW,
                                                      float* __restrict__ head, float* __restrict__ tail) {
  __shared__ uint64_t sk[kChunk + 2];  // keys of rows lo-1 .. hi (kNoKey outside [0, n))
  const int64_t c = blockIdx.x;
  const int64_t lo = c * kChunk;
  const int m = (int)min<int64_t>(kChunk, n - lo);
  if (threadIdx.x < kChunk + 2) {
    const int64_t r = lo - 1 + threadIdx.x;
    sk[threadIdx.x] = (r >= 0 && r < n) ? keys[r] : kNoKey;
  }
  __syncthreads();
  if (sk[1] == kNoKey) return;
  // which rows end a piece and where its sum goes (the same for every column): bit i of `direct` /
  // `to_head` / `to_tail` marks the piece ending at row lo + i
  uint32_t direct = 0, to_head = 0, to_tail = 0;
  {
    bool first_piece = true;
    for (int i = 0; i < m; ++i) {
      const uint64_t k = sk[i + 1];
      if (k == kNoKey) break;
      const uint64_t next = sk[i + 2];  // row lo + i + 1 (the next chunk's first row when i = m - 1)
      const bool same_next = next != kNoKey && key_id(next) == key_id(k);
      if (same_next && i + 1 < m) continue;  // the id goes on inside this chunk
      const bool open_start = first_piece && sk[0] != kNoKey && key_id(sk[0]) == key_id(k);
      if (open_start) to_head |= 1u << i;
      else if (same_next) to_tail |= 1u << i;
      else direct |= 1u << i;
      first_piece = false;
    }
  }
  const uint32_t live = direct | to_head | to_tail;
  const int col = (int)blockIdx.y * 64 + (int)threadIdx.x;
  if (col < dim) {
    float val[kChunk], old[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const uint64_t k = sk[i + 1];
      val[i] = (i < m && k != kNoKey) ? ld_f32(dout + (int64_t)(k & 0xffffffffu) * dim + col) : 0.f;
    }
    // the gradient rows the direct pieces add to, all loads issued before any is used
#pragma unroll
    for (int i = 0; i < kChunk; ++i)
      old[i] = (direct >> i) & 1u ? ld_f32(dW + (int64_t)key_id(sk[i + 1]) * dim + col) : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      acc += val[i];
      if (!((live >> i) & 1u)) continue;
      if ((to_head >> i) & 1u) head[c * dim + col] = acc;
      else if ((to_tail >> i) & 1u) tail[c * dim + col] = acc;
      else st_f32(dW + (int64_t)key_id(sk[i + 1]) * dim + col, old[i] + acc);
      acc = 0.f;
    }
  }
}

// Level 2: an id that begins in chunk c and continues past it sums tail[c] and the head slots
// of the following chunks it covers, then adds the sum to its gradient row.  Its last row is
// found by a binary search of the sorted keys; workgroup (c, y) covers columns 64y .. 64y+63,
// wave w sums pieces w, w+4, ... in order and the four wave sums are added in wave order.
template <typename T>
__global__ __launch_bounds__(256) void emb_chunk_join(int64_t n, int dim, const uint64_t* __restrict__ keys,
                                                       T* __restrict__ dW, const float* __restrict__ head,
                                                       const float* __restrict__ tail) {
  __shared__ float part[4][64];
  const int64_t c = blockIdx.x;
  const int64_t lo = c * kChunk;
  const int64_t last = min(n, lo + kChunk) - 1;  // last row of chunk c
  if (last + 1 >= n) return;
  const uint64_t k = keys[last], nk = keys[last + 1];
  if (k == kNoKey || nk == kNoKey || key_id(nk) != key_id(k)) return;  // nothing continues
  const uint64_t id = key_id(k);
  // a chunk holding only this id, which also began before it, is a middle piece (head slot)
  if (key_id(keys[lo]) == id && lo > 0 && key_id(keys[lo - 1]) == id) return;
  int64_t a = last + 1, b = n;  // first row past this id: keys are sorted, kNoKey last
  while (a < b) {
    const int64_t mid = (a + b) / 2;
    const uint64_t km = keys[mid];
    if (km != kNoKey && key_id(km) == id) a = mid + 1;
    else b = mid;
  }
  const int64_t pieces = (a - 1) / kChunk - c + 1;  // tail[c], head[c + 1 .. (a - 1) / 32]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.y * 64 + lane;
  float acc = 0.f;
  if (col < dim) {
    for (int64_t q = wave; q < pieces; q += 4) acc += q == 0 ? tail[c * dim + col] : head[(c + q) * dim + col];
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && col < dim) {
    const float sum = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    T* w = dW + (int64_t)id * dim + col;
    st_f32(w, ld_f32(w) + sum);
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

// sort keys (next power of two >= tokens) + head and tail piece slots of every 32-row chunk
static int64_t emb_ws_layout(int64_t rows, int64_t dim, int64_t* N_out, int64_t* chunks_out) {
  int64_t N = 1;
  while (N < rows) N <<= 1;
  const int64_t chunks = rh_cdiv(rows, kChunk);
  if (N_out) *N_out = N;
  if (chunks_out) *chunks_out = chunks;
  return N * (int64_t)sizeof(uint64_t) + 2 * chunks * dim * (int64_t)sizeof(float);
}

extern "C" int rh_embedding_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t dim, int64_t* bytes) {
  RH_REQUIRE(bytes && batch >= 0 && seq >= 0 && dim >= 0, "rh_embedding_bwd_workspace_bytes: bad arguments");
  *bytes = batch * seq == 0 ? 0 : emb_ws_layout(batch * seq, dim, nullptr, nullptr);
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
      RH_REQUIRE(rows < (1ll << 31), "rh_embedding_bwd: %lld tokens per call exceeds 2^31 - 1", (long long)rows);
      int64_t N = 0, chunks = 0;
      const int64_t need = emb_ws_layout(rows, dim, &N, &chunks);
      RH_REQUIRE(workspace && workspace_bytes >= need && rh_aligned(workspace, 16),
                 "rh_embedding_bwd: workspace of %lld bytes is too small (%lld needed, 16-byte aligned)",
                 (long long)workspace_bytes, (long long)need);
      uint64_t* keys = static_cast<uint64_t*>(workspace);
      float* head = reinterpret_cast<float*>(keys + N);
      float* tail = head + chunks * dim;
      const unsigned gk = (unsigned)std::min<int64_t>(rh_cdiv(N, 256), 65536);
      hipLaunchKernelGGL(emb_keys_kernel, dim3(gk), dim3(256), 0, st, rows, N, tokens, vocab_start, vocab_rows, keys);
      // bitonic sort: stages up to the tile size inside LDS, then per larger stage the global
      // compare distances down to the tile size and one LDS launch for the rest
      const int tile = (int)std::min<int64_t>(N, kTile);
      const unsigned tiles = (unsigned)(N / tile);
      // stages up to 1024 on 1024-key tiles (many workgroups at once), the rest on whole tiles
      const int small = std::min(tile, 1024);
      hipLaunchKernelGGL(emb_bitonic_tile, dim3((unsigned)(N / small)), dim3(1024), 0, st, keys, small, (int64_t)2,
                         (int64_t)small);
      if (tile > small)
        hipLaunchKernelGGL(emb_bitonic_tile, dim3(tiles), dim3(1024), 0, st, keys, tile, (int64_t)(2 * small),
                           (int64_t)tile);
      const unsigned gg = (unsigned)std::min<int64_t>(rh_cdiv(N / 2, 256), 65536);
      for (int64_t k = 2 * (int64_t)tile; k <= N; k <<= 1) {
        for (int64_t j = k >> 1; j >= tile; j >>= 1)
          hipLaunchKernelGGL(emb_bitonic_global, dim3(gg), dim3(256), 0, st, keys, N, k, j);
        hipLaunchKernelGGL(emb_bitonic_tile, dim3(tiles), dim3(1024), 0, st, keys, tile, k, k);
      }
      const dim3 gj((unsigned)chunks, (unsigned)rh_cdiv(dim, 64));
      if (bf16) {
        hipLaunchKernelGGL(emb_chunk_sum<bf16_t>, gj, dim3(64), 0, st, rows, (int)dim, keys,
                           (const bf16_t*)dout, (bf16_t*)dtok, head, tail);
        hipLaunchKernelGGL(emb_chunk_join<bf16_t>, gj, dim3(256), 0, st, rows, (int)dim, keys, (bf16_t*)dtok,
                           head, tail);
      } else {
        hipLaunchKernelGGL(emb_chunk_sum<float>, gj, dim3(64), 0, st, rows, (int)dim, keys,
                           (const float*)dout, (float*)dtok, head, tail);
        hipLaunchKernelGGL(emb_chunk_join<float>, gj, dim3(256), 0, st, rows, (int)dim, keys, (float*)dtok, head,
                           tail);
      }
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
