// Dense GEMMs of the decoder block (F.linear and its backward) for gfx950.
//
// bf16 path: 128x128x64 workgroup tile, 4 waves in a 2x2 grid, each wave a
// 64x64 sub-tile built from v_mfma_f32_16x16x32_bf16 (fp32 accumulators).
// Both operands are staged through LDS in a k-contiguous layout
// ([rows][BK+8], the +8 pad keeps the 16-byte fragment reads of 16 lanes on
// distinct banks) and double-buffered: the global loads of tile k+1 are issued
// before the MFMAs of tile k and written to the other LDS buffer afterwards,
// so one barrier per k-tile suffices.  Operands whose memory layout is
// m/n-contiguous (dgrad's weight, both wgrad operands) are transposed while
// being written to LDS.
//
// fp32 path: 64x64x16 FMA tile (4x4 outputs per thread).  Used for the fp32
// parity mode, where no bf16 rounding may enter.
//
// Split-K: when the output has fewer tiles than the chip has CUs and K is
// long (the wgrad shapes), grid.z partitions K, every split writes fp32
// partials to the caller's workspace, and a reduce kernel sums them in split
// order (deterministic) and applies the epilogue.
#include <type_traits>

#include "common.hpp"

int rh_device_cus();

namespace {

template <typename T>
struct GemmParams {
  int64_t M, N, K;
  const T* A;
  int64_t lda;
  const T* B[RH_MAX_SEG];
  int64_t ldb;
  int64_t b_seg;
  int b_nseg;
  int d_nseg;
  float alpha, beta;
  const T* C;  // nullptr -> read C from D (in-place)
  int64_t ldc;
  T* D[RH_MAX_SEG];
  int64_t ldd;
  int64_t d_seg;
  const T* aux;
  T* aux_out;
  int64_t ldaux;
  float* ws;            // split-K partials [splits][M][N]
  int64_t k_per_split;  // multiple of the k-tile
  int aligned;          // all rows 16-byte aligned -> vector loads
};

template <typename T>
__device__ __forceinline__ const T* b_row(const GemmParams<T>& p, int64_t r) {
  if (p.b_nseg == 1) return p.B[0] + r * p.ldb;
  const int64_t s = r / p.b_seg;
  return p.B[s] + (r - s * p.b_seg) * p.ldb;
}
template <typename T>
__device__ __forceinline__ T* d_row(const GemmParams<T>& p, int64_t m) {
  if (p.d_nseg == 1) return p.D[0] + m * p.ldd;
  const int64_t s = m / p.d_seg;
  return p.D[s] + (m - s * p.d_seg) * p.ldd;
}

// v = alpha*acc + beta*C ; epilogue ; store.  Shared by every GEMM kernel.
template <typename T, int EPI>
__device__ __forceinline__ void epilogue_store(const GemmParams<T>& p, int64_t m, int64_t n, float acc) {
  T* drow = d_row(p, m);
  float v = p.alpha * acc;
  if (p.beta != 0.f) {
    const T* c = p.C ? (p.C + m * p.ldc + n) : (drow + n);
    v += p.beta * ld_f32(c);
  }
  if (EPI == RH_EPI_GELU) {
    st_f32(p.aux_out + m * p.ldaux + n, v);
    v = gelu_f(v);
  } else if (EPI == RH_EPI_GELU_GRAD) {
    v *= gelu_grad_f(ld_f32(p.aux + m * p.ldaux + n));
  }
  st_f32(drow + n, v);
}

// ---------------------------------------------------------------------------
// bf16 MFMA kernel
// ---------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64, kPad = 8, kLdsP = kBK + kPad;

// One operand tile of ROWS (m or n) x BK, loaded from global into registers
// and written to LDS as s[row][k].
//   KC = true : global row r is k-contiguous: element (r, k) = rowptr(r)[k]
//   KC = false: global row k is r-contiguous: element (r, k) = rowptr(k)[r]
template <int ROWS, bool KC>
struct TileIO {
  static constexpr int kChunks = ROWS * kBK / 8;
  static constexpr int kPer = kChunks / 256;
  u16x8_t reg[kPer];

  // `outer_lim` bounds the row index (M or N), `k_lim` bounds k.
  template <typename RowFn>
  __device__ __forceinline__ void load(RowFn rowptr, int64_t o0, int64_t k0, int64_t outer_lim, int64_t k_lim,
                                       bool aligned) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * 256;
      int64_t r, k;  // first element of the chunk
      if (KC) {
        r = o0 + c / (kBK / 8);
        k = k0 + (c % (kBK / 8)) * 8;
      } else {
        k = k0 + c / (ROWS / 8);
        r = o0 + (c % (ROWS / 8)) * 8;
      }
      u16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (KC) {
        if (r < outer_lim && k < k_lim) {
          const bf16_t* src = rowptr(r) + k;
          if (aligned && k + 8 <= k_lim) {
            v = *reinterpret_cast<const u16x8_t*>(src);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (k + j < k_lim) v[j] = src[j];
          }
        }
      } else {
        if (k < k_lim && r < outer_lim) {
          const bf16_t* src = rowptr(k) + r;
          if (aligned && r + 8 <= outer_lim) {
            v = *reinterpret_cast<const u16x8_t*>(src);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (r + j < outer_lim) v[j] = src[j];
          }
        }
      }
      reg[i] = v;
    }
  }

  __device__ __forceinline__ void store(bf16_t (*s)[kLdsP]) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * 256;
      if (KC) {
        const int r = c / (kBK / 8), k = (c % (kBK / 8)) * 8;
        *reinterpret_cast<u16x8_t*>(&s[r][k]) = reg[i];
      } else {
        const int k = c / (ROWS / 8), r = (c % (ROWS / 8)) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) s[r + j][k] = reg[i][j];
      }
    }
  }
};

template <int L, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_bf16_mfma(GemmParams<bf16_t> p) {
  constexpr bool A_KC = (L != RH_GEMM_TN);
  constexpr bool B_KC = (L == RH_GEMM_NT);
  constexpr int WTM = kBM / 2, WTN = kBN / 2, FM = WTM / 16, FN = WTN / 16;

  __shared__ __attribute__((aligned(16))) bf16_t sA[2][kBM][kLdsP];
  __shared__ __attribute__((aligned(16))) bf16_t sB[2][kBN][kLdsP];

  const int64_t tiles_n = (p.N + kBN - 1) / kBN;
  const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int64_t m0 = tm * kBM, n0 = tn * kBN;
  const int64_t kbeg = (int64_t)blockIdx.z * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nk = (int)((kend - kbeg + kBK - 1) / kBK);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const bool aligned = p.aligned != 0;

  auto a_row = [&](int64_t r) -> const bf16_t* { return p.A + r * p.lda; };
  auto bb_row = [&](int64_t r) -> const bf16_t* { return b_row(p, r); };

  TileIO<kBM, A_KC> ta;
  TileIO<kBN, B_KC> tb;

  floatx4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    ta.load(a_row, m0, kbeg, p.M, kend, aligned);
    tb.load(bb_row, n0, kbeg, p.N, kend, aligned);
    ta.store(sA[0]);
    tb.store(sB[0]);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = (kt + 1) < nk;
    if (more) {
      const int64_t k0 = kbeg + (int64_t)(kt + 1) * kBK;
      ta.load(a_row, m0, k0, p.M, kend, aligned);
      tb.load(bb_row, n0, k0, p.N, kend, aligned);
    }
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[cur][wm * WTM + i * 16 + (lane & 15)][ks * 32 + (lane >> 4) * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(&sB[cur][wn * WTN + j * 16 + (lane & 15)][ks * 32 + (lane >> 4) * 8]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      ta.store(sA[cur ^ 1]);
      tb.store(sB[cur ^ 1]);
    }
    __syncthreads();
  }

  // Output fragment (i, j), register r of lane l holds
  //   row = 16*i + 4*(l/16) + r, col = 16*j + l%16   of the wave's sub-tile.
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t n = n0 + wn * WTN + j * 16 + (lane & 15);
        if (n >= p.N) continue;
        if (SPLIT) {
          p.ws[(int64_t)blockIdx.z * p.M * p.N + m * p.N + n] = acc[i][j][r];
        } else {
          epilogue_store<bf16_t, EPI>(p, m, n, acc[i][j][r]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 FMA kernel
// ---------------------------------------------------------------------------
constexpr int fBM = 64, fBN = 64, fBK = 16;

template <int L, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_f32_fma(GemmParams<float> p) {
  constexpr bool A_KC = (L != RH_GEMM_TN);
  constexpr bool B_KC = (L == RH_GEMM_NT);
  __shared__ float sA[fBK][fBM + 4];
  __shared__ float sB[fBK][fBN + 4];

  const int64_t tiles_n = (p.N + fBN - 1) / fBN;
  const int64_t m0 = (blockIdx.x / tiles_n) * fBM, n0 = (blockIdx.x % tiles_n) * fBN;
  const int64_t kbeg = (int64_t)blockIdx.z * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int64_t k0 = kbeg; k0 < kend; k0 += fBK) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;
      int mm, kk;
      if (A_KC) { mm = idx / fBK; kk = idx % fBK; } else { kk = idx / fBM; mm = idx % fBM; }
      const int64_t m = m0 + mm, k = k0 + kk;
      float v = 0.f;
      if (m < p.M && k < kend) v = A_KC ? p.A[m * p.lda + k] : p.A[k * p.lda + m];
      sA[kk][mm] = v;
      int nn;
      if (B_KC) { nn = idx / fBK; kk = idx % fBK; } else { kk = idx / fBN; nn = idx % fBN; }
      const int64_t n = n0 + nn, k2 = k0 + kk;
      float w = 0.f;
      if (n < p.N && k2 < kend) w = B_KC ? b_row(p, n)[k2] : b_row(p, k2)[n];
      sB[kk][nn] = w;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < fBK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = sA[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = sB[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n >= p.N) continue;
      if (SPLIT) p.ws[(int64_t)blockIdx.z * p.M * p.N + m * p.N + n] = acc[i][j];
      else epilogue_store<float, EPI>(p, m, n, acc[i][j]);
    }
  }
}

// Sum split-K partials in split order and apply the epilogue.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmParams<T> p, int splits) {
  const int64_t total = p.M * p.N;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += p.ws[(int64_t)z * total + idx];
    epilogue_store<T, EPI>(p, idx / p.N, idx % p.N, s);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct Plan {
  int splits;
  int64_t k_per_split;
  int64_t ws_bytes;
};

Plan plan_gemm(const rh_gemm_desc* d) {
  Plan pl{1, d->K, 0};
  const bool bf16 = d->dtype == RH_DTYPE_BF16;
  const int64_t bm = bf16 ? kBM : fBM, bn = bf16 ? kBN : fBN, bk = bf16 ? kBK : fBK;
  const int64_t tiles = rh_cdiv(d->M, bm) * rh_cdiv(d->N, bn);
  const int64_t cus = rh_device_cus();
  if (!bf16 || d->K < 1024 || tiles >= cus) {
    pl.k_per_split = rh_cdiv(d->K, bk) * bk;
    return pl;
  }
  int64_t splits = rh_cdiv(2 * cus, tiles);
  if (splits > 8) splits = 8;
  int64_t kps = rh_cdiv(rh_cdiv(d->K, splits), bk) * bk;
  if (kps < 512) kps = 512;
  splits = rh_cdiv(d->K, kps);
  if (splits <= 1) {
    pl.k_per_split = rh_cdiv(d->K, bk) * bk;
    return pl;
  }
  pl.splits = (int)splits;
  pl.k_per_split = kps;
  pl.ws_bytes = splits * d->M * d->N * (int64_t)sizeof(float);
  return pl;
}

int validate(const rh_gemm_desc* d) {
  RH_REQUIRE(d != nullptr, "rh_gemm: null descriptor");
  RH_REQUIRE(d->dtype == RH_DTYPE_F32 || d->dtype == RH_DTYPE_BF16, "rh_gemm: unknown dtype %d", d->dtype);
  RH_REQUIRE(d->layout >= RH_GEMM_NT && d->layout <= RH_GEMM_TN, "rh_gemm: unknown layout %d", d->layout);
  RH_REQUIRE(d->epilogue >= RH_EPI_NONE && d->epilogue <= RH_EPI_GELU_GRAD, "rh_gemm: unknown epilogue %d",
             d->epilogue);
  RH_REQUIRE(d->M >= 0 && d->N >= 0 && d->K >= 0, "rh_gemm: negative extent M=%lld N=%lld K=%lld",
             (long long)d->M, (long long)d->N, (long long)d->K);
  RH_REQUIRE(d->b_nseg >= 1 && d->b_nseg <= RH_MAX_SEG && d->d_nseg >= 1 && d->d_nseg <= RH_MAX_SEG,
             "rh_gemm: segment count out of range (b %d, d %d)", d->b_nseg, d->d_nseg);
  if (d->M == 0 || d->N == 0) return RH_OK;
  RH_REQUIRE(d->A || d->K == 0, "rh_gemm: null A");
  RH_REQUIRE(d->D[0], "rh_gemm: null D");
  const int64_t a_rows = d->layout == RH_GEMM_TN ? d->K : d->M;
  const int64_t a_cols = d->layout == RH_GEMM_TN ? d->M : d->K;
  const int64_t b_rows = d->layout == RH_GEMM_NT ? d->N : d->K;
  const int64_t b_cols = d->layout == RH_GEMM_NT ? d->K : d->N;
  (void)a_rows;
  RH_REQUIRE(d->lda >= a_cols, "rh_gemm: lda %lld < %lld", (long long)d->lda, (long long)a_cols);
  RH_REQUIRE(d->ldb >= b_cols, "rh_gemm: ldb %lld < %lld", (long long)d->ldb, (long long)b_cols);
  RH_REQUIRE(d->ldd >= d->N, "rh_gemm: ldd %lld < N %lld", (long long)d->ldd, (long long)d->N);
  if (d->b_nseg > 1) {
    RH_REQUIRE(d->b_seg_rows > 0 && d->b_seg_rows * d->b_nseg >= b_rows,
               "rh_gemm: %d B segments of %lld rows do not cover %lld rows", d->b_nseg, (long long)d->b_seg_rows,
               (long long)b_rows);
    for (int s = 0; s < d->b_nseg; ++s) RH_REQUIRE(d->B[s], "rh_gemm: null B segment %d", s);
  } else {
    RH_REQUIRE(d->B[0] || d->K == 0, "rh_gemm: null B");
  }
  if (d->d_nseg > 1) {
    RH_REQUIRE(d->d_seg_rows > 0 && d->d_seg_rows * d->d_nseg >= d->M,
               "rh_gemm: %d D segments of %lld rows do not cover M=%lld", d->d_nseg, (long long)d->d_seg_rows,
               (long long)d->M);
    for (int s = 0; s < d->d_nseg; ++s) RH_REQUIRE(d->D[s], "rh_gemm: null D segment %d", s);
  }
  if (d->beta != 0.f && d->C) RH_REQUIRE(d->ldc >= d->N, "rh_gemm: ldc %lld < N", (long long)d->ldc);
  if (d->epilogue != RH_EPI_NONE) {
    RH_REQUIRE(d->ldaux >= d->N, "rh_gemm: ldaux %lld < N", (long long)d->ldaux);
    if (d->epilogue == RH_EPI_GELU) RH_REQUIRE(d->aux_out, "rh_gemm: GELU epilogue needs aux_out");
    if (d->epilogue == RH_EPI_GELU_GRAD) RH_REQUIRE(d->aux, "rh_gemm: GELU_GRAD epilogue needs aux");
  }
  return RH_OK;
}

template <typename T>
GemmParams<T> make_params(const rh_gemm_desc* d, const Plan& pl, void* ws) {
  GemmParams<T> p;
  p.M = d->M; p.N = d->N; p.K = d->K;
  p.A = static_cast<const T*>(d->A); p.lda = d->lda;
  for (int s = 0; s < RH_MAX_SEG; ++s) {
    p.B[s] = static_cast<const T*>(s < d->b_nseg ? d->B[s] : d->B[0]);
    p.D[s] = static_cast<T*>(s < d->d_nseg ? d->D[s] : d->D[0]);
  }
  p.ldb = d->ldb;
  p.b_seg = d->b_nseg > 1 ? d->b_seg_rows : INT64_MAX;
  p.b_nseg = d->b_nseg;
  p.d_nseg = d->d_nseg;
  p.alpha = d->alpha; p.beta = d->beta;
  p.C = static_cast<const T*>(d->C); p.ldc = d->ldc;
  p.ldd = d->ldd;
  p.d_seg = d->d_nseg > 1 ? d->d_seg_rows : INT64_MAX;
  p.aux = static_cast<const T*>(d->aux); p.aux_out = static_cast<T*>(d->aux_out); p.ldaux = d->ldaux;
  p.ws = static_cast<float*>(ws);
  p.k_per_split = pl.k_per_split;
  bool al = true;
  const int64_t vec = 16 / (int64_t)sizeof(T);
  al = al && rh_aligned(d->A, 16) && d->lda % vec == 0 && d->ldb % vec == 0;
  for (int s = 0; s < d->b_nseg; ++s) al = al && rh_aligned(d->B[s], 16);
  p.aligned = al ? 1 : 0;
  return p;
}

template <typename T, int L, int EPI, bool SPLIT>
void launch_main(const GemmParams<T>& p, dim3 grid, hipStream_t st) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    hipLaunchKernelGGL((gemm_bf16_mfma<L, EPI, SPLIT>), grid, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((gemm_f32_fma<L, EPI, SPLIT>), grid, dim3(256), 0, st, p);
  }
}

template <typename T, int L, int EPI>
int launch_layout(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st) {
  constexpr bool bf16 = std::is_same<T, bf16_t>::value;
  GemmParams<T> p = make_params<T>(d, pl, ws);
  const int64_t bm = bf16 ? kBM : fBM, bn = bf16 ? kBN : fBN;
  const int64_t tiles = rh_cdiv(d->M, bm) * rh_cdiv(d->N, bn);
  if (tiles > INT32_MAX) return rh_set_error(RH_ERR_INVALID, "rh_gemm: too many tiles (%lld)", (long long)tiles);
  dim3 grid((unsigned)tiles, 1, (unsigned)pl.splits);
  if (pl.splits > 1) {
    launch_main<T, L, EPI, true>(p, grid, st);
    int rc = rh_check_launch("rh_gemm");
    if (rc) return rc;
    const int64_t total = d->M * d->N;
    int64_t blocks = rh_cdiv(total, 256);
    if (blocks > 4 * 1024) blocks = 4 * 1024;
    hipLaunchKernelGGL((gemm_splitk_reduce<T, EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, pl.splits);
    return rh_check_launch("rh_gemm split-k reduce");
  }
  launch_main<T, L, EPI, false>(p, grid, st);
  return rh_check_launch("rh_gemm");
}

template <typename T, int EPI>
int launch_epi(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st) {
  switch (d->layout) {
    case RH_GEMM_NT: return launch_layout<T, RH_GEMM_NT, EPI>(d, pl, ws, st);
    case RH_GEMM_NN: return launch_layout<T, RH_GEMM_NN, EPI>(d, pl, ws, st);
    default: return launch_layout<T, RH_GEMM_TN, EPI>(d, pl, ws, st);
  }
}

template <typename T>
int launch_dtype(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st) {
  switch (d->epilogue) {
    case RH_EPI_NONE: return launch_epi<T, RH_EPI_NONE>(d, pl, ws, st);
    case RH_EPI_GELU: return launch_epi<T, RH_EPI_GELU>(d, pl, ws, st);
    default: return launch_epi<T, RH_EPI_GELU_GRAD>(d, pl, ws, st);
  }
}

// Epilogue-only pass for K == 0 (acc = 0).
template <typename T, int EPI>
int launch_k0(const rh_gemm_desc* d, hipStream_t st) {
  Plan pl{1, 0, 0};
  GemmParams<T> p = make_params<T>(d, pl, nullptr);
  // reuse the reduce kernel with zero splits: s = 0 for every element
  const int64_t total = d->M * d->N;
  int64_t blocks = rh_cdiv(total, 256);
  if (blocks > 4 * 1024) blocks = 4 * 1024;
  hipLaunchKernelGGL((gemm_splitk_reduce<T, EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, 0);
  return rh_check_launch("rh_gemm (K=0)");
}

}  // namespace

extern "C" int rh_gemm_workspace_bytes(const rh_gemm_desc* desc, int64_t* bytes) {
  int rc = validate(desc);
  if (rc) return rc;
  RH_REQUIRE(bytes != nullptr, "rh_gemm_workspace_bytes: null output");
  *bytes = (desc->M == 0 || desc->N == 0 || desc->K == 0) ? 0 : plan_gemm(desc).ws_bytes;
  return RH_OK;
}

extern "C" int rh_gemm(const rh_gemm_desc* desc, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = validate(desc);
  if (rc) return rc;
  if (desc->M == 0 || desc->N == 0) return RH_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf16 = desc->dtype == RH_DTYPE_BF16;
  if (desc->K == 0) {
    switch (desc->epilogue) {
      case RH_EPI_NONE: return bf16 ? launch_k0<bf16_t, RH_EPI_NONE>(desc, st) : launch_k0<float, RH_EPI_NONE>(desc, st);
      case RH_EPI_GELU: return bf16 ? launch_k0<bf16_t, RH_EPI_GELU>(desc, st) : launch_k0<float, RH_EPI_GELU>(desc, st);
      default: return bf16 ? launch_k0<bf16_t, RH_EPI_GELU_GRAD>(desc, st) : launch_k0<float, RH_EPI_GELU_GRAD>(desc, st);
    }
  }
  Plan pl = plan_gemm(desc);
  if (pl.splits > 1 && (workspace == nullptr || workspace_bytes < pl.ws_bytes || !rh_aligned(workspace, 16))) {
    pl.splits = 1;
    pl.k_per_split = rh_cdiv(desc->K, bf16 ? kBK : fBK) * (bf16 ? kBK : fBK);
    pl.ws_bytes = 0;
  }
  return bf16 ? launch_dtype<bf16_t>(desc, pl, workspace, st) : launch_dtype<float>(desc, pl, workspace, st);
}
