// Fused causal self-attention (forward and backward) for gfx950.
//
// Math (per batch b, head h, query i, key j; scale = 1/sqrt(Dh)):
//   s_ij = scale * q_i.k_j,  masked to -inf for j > i when causal,
//   P = softmax_j(s),  o_i = sum_j P_ij v_j,  lse_i = log sum_j exp(s_ij)
// backward (delta_i = do_i.o_i):
//   dP_ij = do_i.v_j,  dS_ij = P_ij (dP_ij - delta_i)
//   dq_i = scale sum_j dS_ij k_j,  dk_j = scale sum_i dS_ij q_i,  dv_j = sum_i P_ij do_i
// P is rebuilt from lse in the backward; the [S,S] matrix never reaches HBM.
//
// bf16 / head_dim 64 or 128: MFMA kernels built on v_mfma_f32_32x32x16_bf16.
// Scores are computed transposed (S^T = K Q^T) so that every lane owns ONE
// query (its column) and 16 keys per 32-key block: the row max / row sum of
// the online softmax are lane-local plus one exchange with lane^32, and the
// probabilities feed the next MFMA (O^T += V^T P^T) straight from registers.
// 32x32 accumulator layout used throughout: register r of lane l holds
//   row 8*(r/4) + 4*(l/32) + r%4, column l%32;
// an operand fragment of lane l holds row/column l%32 and eight k values.
// The eight k values of lane group g = l/32 at step s of a 32-key block are the
// keys 16s + {4g..4g+3, 8+4g..8+4g+3}: exactly accumulator registers 8s..8s+7
// of the score tile, so P^T needs no data movement.  The matching V^T / Q^T /
// dO^T / K^T fragments are gathered from row-major LDS tiles.
//
// Everything else (fp32, other head sizes): one thread per query (forward, dq)
// or per key (dk/dv) with K/V or Q/dO tiles staged in LDS; fp32 FMA.
#include <initializer_list>

#include "common.hpp"

namespace {

constexpr float kLog2e = 1.4426950408889634074f;
constexpr float kLn2 = 0.69314718055994530942f;

template <typename T>
struct AttnArgs {
  const T* q;
  const T* k;
  const T* v;
  int64_t ld_qkv;
  const T* o;
  T* o_out;
  int64_t ld_o;
  const T* dout;
  int64_t ld_do;
  const float* lse;
  float* lse_out;
  const float* delta;
  float* delta_out;
  T* dq;
  T* dk;
  T* dv;
  int64_t ld_d;
  int B, S, H, D;
  float scale;
  int causal;
};

// ---------------------------------------------------------------------------
// delta_i = do_i . o_i   (fp32)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_delta(AttnArgs<T> a) {
  const int64_t total = (int64_t)a.B * a.S * a.H;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int h = (int)(idx % a.H);
  const int64_t t = idx / a.H;
  const T* o = a.o + t * a.ld_o + (int64_t)h * a.D;
  const T* d = a.dout + t * a.ld_do + (int64_t)h * a.D;
  float s = 0.f;
  for (int i = 0; i < a.D; ++i) s = fmaf(ld_f32(o + i), ld_f32(d + i), s);
  const int64_t b = t / a.S, sq = t % a.S;
  a.delta_out[(b * a.H + h) * a.S + sq] = s;
}

// bf16 rows with head_dim % 8 == 0 and 16-byte aligned rows: D/8 lanes per (token, head),
// one 16-byte load of o and of do per lane, shuffle reduction over the D/8 lanes.
template <int D>
__global__ __launch_bounds__(256) void attn_delta_vec(AttnArgs<bf16_t> a) {
  constexpr int L = D / 8;  // lanes per row (8 or 16)
  const int64_t total = (int64_t)a.B * a.S * a.H;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / L;
  const int part = threadIdx.x % L;
  float s = 0.f;
  int h = 0;
  int64_t t = 0;
  if (row < total) {
    h = (int)(row % a.H);
    t = row / a.H;
    const u16x8_t o = *reinterpret_cast<const u16x8_t*>(a.o + t * a.ld_o + (int64_t)h * D + part * 8);
    const u16x8_t d = *reinterpret_cast<const u16x8_t*>(a.dout + t * a.ld_do + (int64_t)h * D + part * 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) s = fmaf(bf16_to_f32(o[j]), bf16_to_f32(d[j]), s);
  }
#pragma unroll
  for (int off = L / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (row < total && part == 0) {
    const int64_t b = t / a.S, sq = t % a.S;
    a.delta_out[(b * a.H + h) * a.S + sq] = s;
  }
}

// ---------------------------------------------------------------------------
// generic kernels (any dtype, head_dim <= DMAX)
// ---------------------------------------------------------------------------
constexpr int gQ = 64, gKV = 32;

template <typename T, int DMAX>
__global__ __launch_bounds__(gQ) void attn_fwd_generic(AttnArgs<T> a) {
  __shared__ float sK[gKV][DMAX], sV[gKV][DMAX];
  const int S = a.S, D = a.D, H = a.H;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int qi = blockIdx.x * gQ + threadIdx.x;
  const float c = a.scale * kLog2e;
  float qv[DMAX], o[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    qv[d] = (qi < S && d < D) ? ld_f32(a.q + (tok0 + qi) * a.ld_qkv + (int64_t)h * D + d) * c : 0.f;
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int kv_end = a.causal ? min(S, (int)(blockIdx.x + 1) * gQ) : S;
  for (int kt = 0; kt < kv_end; kt += gKV) {
    __syncthreads();
    for (int e = threadIdx.x; e < gKV * DMAX; e += gQ) {
      const int r = e / DMAX, d = e % DMAX, key = kt + r;
      float kvv = 0.f, vvv = 0.f;
      if (key < S && d < D) {
        kvv = ld_f32(a.k + (tok0 + key) * a.ld_qkv + (int64_t)h * D + d);
        vvv = ld_f32(a.v + (tok0 + key) * a.ld_qkv + (int64_t)h * D + d);
      }
      sK[r][d] = kvv;
      sV[r][d] = vvv;
    }
    __syncthreads();
    for (int j = 0; j < gKV; ++j) {
      const int key = kt + j;
      if (key >= kv_end) break;
      if (a.causal && key > qi) break;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) s = fmaf(qv[d], sK[j][d], s);
      if (s > m) {
        const float corr = exp2f(m - s);
        l *= corr;
#pragma unroll
        for (int d = 0; d < DMAX; ++d) o[d] *= corr;
        m = s;
      }
      const float p = exp2f(s - m);
      l += p;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) o[d] = fmaf(p, sV[j][d], o[d]);
    }
  }
  if (qi >= S) return;
  const float inv = 1.f / l;
  T* op = a.o_out + (tok0 + qi) * a.ld_o + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DMAX; ++d)
    if (d < D) st_f32(op + d, o[d] * inv);
  a.lse_out[(int64_t)bh * S + qi] = (m + log2f(l)) * kLn2;
}

template <typename T, int DMAX>
__global__ __launch_bounds__(gQ) void attn_bwd_dq_generic(AttnArgs<T> a) {
  __shared__ float sK[gKV][DMAX], sV[gKV][DMAX];
  const int S = a.S, D = a.D, H = a.H;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int qi = blockIdx.x * gQ + threadIdx.x;
  const float c = a.scale * kLog2e;
  float qv[DMAX], dov[DMAX], dq[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    const bool ok = qi < S && d < D;
    qv[d] = ok ? ld_f32(a.q + (tok0 + qi) * a.ld_qkv + (int64_t)h * D + d) * c : 0.f;
    dov[d] = ok ? ld_f32(a.dout + (tok0 + qi) * a.ld_do + (int64_t)h * D + d) : 0.f;
    dq[d] = 0.f;
  }
  const float lse2 = qi < S ? a.lse[(int64_t)bh * S + qi] * kLog2e : 0.f;
  const float del = qi < S ? a.delta[(int64_t)bh * S + qi] : 0.f;
  const int kv_end = a.causal ? min(S, (int)(blockIdx.x + 1) * gQ) : S;
  for (int kt = 0; kt < kv_end; kt += gKV) {
    __syncthreads();
    for (int e = threadIdx.x; e < gKV * DMAX; e += gQ) {
      const int r = e / DMAX, d = e % DMAX, key = kt + r;
      float kvv = 0.f, vvv = 0.f;
      if (key < S && d < D) {
        kvv = ld_f32(a.k + (tok0 + key) * a.ld_qkv + (int64_t)h * D + d);
        vvv = ld_f32(a.v + (tok0 + key) * a.ld_qkv + (int64_t)h * D + d);
      }
      sK[r][d] = kvv;
      sV[r][d] = vvv;
    }
    __syncthreads();
    if (qi >= S) continue;
    for (int j = 0; j < gKV; ++j) {
      const int key = kt + j;
      if (key >= kv_end) break;
      if (a.causal && key > qi) break;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) {
        s = fmaf(qv[d], sK[j][d], s);
        dp = fmaf(dov[d], sV[j][d], dp);
      }
      const float p = exp2f(s - lse2);
      const float ds = p * (dp - del);
#pragma unroll
      for (int d = 0; d < DMAX; ++d) dq[d] = fmaf(ds, sK[j][d], dq[d]);
    }
  }
  if (qi >= S) return;
  T* dqp = a.dq + (tok0 + qi) * a.ld_d + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DMAX; ++d)
    if (d < D) st_f32(dqp + d, dq[d] * a.scale);
}

template <typename T, int DMAX>
__global__ __launch_bounds__(gQ) void attn_bwd_dkdv_generic(AttnArgs<T> a) {
  __shared__ float sQ[gKV][DMAX], sO[gKV][DMAX];
  __shared__ float sL[gKV], sDel[gKV];
  const int S = a.S, D = a.D, H = a.H;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int kj = blockIdx.x * gQ + threadIdx.x;
  const float c = a.scale * kLog2e;
  float kv[DMAX], vv[DMAX], dk[DMAX], dv[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    const bool ok = kj < S && d < D;
    kv[d] = ok ? ld_f32(a.k + (tok0 + kj) * a.ld_qkv + (int64_t)h * D + d) * c : 0.f;
    vv[d] = ok ? ld_f32(a.v + (tok0 + kj) * a.ld_qkv + (int64_t)h * D + d) : 0.f;
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  const int q_start = a.causal ? (int)blockIdx.x * gQ : 0;
  for (int qt = q_start; qt < S; qt += gKV) {
    __syncthreads();
    for (int e = threadIdx.x; e < gKV * DMAX; e += gQ) {
      const int r = e / DMAX, d = e % DMAX, q = qt + r;
      float qq = 0.f, oo = 0.f;
      if (q < S && d < D) {
        qq = ld_f32(a.q + (tok0 + q) * a.ld_qkv + (int64_t)h * D + d);
        oo = ld_f32(a.dout + (tok0 + q) * a.ld_do + (int64_t)h * D + d);
      }
      sQ[r][d] = qq;
      sO[r][d] = oo;
    }
    for (int r = threadIdx.x; r < gKV; r += gQ) {
      const int q = qt + r;
      sL[r] = q < S ? a.lse[(int64_t)bh * S + q] * kLog2e : 0.f;
      sDel[r] = q < S ? a.delta[(int64_t)bh * S + q] : 0.f;
    }
    __syncthreads();
    if (kj >= S) continue;
    for (int i = 0; i < gKV; ++i) {
      const int q = qt + i;
      if (q >= S) break;
      if (a.causal && kj > q) continue;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) {
        s = fmaf(kv[d], sQ[i][d], s);
        dp = fmaf(vv[d], sO[i][d], dp);
      }
      const float p = exp2f(s - sL[i]);
      const float ds = p * (dp - sDel[i]);
#pragma unroll
      for (int d = 0; d < DMAX; ++d) {
        dv[d] = fmaf(p, sO[i][d], dv[d]);
        dk[d] = fmaf(ds, sQ[i][d], dk[d]);
      }
    }
  }
  if (kj >= S) return;
  T* dkp = a.dk + (tok0 + kj) * a.ld_d + (int64_t)h * D;
  T* dvp = a.dv + (tok0 + kj) * a.ld_d + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    if (d < D) {
      st_f32(dkp + d, dk[d] * a.scale);
      st_f32(dvp + d, dv[d]);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA kernels (bf16, head_dim D in {64, 128})
// ---------------------------------------------------------------------------
__device__ __forceinline__ floatx16_t mfma32(bf16x8_t a, bf16x8_t b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16_t zero16() {
  floatx16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Eight consecutive accumulator registers (8s..8s+7) as a bf16 operand.
__device__ __forceinline__ bf16x8_t pack8(const floatx16_t& v, int s) {
  bf16x8_t r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (__bf16)v[8 * s + j];
  return r;
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// Transposed operand fragment from a row-major [token][P] LDS tile: rows of the MFMA operand are
// 32 consecutive columns starting at c0, its eight k values are the tokens
// r0 + {4g..4g+3, 8+4g..8+4g+3} (g = lane/32) -- the k order of accumulator registers
// 8s..8s+7.  Two ds_read_b64_tr_b16: in each 16-lane block lane i addresses token row
// (r0 + 4g + i/4 [+8]), columns c0 + 16*(block&1) + 4*(i%4) .. +3, and lane j receives
// the four rows of column c0 + 16*(block&1) + j.
template <int P>
__device__ __forceinline__ bf16x8_t tr_frag(const bf16_t* tile, int r0, int c0, int lane) {
  const int q = lane >> 4, i = lane & 15, g = q >> 1;
  const int col = c0 + 16 * (q & 1) + 4 * (i & 3);
  const int row = r0 + 4 * g + (i >> 2);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(tile + row * P + col));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(tile + (row + 8) * P + col));
  s16x4_t both[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8_t, both);
}

__device__ __forceinline__ bf16x8_t ld_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

// Store 4 consecutive head-dim values (registers 4rr..4rr+3) as bf16.
__device__ __forceinline__ void st4(bf16_t* p, const floatx16_t& v, int rr, float mul) {
  u16x4_t u;
#pragma unroll
  for (int t = 0; t < 4; ++t) u[t] = f32_to_bf16(v[4 * rr + t] * mul);
  *reinterpret_cast<u16x4_t*>(p) = u;
}

// ROWS x D bf16 rows staged global -> registers -> LDS (zero past `limit`), 256 threads.
// `store` writes the row-major tile with pitch P1 and, when P2 > 0, a second copy with
// pitch P2 (the copy read with transpose reads).
template <int D, int ROWS>
struct RowTile {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int PER = ROWS * CPR / 256;      // chunks per thread
  static_assert((ROWS * CPR) % 256 == 0, "tile must split evenly over 256 threads");
  u16x8_t reg[PER];

  __device__ __forceinline__ void load(const bf16_t* base, int64_t ld, int r0, int limit) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + i * 256, r = c / CPR, col = (c % CPR) * 8;
      u16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (r0 + r < limit) v = *reinterpret_cast<const u16x8_t*>(base + (int64_t)(r0 + r) * ld + col);
      reg[i] = v;
    }
  }
  template <int P1, int P2>
  __device__ __forceinline__ void store(bf16_t* s1, bf16_t* s2) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + i * 256, r = c / CPR, col = (c % CPR) * 8;
      *reinterpret_cast<u16x8_t*>(s1 + r * P1 + col) = reg[i];
      if (P2 > 0) *reinterpret_cast<u16x8_t*>(s2 + r * P2 + col) = reg[i];
    }
  }
};

// LDS pitches (elements): row reads with ds_read_b128 want 16 consecutive rows on distinct
// 16-byte bank groups (pitch = D + 8); transpose reads touch 4 rows x 32 bytes per 16 lanes
// and want rows 64 bytes apart modulo the 256-byte bank window (pitch = D + 32).
template <int D> struct Pitch {
  static constexpr int ROW = D + 8;
  static constexpr int TR = D + 32;
};

template <int D>
__global__ __launch_bounds__(256) void attn_fwd_mfma(AttnArgs<bf16_t> a) {
  constexpr int BQ = 128, BKV = 64, KP = Pitch<D>::ROW, VP = Pitch<D>::TR, KS = D / 16, DB = D / 32;
  constexpr int STAGE = BKV * KP + BKV * VP;
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int S = a.S, H = a.H;
  const int nqb = (S + BQ - 1) / BQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // longest causal rows first
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int wq0 = qb * BQ + w * 32, wq1 = wq0 + 31;
  const int q_row = wq0 + l32;
  const float c = a.scale * kLog2e;

  bf16x8_t qreg[KS];
  {
    const bf16_t* qp = a.q + (tok0 + q_row) * a.ld_qkv + (int64_t)h * D;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      u16x8_t u = {0, 0, 0, 0, 0, 0, 0, 0};
      if (q_row < S) u = *reinterpret_cast<const u16x8_t*>(qp + 16 * i + 8 * g);
      qreg[i] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  floatx16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = zero16();
  float m = -INFINITY, lsum = 0.f;

  const bf16_t* kbase = a.k + tok0 * a.ld_qkv + (int64_t)h * D;
  const bf16_t* vbase = a.v + tok0 * a.ld_qkv + (int64_t)h * D;
  const int kv_end = a.causal ? min(S, qb * BQ + BQ) : S;
  const int ntiles = (kv_end + BKV - 1) / BKV;
  RowTile<D, BKV> tk, tv;
  tk.load(kbase, a.ld_qkv, 0, S);
  tv.load(vbase, a.ld_qkv, 0, S);
  tk.template store<KP, 0>(smem, nullptr);
  tv.template store<VP, 0>(smem + BKV * KP, nullptr);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * BKV;
    const bool more = t + 1 < ntiles;
    if (more) {
      tk.load(kbase, a.ld_qkv, kt + BKV, S);
      tv.load(vbase, a.ld_qkv, kt + BKV, S);
    }
    const bf16_t* sK = smem + (t & 1) * STAGE;
    const bf16_t* sV = sK + BKV * KP;
    if (wq0 < S && !(a.causal && kt > wq1)) {
      floatx16_t st[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        st[kb] = zero16();
#pragma unroll
        for (int i = 0; i < KS; ++i) st[kb] = mfma32(ld_frag(sK + (kb * 32 + l32) * KP + 16 * i + 8 * g), qreg[i], st[kb]);
      }
      float mx = -INFINITY;
      const bool diag = a.causal && kt + BKV - 1 > wq0;  // some key in this tile is after some query
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          float sv = st[kb][r] * c;
          if (key >= S || (diag && key > q_row)) sv = -INFINITY;
          st[kb][r] = sv;
          mx = fmaxf(mx, sv);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m, mx);
      const float corr = exp2f(m - mnew);
      lsum *= corr;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[d][r] *= corr;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f(st[kb][r] - mnew);
          st[kb][r] = p;
          lsum += p;
        }
      m = mnew;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t pb = pack8(st[kb], s2);
#pragma unroll
          for (int d = 0; d < DB; ++d) oacc[d] = mfma32(tr_frag<VP>(sV, kb * 32 + 16 * s2, d * 32, lane), pb, oacc[d]);
        }
    }
    if (more) {
      bf16_t* nK = smem + ((t + 1) & 1) * STAGE;
      tk.template store<KP, 0>(nK, nullptr);
      tv.template store<VP, 0>(nK + BKV * KP, nullptr);
    }
    __syncthreads();
  }
  lsum += __shfl_xor(lsum, 32, 64);
  if (q_row >= S) return;
  const float inv = 1.f / lsum;
  bf16_t* op = a.o_out + (tok0 + q_row) * a.ld_o + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) st4(op + d * 32 + 8 * rr + 4 * g, oacc[d], rr, inv);
  if (g == 0) a.lse_out[(int64_t)bh * S + q_row] = (m + log2f(lsum)) * kLn2;
}

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_mfma(AttnArgs<bf16_t> a) {
  constexpr int BQ = 128, BKV = 64, KP = Pitch<D>::ROW, TP = Pitch<D>::TR, KS = D / 16, DB = D / 32;
  constexpr int STAGE = BKV * KP + BKV * TP + BKV * KP;  // K (row reads), K (transpose reads), V
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int S = a.S, H = a.H;
  const int nqb = (S + BQ - 1) / BQ;
  const int qb = nqb - 1 - (int)blockIdx.x;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int wq0 = qb * BQ + w * 32, wq1 = wq0 + 31;
  const int q_row = wq0 + l32;
  const float c = a.scale * kLog2e;

  bf16x8_t qreg[KS], doreg[KS];
  {
    const bf16_t* qp = a.q + (tok0 + q_row) * a.ld_qkv + (int64_t)h * D;
    const bf16_t* dp = a.dout + (tok0 + q_row) * a.ld_do + (int64_t)h * D;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      u16x8_t u = {0, 0, 0, 0, 0, 0, 0, 0}, v = u;
      if (q_row < S) {
        u = *reinterpret_cast<const u16x8_t*>(qp + 16 * i + 8 * g);
        v = *reinterpret_cast<const u16x8_t*>(dp + 16 * i + 8 * g);
      }
      qreg[i] = __builtin_bit_cast(bf16x8_t, u);
      doreg[i] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  const float lse2 = q_row < S ? a.lse[(int64_t)bh * S + q_row] * kLog2e : 0.f;
  const float del = q_row < S ? a.delta[(int64_t)bh * S + q_row] : 0.f;
  floatx16_t dqt[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) dqt[d] = zero16();

  const bf16_t* kbase = a.k + tok0 * a.ld_qkv + (int64_t)h * D;
  const bf16_t* vbase = a.v + tok0 * a.ld_qkv + (int64_t)h * D;
  const int kv_end = a.causal ? min(S, qb * BQ + BQ) : S;
  const int ntiles = (kv_end + BKV - 1) / BKV;
  RowTile<D, BKV> tk, tv;
  tk.load(kbase, a.ld_qkv, 0, S);
  tv.load(vbase, a.ld_qkv, 0, S);
  tk.template store<KP, TP>(smem, smem + BKV * KP);
  tv.template store<KP, 0>(smem + BKV * KP + BKV * TP, nullptr);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * BKV;
    const bool more = t + 1 < ntiles;
    if (more) {
      tk.load(kbase, a.ld_qkv, kt + BKV, S);
      tv.load(vbase, a.ld_qkv, kt + BKV, S);
    }
    const bf16_t* sK = smem + (t & 1) * STAGE;
    const bf16_t* sKt = sK + BKV * KP;
    const bf16_t* sV = sKt + BKV * TP;
    if (wq0 < S && !(a.causal && kt > wq1)) {
      const bool diag = a.causal && kt + BKV - 1 > wq0;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        floatx16_t st = zero16(), dpt = zero16();
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          st = mfma32(ld_frag(sK + (kb * 32 + l32) * KP + 16 * i + 8 * g), qreg[i], st);
          dpt = mfma32(ld_frag(sV + (kb * 32 + l32) * KP + 16 * i + 8 * g), doreg[i], dpt);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = key < S && q_row < S && !(diag && key > q_row);
          const float p = ok ? exp2f(st[r] * c - lse2) : 0.f;
          st[r] = p * (dpt[r] - del);
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t dsb = pack8(st, s2);
#pragma unroll
          for (int d = 0; d < DB; ++d) dqt[d] = mfma32(tr_frag<TP>(sKt, kb * 32 + 16 * s2, d * 32, lane), dsb, dqt[d]);
        }
      }
    }
    if (more) {
      bf16_t* nK = smem + ((t + 1) & 1) * STAGE;
      tk.template store<KP, TP>(nK, nK + BKV * KP);
      tv.template store<KP, 0>(nK + BKV * KP + BKV * TP, nullptr);
    }
    __syncthreads();
  }
  if (q_row >= S) return;
  bf16_t* dqp = a.dq + (tok0 + q_row) * a.ld_d + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) st4(dqp + d * 32 + 8 * rr + 4 * g, dqt[d], rr, a.scale);
}

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_mfma(AttnArgs<bf16_t> a) {
  constexpr int BK = 128, BQT = 32, RP = Pitch<D>::ROW, TP = Pitch<D>::TR, KS = D / 16, DB = D / 32;
  constexpr int STAGE = 2 * BQT * RP + 2 * BQT * TP;  // Q, dO (row reads); Q, dO (transpose reads)
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * STAGE];
  __shared__ float sL[2][BQT], sDel[2][BQT];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int S = a.S, H = a.H;
  const int kblk = blockIdx.x;  // block 0 has the most causal work; launched first
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t tok0 = (int64_t)b * S;
  const int wk0 = kblk * BK + w * 32;
  const int key = wk0 + l32;
  const float c = a.scale * kLog2e;

  bf16x8_t kreg[KS], vreg[KS];
  {
    const bf16_t* kp = a.k + (tok0 + key) * a.ld_qkv + (int64_t)h * D;
    const bf16_t* vp = a.v + (tok0 + key) * a.ld_qkv + (int64_t)h * D;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      u16x8_t u = {0, 0, 0, 0, 0, 0, 0, 0}, v = u;
      if (key < S) {
        u = *reinterpret_cast<const u16x8_t*>(kp + 16 * i + 8 * g);
        v = *reinterpret_cast<const u16x8_t*>(vp + 16 * i + 8 * g);
      }
      kreg[i] = __builtin_bit_cast(bf16x8_t, u);
      vreg[i] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  floatx16_t dvt[DB], dkt[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    dvt[d] = zero16();
    dkt[d] = zero16();
  }
  const bf16_t* qbase = a.q + tok0 * a.ld_qkv + (int64_t)h * D;
  const bf16_t* dbase = a.dout + tok0 * a.ld_do + (int64_t)h * D;
  const int q_start = a.causal ? kblk * BK : 0;
  const int ntiles = q_start < S ? (S - q_start + BQT - 1) / BQT : 0;
  RowTile<D, BQT> tq, td;
  float l_pref = 0.f, d_pref = 0.f;
  auto load_tile = [&](int qt) {
    tq.load(qbase, a.ld_qkv, qt, S);
    td.load(dbase, a.ld_do, qt, S);
    if (tid < BQT) {
      const int q = qt + tid;
      l_pref = q < S ? a.lse[(int64_t)bh * S + q] * kLog2e : 0.f;
      d_pref = q < S ? a.delta[(int64_t)bh * S + q] : 0.f;
    }
  };
  auto store_tile = [&](int stage) {
    bf16_t* base = smem + stage * STAGE;
    tq.template store<RP, TP>(base, base + 2 * BQT * RP);
    td.template store<RP, TP>(base + BQT * RP, base + 2 * BQT * RP + BQT * TP);
    if (tid < BQT) {
      sL[stage][tid] = l_pref;
      sDel[stage][tid] = d_pref;
    }
  };
  if (ntiles > 0) {
    load_tile(q_start);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int qt = q_start + t * BQT;
    const bool more = t + 1 < ntiles;
    if (more) load_tile(qt + BQT);
    const int cur = t & 1;
    const bf16_t* sQ = smem + cur * STAGE;
    const bf16_t* sdO = sQ + BQT * RP;
    const bf16_t* sQt = sQ + 2 * BQT * RP;
    const bf16_t* sdOt = sQt + BQT * TP;
    if (wk0 < S && !(a.causal && qt + BQT - 1 < wk0)) {
      floatx16_t sc = zero16(), dp = zero16();
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        sc = mfma32(ld_frag(sQ + l32 * RP + 16 * i + 8 * g), kreg[i], sc);
        dp = mfma32(ld_frag(sdO + l32 * RP + 16 * i + 8 * g), vreg[i], dp);
      }
      const bool diag = a.causal && qt < wk0 + 31;  // some query in this tile precedes some key
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = 8 * (r >> 2) + 4 * g + (r & 3);
        const int q = qt + qi;
        const bool ok = q < S && key < S && !(diag && key > q);
        const float p = ok ? exp2f(sc[r] * c - sL[cur][qi]) : 0.f;
        dp[r] = p * (dp[r] - sDel[cur][qi]);
        sc[r] = p;
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const bf16x8_t pb = pack8(sc, s2), dsb = pack8(dp, s2);
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          dvt[d] = mfma32(tr_frag<TP>(sdOt, 16 * s2, d * 32, lane), pb, dvt[d]);
          dkt[d] = mfma32(tr_frag<TP>(sQt, 16 * s2, d * 32, lane), dsb, dkt[d]);
        }
      }
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }
  if (key >= S) return;
  bf16_t* dkp = a.dk + (tok0 + key) * a.ld_d + (int64_t)h * D;
  bf16_t* dvp = a.dv + (tok0 + key) * a.ld_d + (int64_t)h * D;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      st4(dkp + d * 32 + 8 * rr + 4 * g, dkt[d], rr, a.scale);
      st4(dvp + d * 32 + 8 * rr + 4 * g, dvt[d], rr, 1.f);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int check_common(int dtype, int64_t B, int64_t S, int64_t H, int64_t D) {
  RH_REQUIRE(dtype == RH_DTYPE_F32 || dtype == RH_DTYPE_BF16, "rh_attn: unknown dtype %d", dtype);
  RH_REQUIRE(B >= 0 && S >= 0 && H >= 0, "rh_attn: negative extent");
  RH_REQUIRE(D >= 1 && D <= 128, "rh_attn: head_dim %lld outside [1, 128]", (long long)D);
  RH_REQUIRE(S <= (1 << 24) && B * H <= 65535, "rh_attn: batch*heads %lld or seq %lld too large",
             (long long)(B * H), (long long)S);
  return RH_OK;
}

bool mfma_ok(int dtype, int64_t D, std::initializer_list<const void*> ptrs, std::initializer_list<int64_t> lds) {
  if (dtype != RH_DTYPE_BF16 || (D != 64 && D != 128)) return false;
  for (const void* p : ptrs)
    if (!rh_aligned(p, 16)) return false;
  for (int64_t ld : lds)
    if (ld % 8) return false;
  return true;
}

template <typename T>
AttnArgs<T> make_args(int64_t B, int64_t S, int64_t H, int64_t D, float scale, int causal) {
  AttnArgs<T> a{};
  a.B = (int)B; a.S = (int)S; a.H = (int)H; a.D = (int)D;
  a.scale = scale;
  a.causal = causal ? 1 : 0;
  return a;
}

template <typename T, int DMAX>
void launch_generic_fwd(const AttnArgs<T>& a, hipStream_t st) {
  dim3 grid((unsigned)((a.S + gQ - 1) / gQ), (unsigned)(a.B * a.H));
  hipLaunchKernelGGL((attn_fwd_generic<T, DMAX>), grid, dim3(gQ), 0, st, a);
}
template <typename T, int DMAX>
void launch_generic_bwd(const AttnArgs<T>& a, hipStream_t st) {
  dim3 grid((unsigned)((a.S + gQ - 1) / gQ), (unsigned)(a.B * a.H));
  hipLaunchKernelGGL((attn_bwd_dq_generic<T, DMAX>), grid, dim3(gQ), 0, st, a);
  hipLaunchKernelGGL((attn_bwd_dkdv_generic<T, DMAX>), grid, dim3(gQ), 0, st, a);
}

template <typename T>
void dispatch_generic(const AttnArgs<T>& a, hipStream_t st, bool fwd) {
  if (a.D <= 16) fwd ? launch_generic_fwd<T, 16>(a, st) : launch_generic_bwd<T, 16>(a, st);
  else if (a.D <= 32) fwd ? launch_generic_fwd<T, 32>(a, st) : launch_generic_bwd<T, 32>(a, st);
  else if (a.D <= 64) fwd ? launch_generic_fwd<T, 64>(a, st) : launch_generic_bwd<T, 64>(a, st);
  else fwd ? launch_generic_fwd<T, 128>(a, st) : launch_generic_bwd<T, 128>(a, st);
}

}  // namespace

extern "C" int rh_attn_fwd(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, const void* q,
                           const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
                           float scale, int causal, void* stream) {
  int rc = check_common(dtype, batch, seq, heads, head_dim);
  if (rc) return rc;
  if (batch == 0 || seq == 0 || heads == 0) return RH_OK;
  RH_REQUIRE(q && k && v && o && lse, "rh_attn_fwd: null pointer");
  RH_REQUIRE(ld_qkv >= heads * head_dim && ld_o >= heads * head_dim, "rh_attn_fwd: leading dimension too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mfma_ok(dtype, head_dim, {q, k, v, o}, {ld_qkv, ld_o})) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o_out = (bf16_t*)o; a.ld_o = ld_o; a.lse_out = lse;
    dim3 grid((unsigned)((seq + 127) / 128), (unsigned)(batch * heads));
    if (head_dim == 64) hipLaunchKernelGGL(attn_fwd_mfma<64>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(attn_fwd_mfma<128>, grid, dim3(256), 0, st, a);
    return rh_check_launch("rh_attn_fwd");
  }
  if (dtype == RH_DTYPE_BF16) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o_out = (bf16_t*)o; a.ld_o = ld_o; a.lse_out = lse;
    dispatch_generic(a, st, true);
  } else {
    AttnArgs<float> a = make_args<float>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const float*)q; a.k = (const float*)k; a.v = (const float*)v; a.ld_qkv = ld_qkv;
    a.o_out = (float*)o; a.ld_o = ld_o; a.lse_out = lse;
    dispatch_generic(a, st, true);
  }
  return rh_check_launch("rh_attn_fwd");
}

extern "C" int rh_attn_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t heads, int64_t* bytes) {
  RH_REQUIRE(bytes && batch >= 0 && seq >= 0 && heads >= 0, "rh_attn_bwd_workspace_bytes: bad arguments");
  *bytes = batch * seq * heads * (int64_t)sizeof(float);
  return RH_OK;
}

extern "C" int rh_attn_bwd(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, const void* q,
                           const void* k, const void* v, int64_t ld_qkv, const void* o, int64_t ld_o,
                           const void* dout, int64_t ld_do, const float* lse, void* dq, void* dk, void* dv,
                           int64_t ld_dqkv, float scale, int causal, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  int rc = check_common(dtype, batch, seq, heads, head_dim);
  if (rc) return rc;
  if (batch == 0 || seq == 0 || heads == 0) return RH_OK;
  RH_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, "rh_attn_bwd: null pointer");
  const int64_t width = heads * head_dim;
  RH_REQUIRE(ld_qkv >= width && ld_o >= width && ld_do >= width && ld_dqkv >= width,
             "rh_attn_bwd: leading dimension too small");
  RH_REQUIRE(workspace && workspace_bytes >= batch * seq * heads * (int64_t)sizeof(float),
             "rh_attn_bwd: workspace of %lld bytes is too small", (long long)workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* delta = static_cast<float*>(workspace);
  const int64_t rows = batch * seq * heads;
  const unsigned dblocks = (unsigned)((rows + 255) / 256);
  if (dtype == RH_DTYPE_BF16) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o = (const bf16_t*)o; a.ld_o = ld_o; a.dout = (const bf16_t*)dout; a.ld_do = ld_do;
    a.lse = lse; a.delta = delta; a.delta_out = delta;
    a.dq = (bf16_t*)dq; a.dk = (bf16_t*)dk; a.dv = (bf16_t*)dv; a.ld_d = ld_dqkv;
    if (mfma_ok(dtype, head_dim, {o, dout}, {ld_o, ld_do})) {
      const unsigned vblocks = (unsigned)((rows * (head_dim / 8) + 255) / 256);
      if (head_dim == 64) hipLaunchKernelGGL(attn_delta_vec<64>, dim3(vblocks), dim3(256), 0, st, a);
      else hipLaunchKernelGGL(attn_delta_vec<128>, dim3(vblocks), dim3(256), 0, st, a);
    } else {
      hipLaunchKernelGGL(attn_delta<bf16_t>, dim3(dblocks), dim3(256), 0, st, a);
    }
    if (mfma_ok(dtype, head_dim, {q, k, v, dout, dq, dk, dv}, {ld_qkv, ld_do, ld_dqkv})) {
      dim3 gq((unsigned)((seq + 127) / 128), (unsigned)(batch * heads));
      dim3 gk((unsigned)((seq + 127) / 128), (unsigned)(batch * heads));
      if (head_dim == 64) {
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<64>, gk, dim3(256), 0, st, a);
        hipLaunchKernelGGL(attn_bwd_dq_mfma<64>, gq, dim3(256), 0, st, a);
      } else {
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<128>, gk, dim3(256), 0, st, a);
        hipLaunchKernelGGL(attn_bwd_dq_mfma<128>, gq, dim3(256), 0, st, a);
      }
    } else {
      dispatch_generic(a, st, false);
    }
  } else {
    AttnArgs<float> a = make_args<float>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const float*)q; a.k = (const float*)k; a.v = (const float*)v; a.ld_qkv = ld_qkv;
    a.o = (const float*)o; a.ld_o = ld_o; a.dout = (const float*)dout; a.ld_do = ld_do;
    a.lse = lse; a.delta = delta; a.delta_out = delta;
    a.dq = (float*)dq; a.dk = (float*)dk; a.dv = (float*)dv; a.ld_d = ld_dqkv;
    hipLaunchKernelGGL(attn_delta<float>, dim3(dblocks), dim3(256), 0, st, a);
    dispatch_generic(a, st, false);
  }
  return rh_check_launch("rh_attn_bwd");
}
