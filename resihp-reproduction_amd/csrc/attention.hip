// Fused causal self-attention (forward and backward) for gfx950.
//
// Math (per batch b, head h, query i, key j; scale = 1/sqrt(Dh)):
//   s_ij = scale * q_i.k_j,  masked to -inf for j > i when causal,
//   P = softmax_j(s),  o_i = sum_j P_ij v_j,  lse_i = log sum_j exp(s_ij)
// backward (delta_i = do_i.o_i):
//   dP_ij = do_i.v_j,  dS_ij = P_ij (dP_ij - delta_i)
//   dq_i = scale sum_j dS_ij k_j,  dk_j = scale sum_i dS_ij q_i,  dv_j = sum_i P_ij do_i
// P is rebuilt from lse in the backward; the [S,S] matrix never reaches HBM.
// delta must equal sum_j P_ij dP_ij (the identity that makes every row of dS sum to zero,
// so that dq_i = scale sum_j dS_ij (k_j - c) for any c): with bf16 outputs the forward also
// stores the rounding residual o - bf16(o) (in bf16), and delta is formed from both parts.
// From the rounded o alone, each row of dS sums to do_i.(o_i - bf16(o_i)) instead of zero
// and dq / dk pick up that error times the keys' / queries' common component (measured:
// ~2 % of the q/k projection gradients of a 12-layer GPT-2-small at its random init, 0.3 %
// with the residual).
//
// bf16 / head_dim 64 or 128: MFMA kernels built on v_mfma_f32_32x32x16_bf16.
// Scores are computed transposed (S^T = K Q^T, or S = Q K^T in the dK/dV kernel) so that
// every lane owns ONE query (one key) and 16 rows of each 32-row block: row max / row sum
// of the online softmax are lane-local plus one exchange with lane^32, and the
// probabilities feed the next MFMA straight from registers.
// 32x32 accumulator layout used throughout: register r of lane l holds
//   row 8*(r/4) + 4*(l/32) + r%4, column l%32;
// an operand fragment of lane l holds row/column l%32 and eight k values.
// The eight k values of lane group g = l/32 at step s of a 32-row block are the rows
// 16s + {4g..4g+3, 8+4g..8+4g+3}: exactly accumulator registers 8s..8s+7 of the score
// tile, so P^T needs no data movement; the matching V^T / K^T / dO^T / Q^T fragments
// are read from the same swizzled LDS tiles with ds_read_b64_tr_b16.
// Backward runs dQ first (it also produces delta) and then dK/dV; neither uses atomics,
// so results are bit-reproducible.
// Everything else (fp32, other head sizes): one thread per query (forward, dq)
// or per key (dk/dv) with K/V or Q/dO tiles staged in LDS; fp32 FMA.
#include <initializer_list>
#include <mutex>

#include "common.hpp"

namespace {

constexpr int kMaxDevices = 64;
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
  const T* o_lo;   // residual o - round(o) (bf16 only; may be null)
  T* o_lo_out;
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
  const T* olo = a.o_lo ? a.o_lo + t * a.ld_o + (int64_t)h * a.D : nullptr;
  const T* d = a.dout + t * a.ld_do + (int64_t)h * a.D;
  float s = 0.f;
  for (int i = 0; i < a.D; ++i) s = fmaf(ld_f32(o + i) + (olo ? ld_f32(olo + i) : 0.f), ld_f32(d + i), s);
  const int64_t b = t / a.S, sq = t % a.S;
  a.delta_out[(b * a.H + h) * a.S + sq] = s;
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
  T* olo = a.o_lo_out ? a.o_lo_out + (tok0 + qi) * a.ld_o + (int64_t)h * D : nullptr;
#pragma unroll
  for (int d = 0; d < DMAX; ++d)
    if (d < D) {
      const float v = o[d] * inv;
      st_f32(op + d, v);
      if (olo) st_f32(olo + d, v - ld_f32(op + d));
    }
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
// Work decomposition (all three kernels): an item is one (batch*head, 64-row block) pair --
// 64 queries for the forward and dQ kernels, 64 keys for the dK/dV kernel.  Items are
// numbered longest-causal-work first and workgroup c runs items c and n-1-c, so every
// workgroup gets the same amount of causal work.  A workgroup has 8 waves (two per SIMD):
// wave w owns 32 rows of the item (w & 1) and one of 4 phases (w >> 1).  Each stage streams
// 128 rows of the other operand (keys, or queries for dK/dV) into LDS; phase p works on
// rows 32p..32p+31 of the stage, and the 4 phases' partial results are merged in LDS at the
// end of the item in phase order (deterministic).
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
typedef __attribute__((address_space(3))) void lds_void_t;

// Element offset of (row r, column c) in a swizzled [rows][D] bf16 LDS tile.  The 16-byte
// chunk c/8 of row r is stored at chunk (c/8) ^ sw(r).  sw is chosen so that
//   * a ds_read_b128 of 16 consecutive rows at one chunk touches 16 distinct bank groups;
//   * a ds_read_b64_tr_b16 half-wave (4 consecutive rows x 2 adjacent 32-byte column pieces)
//     touches 8 distinct 32-byte bank groups.
template <int D>
__device__ __forceinline__ int swz(int r, int c) {
  const int sw = D == 128 ? (4 * (r & 3) + ((r >> 2) & 3)) : (4 * ((r >> 1) & 1) + ((r >> 2) & 3));
  return r * D + ((((c >> 3) ^ sw)) << 3) + (c & 7);
}

// Fragment reads by byte address.  In a swizzled tile row r starts at byte 2*D*r, and for the
// fragment shapes below the column-dependent part of the address is a per-lane base XORed
// with a compile-time constant (the k-step / head-dim block), because the swizzle XOR acts
// on the same address bits the constant selects.  Each lane therefore keeps one base per read
// pattern, and a read costs one v_xor on top of (stage base + row block): no per-fragment
// address registers.  Bases: row fragments -> row_base, transposed fragments -> tr_base(0/1).
template <int D>
__device__ __forceinline__ int swz_bits(int r) {
  return D == 128 ? (4 * (r & 3) + ((r >> 2) & 3)) : (4 * ((r >> 1) & 1) + ((r >> 2) & 3));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int D>
struct FragAddr {
  uint32_t row;    // row fragment: row l%32, chunk 2i + l/32
  uint32_t tr[2];  // transposed fragment, lo (rows 4g + i/4) and hi (+8) reads
  __device__ __forceinline__ explicit FragAddr(int lane) {
    const int g = lane >> 5, l32 = lane & 31;
    row = (uint32_t)(2 * D * l32 + 16 * (g ^ swz_bits<D>(l32)));
    const int q = lane >> 4, i = lane & 15;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = 4 * (q >> 1) + (i >> 2) + 8 * h;
      const int x = swz_bits<D>(rl) ^ (2 * (q & 1) + ((i & 3) >> 1));
      tr[h] = (uint32_t)(2 * D * rl + 16 * x + 8 * (i & 1));
    }
  }
};

// Operand fragment of rows r0 + lane%32 (r0 a multiple of 16), eight columns 16*ks + 8*(lane/32)
// (ds_read_b128).  `tile` is 256-byte aligned.
template <int D>
__device__ __forceinline__ bf16x8_t row_frag_at(uint32_t tile, int r0, int ks, const FragAddr<D>& fa) {
  const uint32_t a = (tile + (uint32_t)(2 * D * r0) + fa.row) ^ (uint32_t)(32 * ks);
  return *(const __attribute__((address_space(3))) bf16x8_t*)(uintptr_t)a;
}
template <int D>
__device__ __forceinline__ bf16x8_t row_frag(const bf16_t* tile, int r0, int ks, const FragAddr<D>& fa) {
  return row_frag_at<D>(lds_addr(tile), r0, ks, fa);
}

// Transposed operand fragment: rows of the MFMA operand are the 32 tile columns 32*db..+31,
// its eight k values are the tile rows r0 + {4g..4g+3, 8+4g..8+4g+3} (g = lane/32) -- the k
// order of accumulator registers 8s..8s+7.  Two ds_read_b64_tr_b16: in each 16-lane block,
// lane i addresses tile row r0 + 4g + i/4 (+8), columns 32*db + 16*(block&1) + 4*(i%4)..+3,
// and lane j receives those four rows of column 32*db + 16*(block&1) + j.
template <int D>
__device__ __forceinline__ bf16x8_t tr_frag_at(uint32_t tile, int r0, int db, const FragAddr<D>& fa) {
  const uint32_t base = tile + (uint32_t)(2 * D * r0);
  const uint32_t a0 = (base + fa.tr[0]) ^ (uint32_t)(64 * db);
  const uint32_t a1 = (base + fa.tr[1]) ^ (uint32_t)(64 * db);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(uintptr_t)a0);
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(uintptr_t)a1);
  s16x4_t both[2] = {lo, hi};
  return __builtin_bit_cast(bf16x8_t, both);
}
template <int D>
__device__ __forceinline__ bf16x8_t tr_frag(const bf16_t* tile, int r0, int db, const FragAddr<D>& fa) {
  return tr_frag_at<D>(lds_addr(tile), r0, db, fa);
}

// Every fragment address a wave reads from one 32-row block of a stage slot, precomputed per
// lane: the XOR constant of the k-step / head-dim block and the wave's row block are folded into
// one register per read pattern, so a read is a single ds_read whose immediate offset carries
// the stage slot (and the 16-row half of a transposed read).  Valid because tile slots and row
// blocks are multiples of 2*D*32 bytes and the swizzled in-block offsets stay below that.
template <int D>
struct BlockFrags {
  uint32_t row[D / 16];    // row fragment of k-step ks
  uint32_t tr[D / 32][2];  // transposed fragment of head-dim block db, lo / hi read
  __device__ __forceinline__ BlockFrags(const FragAddr<D>& fa, uint32_t block_base) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) row[ks] = block_base + (fa.row ^ (uint32_t)(32 * ks));
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int h = 0; h < 2; ++h) tr[db][h] = block_base + (fa.tr[h] ^ (uint32_t)(64 * db));
  }
  // row fragment ks of the block at byte offset `slot` (a compile-time constant in the callers)
  __device__ __forceinline__ bf16x8_t rowf(uint32_t slot, int ks) const {
    return *(const __attribute__((address_space(3))) bf16x8_t*)(uintptr_t)(row[ks] + slot);
  }
  // transposed fragment db of rows 16*half.. of the block at byte offset `slot`
  __device__ __forceinline__ bf16x8_t trf(uint32_t slot, int half, int db) const {
    const uint32_t o = slot + (uint32_t)(2 * D * 16 * half);
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(uintptr_t)(tr[db][0] + o));
    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(uintptr_t)(tr[db][1] + o));
    s16x4_t both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8_t, both);
  }
};

// ROWS rows x D of a [token][ld] bf16 matrix (rows r0.., clamped to `last`) into a swizzled
// LDS tile with direct global->LDS loads.  Each wave fills whole 1 KB windows of the tile: lane
// l of a window lands at window byte 16*l, i.e. physical chunk l % (D/8) of row
// l / (D/8); it therefore fetches the logical chunk that the swizzle puts there.  The per-lane
// byte offsets from the tile's first row are computed once (saddr loads: the row-r0 pointer is
// the wave-uniform base); only a stage that runs past `last` recomputes them, clamped so rows
// past `last` repeat row `last` (every consumer masks them out of the result).  The loads are
// asynchronous: callers wait with wait_vm() before the barrier that publishes the tile.
constexpr int kPhases = 4, kStageRows = 128;

template <int D, int ROWS = 128>
struct RowDma {
  static constexpr int CPR = D / 8;           // 16-byte chunks per row
  static constexpr int RPW = 64 / CPR;        // rows per 1 KB window
  static constexpr int WINDOWS = ROWS / RPW;  // windows per tile
  static constexpr int PER = WINDOWS / 8;     // windows per wave
  static_assert(WINDOWS % 8 == 0, "tile windows must split evenly over 8 waves");
  int64_t ld;
  // Byte offset of this lane's chunk from its window's first row.  The swizzle of window row r
  // depends only on r mod 16, and window wave + 8i starts at row (wave + 8i) * RPW, so the
  // offset is the same for every window of the wave: one register per operand.
  uint32_t off;

  __device__ __forceinline__ static int sw_chunk(int row, int pchunk) {
    const int sw = D == 128 ? (4 * (row & 3) + ((row >> 2) & 3)) : (4 * ((row >> 1) & 1) + ((row >> 2) & 3));
    return pchunk ^ sw;
  }
  static_assert((8 * RPW) % 16 == 0, "window rows of one wave must share the swizzle");
  __device__ __forceinline__ RowDma(int64_t ld_, int wave, int lane) : ld(ld_) {
    const int row = wave * RPW + lane / CPR;
    off = (uint32_t)(2 * (int64_t)(lane / CPR) * ld + 16 * sw_chunk(row, lane % CPR));
  }
  // The load, with the tile given as an LDS byte address: the stage's first row of this wave is
  // formed once and each further window is a fixed byte stride from it.
  __device__ __forceinline__ void issue(uint32_t tile, const bf16_t* base, int r0, int last, int wave,
                                        int lane) const {
    if (r0 + ROWS - 1 <= last) {
      const char* g = reinterpret_cast<const char*>(base + ((int64_t)r0 + wave * RPW) * ld);
#pragma unroll
      for (int i = 0; i < PER; ++i) dma16s(g + (int64_t)i * (16 * RPW) * ld, off, tile + (uint32_t)((wave + 8 * i) * 1024));
    } else {
      const bf16_t* sb = base + (int64_t)r0 * ld;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int row = (wave + 8 * i) * RPW + lane / CPR;
        const int grow = max(min(row, last - r0), 0);
        dma16s(sb, (uint32_t)(2 * (int64_t)grow * ld + 16 * sw_chunk(row, lane % CPR)),
               tile + (uint32_t)((wave + 8 * i) * 1024));
      }
    }
  }
};

__device__ __forceinline__ void wait_vm() { wait_vm_le<0>(); }

// Store 4 consecutive head-dim values (registers 4rr..4rr+3) as bf16.
__device__ __forceinline__ void st4(bf16_t* p, const floatx16_t& v, int rr, float mul) {
  u16x4_t u;
#pragma unroll
  for (int t = 0; t < 4; ++t) u[t] = f32_to_bf16(v[4 * rr + t] * mul);
  *reinterpret_cast<u16x4_t*>(p) = u;
}

// st4 plus the rounding residual of the same four values (bf16) at `lo`
__device__ __forceinline__ void st4_split(bf16_t* p, bf16_t* lo, const floatx16_t& v, int rr, float mul) {
  u16x4_t u, r;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float x = v[4 * rr + t] * mul;
    u[t] = f32_to_bf16(x);
    r[t] = f32_to_bf16(x - bf16_to_f32(u[t]));
  }
  *reinterpret_cast<u16x4_t*>(p) = u;
  *reinterpret_cast<u16x4_t*>(lo) = r;
}

// Load the 8 k-slices (16 d each) of one head-row as MFMA operand registers: lane l holds
// d = 16i + 8*(l/32) .. +7 of row `row` for slice i.
template <int KS>
__device__ __forceinline__ void load_head_row(bf16x8_t (&r)[KS], const bf16_t* p, bool ok, int g) {
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    u16x8_t u = {0, 0, 0, 0, 0, 0, 0, 0};
    if (ok) u = *reinterpret_cast<const u16x8_t*>(p + 16 * i + 8 * g);
    r[i] = __builtin_bit_cast(bf16x8_t, u);
  }
}

// item -> (batch*head, block), longest causal work first
struct Item {
  int bh, blk;
};
__device__ __forceinline__ Item item_q(int item, int BH, int nblk) { return {item % BH, nblk - 1 - item / BH}; }
__device__ __forceinline__ Item item_k(int item, int BH) { return {item % BH, item / BH}; }


// Merge per-phase fp32 register tiles (acc[OFF..OFF+NACC) per lane) of the 6 waves with phase > 0
// into the phase-0 waves, in phase order.  `cbuf` needs 6 * NACC * 16 * 64 floats.  On return
// (phase-0 waves) acc holds the sum.  Ends with the LDS free for reuse.
template <int OFF, int NACC, int N>
__device__ __forceinline__ void merge_phases(float* cbuf, floatx16_t (&acc)[N], int wave, int lane) {
  static_assert(OFF + NACC <= N, "merge range outside the accumulator array");
  const int sub = wave & 1, ph = wave >> 1;
  if (ph > 0) {
    float* dst = cbuf + (size_t)((ph - 1) * 2 + sub) * NACC * 16 * 64;
#pragma unroll
    for (int d = 0; d < NACC; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(d * 16 + r) * 64 + lane] = acc[OFF + d][r];
  }
  __syncthreads();
  if (ph == 0) {
#pragma unroll 1
    for (int p = 1; p < kPhases; ++p) {
      const float* src = cbuf + (size_t)((p - 1) * 2 + sub) * NACC * 16 * 64;
#pragma unroll
      for (int d = 0; d < NACC; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[OFF + d][r] += src[(d * 16 + r) * 64 + lane];
    }
  }
  __syncthreads();
}

// Row max of a 32x32 score tile (registers of the lane plus lane ^ 32), times the log2 scale.
__device__ __forceinline__ float tile_row_max(const floatx16_t& s, float c) {
  float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
  mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])), fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]))));
  const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx),
                                                   false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1])) * c;
}

// Lazy rescaling of the forward's running state: keep the running max m while no row's max grows
// by more than 8 (so every p = 2^(s*c - m) stays <= 256, far inside fp32 and bf16 range); the
// final division by the row sum makes the result independent of which max was used.
template <int DB>
__device__ __forceinline__ void lazy_rescale(float mx, floatx16_t (&oacc)[DB], float& m, float& lsum) {
  if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
    const float mnew = fmaxf(m, mx);
    const float corr = __builtin_amdgcn_exp2f(m - mnew);
    lsum *= corr;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[d][r] *= corr;
    m = mnew;
  }
}

// Forward.  Per wave and stage: Sᵀ = K·Qᵀ for the wave's 32 keys x 32 queries, online softmax,
// Oᵀ += Vᵀ·Pᵀ.
//  * Software pipeline across stages: the MFMAs of stage t+1's scores are interleaved, one by
//    one, with the exponentials of stage t's scores, and stage t's Oᵀ MFMAs follow; so the
//    matrix core and the VALU work side by side within each wave.  K therefore runs one stage
//    ahead of V: at the top of iteration t the LDS holds K(t+1) and V(t), and K(t+2) / V(t+1)
//    are loaded into the slots that K(t) / V(t-1) left (two slots per operand).
//  * Every fragment is read from LDS two MFMAs before its use (scheduling barriers keep that
//    order), so LDS latency is covered by the preceding MFMAs.
//  * Loads are explicit saddr direct-to-LDS loads (one offset register serves K and V, which
//    share a leading dimension), issued right after the barrier that frees their slot and
//    awaited just before the next one.
//  * Only the last stage of an item can hold masked keys (the causal diagonal, keys past S), so
//    every earlier stage runs one branch-free body; the loop takes two stages per trip so the
//    two score tiles swap roles without register copies.
//  * The 4 phases' partial outputs are merged by all 8 waves: each wave scales its partial by
//    its share of the row normaliser, writes it to LDS, and then sums (in phase order) and
//    stores 8 whole rows of the output with 16-byte row-contiguous stores.
template <int D>
__global__ __launch_bounds__(512) void attn_fwd_mfma(AttnArgs<bf16_t> a, int nitems) {
  constexpr int KS = D / 16, DB = D / 32, NPV = 2 * DB, TILE = kStageRows * D;
  constexpr int EPS = 16 / KS;       // scores exponentiated per score MFMA
  constexpr uint32_t TB = 2 * TILE;  // bytes per tile
  __shared__ __attribute__((aligned(256))) bf16_t smem[4 * TILE];  // K slots 0, 1 then V slots 0, 1
  __shared__ float mbuf[2][kPhases][2][64];                         // m and lsum of every wave
  __shared__ __attribute__((aligned(256))) bf16_t sQ[64 * D];       // the item's 64 query rows
  static_assert(kPhases * 64 * D * 4 <= 4 * TILE * 2, "merge buffer must fit the stages");
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, held in an SGPR
  const int sub = w & 1, ph = w >> 1;
  const FragAddr<D> fa(lane);
  const RowDma<D> dma(a.ld_qkv, w, lane);
  const RowDma<D, 64> qdma(a.ld_qkv, w, lane);
  const uint32_t sq0 = lds_addr(sQ);
  const int S = a.S, H = a.H, BH = a.B * a.H, nqb = (S + 63) / 64;
  const float c = a.scale * kLog2e;
  const uint32_t ks0 = lds_addr(smem), vs0 = ks0 + 2 * TB;
  // K fragments: the wave's 32 keys of a K slot; V fragments: the same keys of a V slot
  const BlockFrags<D> kf(fa, ks0 + (uint32_t)(2 * D * 32 * ph)), vf(fa, vs0 + (uint32_t)(2 * D * 32 * ph));

  for (int pass = 0; pass < 2; ++pass) {
    const int item = pass == 0 ? (int)blockIdx.x : nitems - 1 - (int)blockIdx.x;
    if (pass == 1 && item <= (int)blockIdx.x) break;
    const Item it = item_q(item, BH, nqb);
    const int b = it.bh / H, h = it.bh % H;
    const int64_t tok0 = (int64_t)b * S;
    const int wq0 = it.blk * 64 + 32 * sub, wq1 = wq0 + 31, q_row = wq0 + l32;
    const bf16_t* kbase = a.k + tok0 * a.ld_qkv + (int64_t)h * D;
    const bf16_t* vbase = a.v + tok0 * a.ld_qkv + (int64_t)h * D;
    const int kv_end = a.causal ? min(S, it.blk * 64 + 64) : S;
    const int nst = (kv_end + kStageRows - 1) / kStageRows;

    // The Q rows come through LDS like K and V (rows past S repeat row S-1; their results are
    // never stored): with no register loads in flight the compiler places no wait of its own,
    // whose count would also cover V(0) and K(1) and hold the first scores until those landed.
    qdma.issue(sq0, a.q + tok0 * a.ld_qkv + (int64_t)h * D, it.blk * 64, S - 1, w, lane);
    dma.issue(ks0, kbase, 0, S - 1, w, lane);
    dma.issue(vs0, vbase, 0, S - 1, w, lane);
    if (nst > 1) {
      dma.issue(ks0 + TB, kbase, kStageRows, S - 1, w, lane);
      wait_vm_le<2 * RowDma<D>::PER>();  // K(0) landed; V(0), K(1) may still be in flight
    } else {
      wait_vm_le<RowDma<D>::PER>();
    }
    __syncthreads();
    bf16x8_t qreg[KS];
#pragma unroll
    for (int i = 0; i < KS; ++i) qreg[i] = row_frag<D>(sQ, 32 * sub, i, fa);
    floatx16_t oacc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) oacc[d] = zero16();
    float m = -INFINITY, lsum = 0.f;
    // scores of the wave's block of stage 0 (computed whether or not the block is masked: the
    // last stage masks or skips it) and their row max
    floatx16_t sa = zero16(), sb;
#pragma unroll
    for (int i = 0; i < KS; ++i) sa = mfma32(kf.rowf(0, i), qreg[i], sa);
    float mxc = tile_row_max(sa, c);

    // One interior stage t (parity par = t & 1): every key of the wave's block precedes every
    // query of the wave, so nothing is masked.  `cur` holds stage t's scores (row max mxc) and
    // becomes its probabilities; `nxt` receives stage t+1's scores and mxc their row max.
    auto interior = [&](floatx16_t& cur, floatx16_t& nxt, int t, const uint32_t par) {
      wait_vm_le<0>();
      __syncthreads();  // K(t+1), V(t) visible; every wave is done with K(t) and V(t-1)
      if (t + 2 < nst) dma.issue(ks0 + par * TB, kbase, (t + 2) * kStageRows, S - 1, w, lane);
      dma.issue(vs0 + (par ^ 1) * TB, vbase, (t + 1) * kStageRows, S - 1, w, lane);
      const uint32_t kso = (par ^ 1) * TB, vso = par * TB;
      lazy_rescale<DB>(mxc, oacc, m, lsum);
      const float nm = -m;
      bf16x8_t kfr[KS], vfr[NPV], pb[2];
      kfr[0] = kf.rowf(kso, 0);
      kfr[1] = kf.rowf(kso, 1);
      nxt = zero16();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        if (i + 2 < KS) kfr[i + 2] = kf.rowf(kso, i + 2);
        else vfr[i + 2 - KS] = vf.trf(vso, (i + 2 - KS) / DB, (i + 2 - KS) % DB);
        nxt = mfma32(kfr[i], qreg[i], nxt);
#pragma unroll
        for (int e = 0; e < EPS; ++e) {
          const int r = i * EPS + e;
          cur[r] = __builtin_amdgcn_exp2f(fmaf(cur[r], c, nm));
          lsum += cur[r];
        }
        if (((i + 1) * EPS) % 8 == 0) pb[(i + 1) * EPS / 8 - 1] = pack8(cur, (i + 1) * EPS / 8 - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        if (j + 2 < NPV) vfr[j + 2] = vf.trf(vso, (j + 2) / DB, (j + 2) % DB);
        oacc[j % DB] = mfma32(vfr[j], pb[j / DB], oacc[j % DB]);
        __builtin_amdgcn_sched_barrier(0);
      }
      mxc = tile_row_max(nxt, c);
    };
    int t = 0;
    for (; t + 2 < nst; t += 2) {
      interior(sa, sb, t, 0u);
      interior(sb, sa, t + 1, 1u);
    }
    if (t + 1 < nst) {
      interior(sa, sb, t, 0u);
      sa = sb;
      ++t;
    }
    // the last stage: masks where a key can lie past the query (diagonal) or past S (tail)
    wait_vm_le<0>();
    __syncthreads();
    {
      const uint32_t vso = (uint32_t)(t & 1) * TB;
      const int kt0 = t * kStageRows + 32 * ph;
      if (wq0 < S && kt0 < kv_end && !(a.causal && kt0 > wq1)) {
        if ((a.causal && kt0 + 31 > wq0) || kt0 + 31 >= S) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= S || (a.causal && key > q_row)) sa[r] = -INFINITY;
          }
        }
        lazy_rescale<DB>(tile_row_max(sa, c), oacc, m, lsum);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sa[r] = __builtin_amdgcn_exp2f(fmaf(sa[r], c, -m));
          lsum += sa[r];
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t pb = pack8(sa, s2);
#pragma unroll
          for (int d = 0; d < DB; ++d) oacc[d] = mfma32(vf.trf(vso, s2, d), pb, oacc[d]);
        }
      }
    }

    // merge: normaliser of each row over the 4 phases, each wave's share of it
    __syncthreads();  // every wave is done with the stages, which become the merge buffer
    mbuf[0][ph][sub][lane] = m;
    mbuf[1][ph][sub][lane] = lsum;
    __syncthreads();
    float mall = -INFINITY;
#pragma unroll
    for (int p = 0; p < kPhases; ++p) mall = fmaxf(mall, mbuf[0][p][sub][lane]);
    float lall = 0.f;  // whole-row sum (both lane halves hold half of each block's keys)
#pragma unroll
    for (int p = 0; p < kPhases; ++p) {
      const float mp = mbuf[0][p][sub][lane];
      const float f = mp == -INFINITY ? 0.f : exp2f(mp - mall);
      lall += f * (mbuf[1][p][sub][lane] + mbuf[1][p][sub][lane ^ 32]);
    }
    const float share = (m == -INFINITY ? 0.f : exp2f(m - mall)) / lall;
    // partial outputs as fp32 [phase][row of the item][D], 16-byte chunk j of row q at j ^ (q & 7)
    float* part = reinterpret_cast<float*>(smem);
    const int q = 32 * sub + l32;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        floatx4_t v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = oacc[db][4 * rr + j] * share;
        const int chunk = 8 * db + 2 * rr + g;
        *reinterpret_cast<floatx4_t*>(part + ((ph * 64 + q) * (D / 4) + (chunk ^ (q & 7))) * 4) = v;
      }
    if (ph == 0 && g == 0 && q_row < S) a.lse_out[(int64_t)it.bh * S + q_row] = (mall + log2f(lall)) * kLn2;
    __syncthreads();
    {
      constexpr int CPL = D / 32;  // 16-byte fp32 chunks per lane: 8 lanes cover a row
      const int rq = 8 * w + (lane >> 3), row = it.blk * 64 + rq;
      floatx4_t acc[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < kPhases; ++p)
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int chunk = CPL * (lane & 7) + j;
          acc[j] += *reinterpret_cast<const floatx4_t*>(part + ((p * 64 + rq) * (D / 4) + (chunk ^ (rq & 7))) * 4);
        }
      if (row < S) {
        const int64_t off = (tok0 + row) * a.ld_o + (int64_t)h * D + 4 * CPL * (lane & 7);
#pragma unroll
        for (int j2 = 0; j2 < CPL / 2; ++j2) {
          u16x8_t hi, lo;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = acc[2 * j2 + e / 4][e % 4];
            hi[e] = f32_to_bf16(x);
            lo[e] = f32_to_bf16(x - bf16_to_f32(hi[e]));
          }
          *reinterpret_cast<u16x8_t*>(a.o_out + off + 8 * j2) = hi;
          if (a.o_lo_out) *reinterpret_cast<u16x8_t*>(a.o_lo_out + off + 8 * j2) = lo;
        }
      }
    }
    __syncthreads();  // the merge buffer is read out before the next item's loads overwrite it
  }
}

// dQ, plus delta_i = do_i . o_i for the dK/dV kernel (which runs after this one).
template <int D>
__global__ __launch_bounds__(512) void attn_bwd_dq_mfma(AttnArgs<bf16_t> a, int nitems) {
  constexpr int KS = D / 16, DB = D / 32, TILE = kStageRows * D;
  __shared__ __attribute__((aligned(256))) bf16_t smem[2 * 2 * TILE];  // 2 stages x (K, V)
  static_assert(6 * DB * 16 * 64 * 4 <= 2 * 2 * TILE * 2, "merge buffer must fit the stages");
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, held in an SGPR
  const int sub = w & 1, ph = w >> 1;
  const FragAddr<D> fa(lane);
  const int S = a.S, H = a.H, BH = a.B * a.H, nqb = (S + 63) / 64;
  const float c = a.scale * kLog2e;
  float* cbuf = reinterpret_cast<float*>(smem);
  // K and V stages load with explicit direct-to-LDS loads awaited by the loop's own wait at the
  // stage barrier; the compiler's waits (which would also count them) stay in the item prologue.
  const RowDma<D> kvdma(a.ld_qkv, w, lane);
  const uint32_t s0 = lds_addr(smem);  // stage st's K at s0 + 4*TILE*st bytes, its V 2*TILE bytes on

  for (int pass = 0; pass < 2; ++pass) {
    const int item = pass == 0 ? (int)blockIdx.x : nitems - 1 - (int)blockIdx.x;
    if (pass == 1 && item <= (int)blockIdx.x) break;
    const Item it = item_q(item, BH, nqb);
    const int b = it.bh / H, h = it.bh % H;
    const int64_t tok0 = (int64_t)b * S;
    const int wq0 = it.blk * 64 + 32 * sub, wq1 = wq0 + 31, q_row = wq0 + l32;
    const bool qok = q_row < S;

    // the first K/V stage goes out before the row loads below, so its latency overlaps theirs
    const bf16_t* kbase = a.k + tok0 * a.ld_qkv + (int64_t)h * D;
    const bf16_t* vbase = a.v + tok0 * a.ld_qkv + (int64_t)h * D;
    const int kv_end = a.causal ? min(S, it.blk * 64 + 64) : S;
    const int nst = (kv_end + kStageRows - 1) / kStageRows;
    kvdma.issue(s0, kbase, 0, S - 1, w, lane);
    kvdma.issue(s0 + 2 * TILE, vbase, 0, S - 1, w, lane);

    bf16x8_t qreg[KS], doreg[KS];
    load_head_row<KS>(qreg, a.q + (tok0 + q_row) * a.ld_qkv + (int64_t)h * D, qok, g);
    load_head_row<KS>(doreg, a.dout + (tok0 + q_row) * a.ld_do + (int64_t)h * D, qok, g);
    float del = 0.f;
    {
      const bf16_t* op = a.o + (tok0 + q_row) * a.ld_o + (int64_t)h * D;
      const bf16_t* olo = a.o_lo + (tok0 + q_row) * a.ld_o + (int64_t)h * D;
      const bool has_lo = a.o_lo != nullptr;
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        if (!qok) break;
        const u16x8_t ov = *reinterpret_cast<const u16x8_t*>(op + 16 * i + 8 * g);
        u16x8_t lv = {0, 0, 0, 0, 0, 0, 0, 0};
        if (has_lo) lv = *reinterpret_cast<const u16x8_t*>(olo + 16 * i + 8 * g);
        const u16x8_t dv = __builtin_bit_cast(u16x8_t, doreg[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) del = fmaf(bf16_to_f32(ov[j]) + bf16_to_f32(lv[j]), bf16_to_f32(dv[j]), del);
      }
      del += __shfl_xor(del, 32, 64);
    }
    if (ph == 0 && g == 0 && qok) a.delta_out[(int64_t)it.bh * S + q_row] = del;
    const float lse2 = qok ? a.lse[(int64_t)it.bh * S + q_row] * kLog2e : 0.f;
    floatx16_t dqt[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) dqt[d] = zero16();
    wait_vm();
    // Q and dO rows are in (the wait above covers every load): consumed here so the compiler's
    // own wait for them is not placed inside the loop, where it would also count the next
    // stage's loads (as in the dK/dV kernel).
#pragma unroll
    for (int i = 0; i < KS; ++i) asm volatile("" ::"v"(qreg[i]), "v"(doreg[i]));
    __syncthreads();
    // One stage in LDS slot `slot` (= t & 1, a compile-time constant: every fragment address of the
    // stage is a per-lane base plus an instruction immediate).
    auto stage = [&](int t, auto slot) {
      constexpr int cur = decltype(slot)::value;
      if (t + 1 < nst) {
        const uint32_t nxt = s0 + (uint32_t)((cur ^ 1) * 4 * TILE);
        kvdma.issue(nxt, kbase, (t + 1) * kStageRows, S - 1, w, lane);
        kvdma.issue(nxt + 2 * TILE, vbase, (t + 1) * kStageRows, S - 1, w, lane);
      }
      const bf16_t* sK = smem + cur * 2 * TILE;
      const bf16_t* sV = sK + TILE;
      const int kt0 = t * kStageRows + 32 * ph;
      if (wq0 < S && kt0 < kv_end && !(a.causal && kt0 > wq1)) {
        floatx16_t st = zero16(), dpt = zero16();
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          st = mfma32(row_frag<D>(sK, 32 * ph, i, fa), qreg[i], st);
          dpt = mfma32(row_frag<D>(sV, 32 * ph, i, fa), doreg[i], dpt);
        }
        // masked scores become -inf (p = 0, dS = 0) and every stage runs one straight-line body
        if ((a.causal && kt0 + 31 > wq0) || kt0 + 31 >= S || wq1 >= S) {  // diagonal or ragged stage
          const bool diag = a.causal && kt0 + 31 > wq0;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (!(qok && key < S && !(diag && key > q_row))) st[r] = -INFINITY;
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) st[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse2)) * (dpt[r] - del);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t dsb = pack8(st, s2);
#pragma unroll
          for (int d = 0; d < DB; ++d) dqt[d] = mfma32(tr_frag<D>(sK, 32 * ph + 16 * s2, d, fa), dsb, dqt[d]);
        }
      }
      wait_vm();
      __syncthreads();
    };
    int t = 0;
    for (; t + 1 < nst; t += 2) {
      stage(t, std::integral_constant<int, 0>{});
      stage(t + 1, std::integral_constant<int, 1>{});
    }
    if (t < nst) stage(t, std::integral_constant<int, 0>{});
    merge_phases<0, DB>(cbuf, dqt, w, lane);
    if (ph == 0 && qok) {
      bf16_t* dqp = a.dq + (tok0 + q_row) * a.ld_d + (int64_t)h * D;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) st4(dqp + d * 32 + 8 * rr + 4 * g, dqt[d], rr, a.scale);
    }
  }
}

template <int D>
__global__ __launch_bounds__(512) void attn_bwd_dkdv_mfma(AttnArgs<bf16_t> a, int nitems) {
  constexpr int KS = D / 16, DB = D / 32, TILE = kStageRows * D;
  __shared__ __attribute__((aligned(256))) bf16_t smem[2 * 2 * TILE];  // 2 stages x (Q, dO)
  __shared__ __attribute__((aligned(256))) bf16_t sVb[64 * D];          // the item's 64 rows of V
  __shared__ __attribute__((aligned(16))) float sL[2][kStageRows];
  __shared__ __attribute__((aligned(16))) float sDel[2][kStageRows];
  static_assert(6 * DB * 16 * 64 * 4 <= 2 * 2 * TILE * 2, "merge buffer must fit the stages");
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, held in an SGPR
  const int sub = w & 1, ph = w >> 1;
  const FragAddr<D> fa(lane);
  const int S = a.S, H = a.H, BH = a.B * a.H;
  const float c = a.scale * kLog2e;
  float* cbuf = reinterpret_cast<float*>(smem);

  for (int pass = 0; pass < 2; ++pass) {
    const int item = pass == 0 ? (int)blockIdx.x : nitems - 1 - (int)blockIdx.x;
    if (pass == 1 && item <= (int)blockIdx.x) break;
    const Item it = item_k(item, BH);
    const int b = it.bh / H, h = it.bh % H;
    const int64_t tok0 = (int64_t)b * S;
    const int wk0 = it.blk * 64 + 32 * sub;
    const int key = wk0 + l32;

    bf16x8_t kreg[KS];
    load_head_row<KS>(kreg, a.k + (tok0 + key) * a.ld_qkv + (int64_t)h * D, key < S, g);
    // V stays in LDS (registers are the binding limit at two waves per SIMD)
    RowDma<D, 64>(a.ld_qkv, w, lane).issue(lds_addr(sVb), a.v + tok0 * a.ld_qkv + (int64_t)h * D, it.blk * 64, S - 1, w, lane);
    floatx16_t acc[2 * DB];  // dK^T blocks 0..DB-1, dV^T blocks DB..2DB-1
#pragma unroll
    for (int d = 0; d < 2 * DB; ++d) acc[d] = zero16();

    const bf16_t* qbase = a.q + tok0 * a.ld_qkv + (int64_t)h * D;
    const bf16_t* dbase = a.dout + tok0 * a.ld_do + (int64_t)h * D;
    const float* lse = a.lse + (int64_t)it.bh * S;
    const float* dlt = a.delta + (int64_t)it.bh * S;
    const int q_start = a.causal ? it.blk * 64 : 0;
    const int nst = (S - q_start + kStageRows - 1) / kStageRows;
    // A stage's lse and delta go global->LDS like its Q and dO rows (waves 0 and 1, one query per
    // lane; queries past S read row S-1, whose results are masked), so the loop holds no load in
    // registers: a register load there makes the compiler wait on vmcnt inside the stage, and that
    // count also covers the next stage's direct-to-LDS loads, which would then land before the
    // stage computes instead of behind it.
    auto stats_dma = [&](int q0, int slot) {
      if (w < 2) {
        const uint32_t off = (uint32_t)(4 * min(q0 + tid, S - 1));
        dma4s(lse, off, lds_addr(&sL[slot][64 * w]));
        dma4s(dlt, off, lds_addr(&sDel[slot][64 * w]));
      }
    };
    const RowDma<D> qdma(a.ld_qkv, w, lane), ddma(a.ld_do, w, lane);
    const uint32_t s0 = lds_addr(smem);  // stage st's Q at s0 + 4*TILE*st bytes, its dO 2*TILE bytes on
    qdma.issue(s0, qbase, q_start, S - 1, w, lane);
    ddma.issue(s0 + 2 * TILE, dbase, q_start, S - 1, w, lane);
    stats_dma(q_start, 0);
    wait_vm();
    // The K rows have landed (the wait above covers every load); the compiler does not read
    // that from the asm, so the rows are consumed here, where its own wait for them is free,
    // rather than at their first use inside the loop, where its wait would count the next
    // stage's loads too.
#pragma unroll
    for (int i = 0; i < KS; ++i) asm volatile("" ::"v"(kreg[i]));
    __syncthreads();
    for (int t = 0; t < nst; ++t) {
      const int q0 = q_start + t * kStageRows;
      if (t + 1 < nst) {
        const uint32_t nxt = s0 + (uint32_t)(((t + 1) & 1) * 4 * TILE);
        qdma.issue(nxt, qbase, q0 + kStageRows, S - 1, w, lane);
        ddma.issue(nxt + 2 * TILE, dbase, q0 + kStageRows, S - 1, w, lane);
        stats_dma(q0 + kStageRows, (t + 1) & 1);
      }
      const int cur = t & 1;
      const bf16_t* sQ = smem + cur * 2 * TILE;
      const bf16_t* sdO = sQ + TILE;
      const int qt0 = q0 + 32 * ph;
      if (wk0 < S && qt0 < S && !(a.causal && qt0 + 31 < wk0)) {
        floatx16_t sc = zero16(), dp = zero16();
        // Q and dO fragments are fetched one k-step ahead, the V fragment at its use (registers
        // are the binding limit here); the scheduling barriers keep the compiler from hoisting
        // every LDS read of the stage
        bf16x8_t fq = row_frag<D>(sQ, 32 * ph, 0, fa), fd = row_frag<D>(sdO, 32 * ph, 0, fa);
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          bf16x8_t nq = fq, nd = fd;
          if (i + 1 < KS) {
            nq = row_frag<D>(sQ, 32 * ph, i + 1, fa);
            nd = row_frag<D>(sdO, 32 * ph, i + 1, fa);
          }
          sc = mfma32(fq, kreg[i], sc);
          dp = mfma32(fd, row_frag<D>(sVb, 32 * sub, i, fa), dp);
          __builtin_amdgcn_sched_barrier(0);
          fq = nq;
          fd = nd;
        }
        const bool diag = a.causal && qt0 < wk0 + 31;
        const bool ragged = diag || qt0 + 31 >= S || wk0 + 31 >= S;  // any element masked
        // Masked scores become -inf (so p = 2^-inf = 0 and dS = 0; lse and delta are finite for
        // every row read) and every stage runs one straight-line softmax body.  Selecting p per
        // element instead makes the compiler branch around each exponential, and that exec-mask
        // juggling (about 8 scalar instructions per score) ran on every stage.
        if (ragged) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int q = q0 + 32 * ph + 8 * (r >> 2) + 4 * g + (r & 3);
            if (!(q < S && key < S && !(diag && key > q))) sc[r] = -INFINITY;
          }
        }
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int qi0 = 32 * ph + 8 * r4 + 4 * g;
          const floatx4_t lq = *reinterpret_cast<const floatx4_t*>(&sL[cur][qi0]);
          const floatx4_t dq4 = *reinterpret_cast<const floatx4_t*>(&sDel[cur][qi0]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * r4 + j;
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[r], c, -lq[j] * kLog2e));
            dp[r] = p * (dp[r] - dq4[j]);
            sc[r] = p;
          }
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t pb = pack8(sc, s2), dsb = pack8(dp, s2);
          bf16x8_t fo = tr_frag<D>(sdO, 32 * ph + 16 * s2, 0, fa), fq2 = tr_frag<D>(sQ, 32 * ph + 16 * s2, 0, fa);
#pragma unroll
          for (int d = 0; d < DB; ++d) {
            bf16x8_t no = fo, nq = fq2;
            if (d + 1 < DB) {
              no = tr_frag<D>(sdO, 32 * ph + 16 * s2, d + 1, fa);
              nq = tr_frag<D>(sQ, 32 * ph + 16 * s2, d + 1, fa);
            }
            acc[DB + d] = mfma32(fo, pb, acc[DB + d]);
            acc[d] = mfma32(fq2, dsb, acc[d]);
            __builtin_amdgcn_sched_barrier(0);
            fo = no;
            fq2 = nq;
          }
        }
      }
      wait_vm();
      __syncthreads();
    }
    // merge dK^T then dV^T over the phases (the merge buffer holds DB accumulators per wave)
    merge_phases<0, DB>(cbuf, acc, w, lane);
    merge_phases<DB, DB>(cbuf, acc, w, lane);
    if (ph == 0 && key < S) {
      bf16_t* dkp = a.dk + (tok0 + key) * a.ld_d + (int64_t)h * D;
      bf16_t* dvp = a.dv + (tok0 + key) * a.ld_d + (int64_t)h * D;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          st4(dkp + d * 32 + 8 * rr + 4 * g, acc[d], rr, a.scale);
          st4(dvp + d * 32 + 8 * rr + 4 * g, acc[DB + d], rr, 1.f);
        }
    }
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
  RH_REQUIRE(B * H * ((S + 63) / 64) < INT32_MAX, "rh_attn: %lld x %lld row blocks exceed the launch limit",
             (long long)(B * H), (long long)((S + 63) / 64));
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

// MFMA kernels: one item per (batch*head, 64-row block); each workgroup runs two items.
int mfma_items(int64_t batch, int64_t seq, int64_t heads) { return (int)(batch * heads * ((seq + 63) / 64)); }

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
                           const void* k, const void* v, int64_t ld_qkv, void* o, void* o_lo, int64_t ld_o,
                           float* lse, float scale, int causal, void* stream) {
  int rc = check_common(dtype, batch, seq, heads, head_dim);
  if (rc) return rc;
  if (batch == 0 || seq == 0 || heads == 0) return RH_OK;
  RH_REQUIRE(q && k && v && o && lse, "rh_attn_fwd: null pointer");
  RH_REQUIRE(ld_qkv >= heads * head_dim && ld_o >= heads * head_dim, "rh_attn_fwd: leading dimension too small");
  RH_REQUIRE(scale > 0.f, "rh_attn_fwd: scale must be positive (got %g)", (double)scale);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype != RH_DTYPE_BF16) o_lo = nullptr;  // fp32 outputs are not rounded
  if (mfma_ok(dtype, head_dim, {q, k, v, o, o_lo ? o_lo : o}, {ld_qkv, ld_o})) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o_out = (bf16_t*)o; a.o_lo_out = (bf16_t*)o_lo; a.ld_o = ld_o; a.lse_out = lse;
    const int nitems = mfma_items(batch, seq, heads);
    dim3 grid((unsigned)((nitems + 1) / 2));
    if (head_dim == 64) hipLaunchKernelGGL(attn_fwd_mfma<64>, grid, dim3(512), 0, st, a, nitems);
    else hipLaunchKernelGGL(attn_fwd_mfma<128>, grid, dim3(512), 0, st, a, nitems);
    return rh_check_launch("rh_attn_fwd");
  }
  if (dtype == RH_DTYPE_BF16) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o_out = (bf16_t*)o; a.o_lo_out = (bf16_t*)o_lo; a.ld_o = ld_o; a.lse_out = lse;
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

static int attn_bwd_check(const char* who, int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                          const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, int64_t ld_o,
                          const void* dout, int64_t ld_do, const float* lse, void* dq, void* dk, void* dv,
                          int64_t ld_dqkv, float scale) {
  int rc = check_common(dtype, batch, seq, heads, head_dim);
  if (rc) return rc;
  if (batch == 0 || seq == 0 || heads == 0) return RH_OK;
  RH_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, "%s: null pointer", who);
  RH_REQUIRE(scale > 0.f, "%s: scale must be positive (got %g)", who, (double)scale);
  const int64_t width = heads * head_dim;
  RH_REQUIRE(ld_qkv >= width && ld_o >= width && ld_do >= width && ld_dqkv >= width,
             "%s: leading dimension too small", who);
  return RH_OK;
}

// The backward after the argument checks.  `delta` holds batch*seq*heads floats; every row is
// written (by the dQ kernel or attn_delta) before the dK/dV pass reads it, so its previous
// contents do not matter.
static int attn_bwd_launch(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, const void* q,
                           const void* k, const void* v, int64_t ld_qkv, const void* o, const void* o_lo,
                           int64_t ld_o, const void* dout, int64_t ld_do, const float* lse, void* dq, void* dk,
                           void* dv, int64_t ld_dqkv, float scale, int causal, float* delta, hipStream_t st) {
  const int64_t rows = batch * seq * heads;  const unsigned dblocks = (unsigned)((rows + 255) / 256);
  if (dtype == RH_DTYPE_BF16) {
    AttnArgs<bf16_t> a = make_args<bf16_t>(batch, seq, heads, head_dim, scale, causal);
    a.q = (const bf16_t*)q; a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.ld_qkv = ld_qkv;
    a.o = (const bf16_t*)o; a.o_lo = (const bf16_t*)o_lo; a.ld_o = ld_o; a.dout = (const bf16_t*)dout; a.ld_do = ld_do;
    a.lse = lse; a.delta = delta; a.delta_out = delta;
    a.dq = (bf16_t*)dq; a.dk = (bf16_t*)dk; a.dv = (bf16_t*)dv; a.ld_d = ld_dqkv;
    if (mfma_ok(dtype, head_dim, {q, k, v, o, o_lo ? o_lo : o, dout, dq, dk, dv}, {ld_qkv, ld_o, ld_do, ld_dqkv})) {
      // the dQ kernel also writes delta, which the dK/dV kernel reads
      const int nitems = mfma_items(batch, seq, heads);
      dim3 grid((unsigned)((nitems + 1) / 2));
      if (head_dim == 64) {
        hipLaunchKernelGGL(attn_bwd_dq_mfma<64>, grid, dim3(512), 0, st, a, nitems);
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<64>, grid, dim3(512), 0, st, a, nitems);
      } else {
        hipLaunchKernelGGL(attn_bwd_dq_mfma<128>, grid, dim3(512), 0, st, a, nitems);
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<128>, grid, dim3(512), 0, st, a, nitems);
      }
    } else {
      hipLaunchKernelGGL(attn_delta<bf16_t>, dim3(dblocks), dim3(256), 0, st, a);
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

extern "C" int rh_attn_bwd(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, const void* q,
                           const void* k, const void* v, int64_t ld_qkv, const void* o, const void* o_lo, int64_t ld_o,
                           const void* dout, int64_t ld_do, const float* lse, void* dq, void* dk, void* dv,
                           int64_t ld_dqkv, float scale, int causal, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  int rc = attn_bwd_check("rh_attn_bwd", dtype, batch, seq, heads, head_dim, q, k, v, ld_qkv, o, ld_o, dout, ld_do,
                          lse, dq, dk, dv, ld_dqkv, scale);
  if (rc || batch == 0 || seq == 0 || heads == 0) return rc;
  RH_REQUIRE(workspace && workspace_bytes >= batch * seq * heads * (int64_t)sizeof(float),
             "rh_attn_bwd: workspace of %lld bytes is too small", (long long)workspace_bytes);
  return attn_bwd_launch(dtype, batch, seq, heads, head_dim, q, k, v, ld_qkv, o, o_lo, ld_o, dout, ld_do, lse, dq, dk,
                         dv, ld_dqkv, scale, causal, static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// rh_attn_bwd_noalloc: the same backward with its delta rows in a static device array.
// In host code `scratch` is only a stand-in for the array: its address on the current GPU
// comes from hipGetSymbolAddress, once per device, and only that address reaches a kernel.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[RH_ATTN_NOALLOC_MAX_ROWS];

static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices] = {};

static int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return rh_set_error(RH_ERR_HIP, "rh_attn_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  RH_REQUIRE(dev >= 0 && dev < kMaxDevices, "rh_attn_bwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return rh_set_error(RH_ERR_HIP, "rh_attn_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                          hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return RH_OK;
}

extern "C" int rh_attn_bwd_noalloc(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                                   const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o,
                                   const void* o_lo, int64_t ld_o, const void* dout, int64_t ld_do, const float* lse,
                                   void* dq, void* dk, void* dv, int64_t ld_dqkv, float scale, int causal,
                                   void* stream) {
  int rc = attn_bwd_check("rh_attn_bwd_noalloc", dtype, batch, seq, heads, head_dim, q, k, v, ld_qkv, o, ld_o, dout,
                          ld_do, lse, dq, dk, dv, ld_dqkv, scale);
  if (rc || batch == 0 || seq == 0 || heads == 0) return rc;
  RH_REQUIRE(batch * seq * heads <= RH_ATTN_NOALLOC_MAX_ROWS,
             "rh_attn_bwd_noalloc: batch*seq*heads = %lld query rows exceeds the static scratch of %d rows",
             (long long)(batch * seq * heads), RH_ATTN_NOALLOC_MAX_ROWS);
  float* delta = nullptr;
  rc = scratch_on_current_device(&delta);
  if (rc) return rc;
  return attn_bwd_launch(dtype, batch, seq, heads, head_dim, q, k, v, ld_qkv, o, o_lo, ld_o, dout, ld_do, lse, dq, dk,
                         dv, ld_dqkv, scale, causal, delta, static_cast<hipStream_t>(stream));
}
