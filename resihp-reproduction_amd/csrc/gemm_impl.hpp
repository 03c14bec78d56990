// Dense GEMMs of the decoder block (F.linear and its backward) for gfx950.
//
// bf16 path (MFMA).  Workgroup tiles of BM x BN x 64 built from
// v_mfma_f32_32x32x16_bf16 (measured on MI355X: ~2.1 PFLOP/s sustained for both the
// 32x32x16 and 16x16x32 forms; the 32x32 form needs half the operand reads).  Three tile
// shapes:
//   256x256, 8 waves (2x4, 128x64 per wave)   -- large outputs
//   256x128, 8 waves (4x2,  64x64 per wave)   -- medium
//   128x128, 4 waves (2x2,  64x64 per wave)   -- small / split-K
// chosen per call by the number of tiles against the CU count.
//
// Two main loops share the LDS layouts, fragment reads and epilogue:
//   gemm_bf16_dma  -- operands go global->LDS with direct-to-LDS loads (the default
//                     whenever the operands can be addressed without bounds checks);
//   gemm_bf16_mfma -- operands staged through registers with bounds checks (ragged
//                     edges, K not a multiple of 64, unaligned rows).
// Both double-buffer the LDS tiles (loads of k-tile t+1 in flight while the MFMAs of
// tile t run; one barrier per k-tile):
//   k-contiguous operand  (A of NT/NN, B of NT): LDS [rows][64], 128-byte rows,
//     16-byte chunk c of row r stored at chunk c ^ ((r >> 1) & 7), so the 16
//     rows a ds_read_b128 phase touches hit 16 distinct bank groups;
//   m/n-contiguous operand (A of TN, B of NN/TN): LDS [64][cols] exactly as in
//     memory, 32-element unit u of row k stored at u ^ (k & 3),
//     and MFMA fragments are read with ds_read_b64_tr_b16: in each 16-lane
//     block, lane i addresses row k0 + i/4, columns c0 + 4*(i%4) .. +3, and lane
//     j receives rows k0..k0+3 of column c0 + j -- a k-major fragment without
//     any scalar transposition.
// Two epilogues (epilogue_sel picks one per call): LDS-staged (epilogue_tile_impl: the fp32 tile
// goes through LDS so stores are 16-byte, whole-row runs) and from registers (epilogue_regs: a
// DPP quad transpose gives each lane 4 consecutive columns of one output row; no LDS round trip,
// no barrier, each wave finishes as soon as its own MFMAs retire).
// Workgroup ids are remapped so that each XCD (ids are dealt round-robin over
// the 8 XCDs) works on one contiguous run of a GROUP_M-grouped tile order:
// tiles sharing A rows / B columns land in the same XCD's L2.
//
// fp32 path: 64x64x16 FMA tile (4x4 outputs per thread) for the fp32 parity
// mode, where no bf16 rounding may enter.
//
// Split-K: when the output has too few tiles for the chip and K is long (the
// wgrad shapes), grid.z partitions K, each split writes fp32 partials to the
// caller's workspace, and a reduce kernel sums them in split order
// (deterministic) and applies the epilogue.
#pragma once

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "common.hpp"

int rh_device_cus();

// Everything the layout translation units (gemm_nt/nn/tn.hip) and the entry points (gemm.hip)
// share; launch_layout is instantiated once per layout, in that layout's unit.
namespace rh_gemm_impl {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

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
  int out_vec;          // D/C/aux rows 8-byte aligned, split partials 16-byte aligned
  int epi_lds;          // finish through LDS (epilogue_tile_impl) instead of epilogue_regs
  int w4;               // the 4-wave 256x256 kernel may address the operands (w4_addressable)
  int tiles_m, tiles_n, group_m;
  // next-token cross-entropy epilogues of the LM head (kEpiLsePartial, kEpiXentGrad); row m of the
  // output is token m = b*seq + s, scored against tokens[m + 1] unless s == seq - 1, and output
  // column n is vocabulary id col_off + n
  const int64_t* tokens;
  const float* lse;     // kEpiXentGrad: natural-log log-sum-exp of each row
  float* part;          // kEpiLsePartial: (max, sum) of each row's 64-column blocks, base-2 units
  float* tgt;           // kEpiLsePartial: the target logit of each scored row
  const float* grad;    // kEpiXentGrad: d loss / d mean loss (device scalar)
  float inv_n;          // 1 / scored rows
  int64_t seq, col_off, n_store, ld_part;
};

// Internal epilogues of the fused LM-head cross-entropy (not part of the public RH_EPI_* set).
constexpr int kEpiLsePartial = 16;
constexpr int kEpiXentGrad = 17;

// Row r of a segmented result: the segment by comparisons (at most RH_MAX_SEG - 1 of them) rather
// than a division, which is a long scalar/vector sequence for 64-bit values, and the epilogues
// form one per output row.  The segment bases pass through an empty asm so the compiler keeps the
// selects instead of re-forming a per-lane indexed read of the argument array (which it would
// place in scratch memory).  (b_row runs once per tile in the loaders' set-up and keeps the
// division.)
template <typename P>
__device__ __forceinline__ P seg_row(const P (&base)[RH_MAX_SEG], int nseg, int64_t seg, int64_t r, int64_t ld) {
  if (nseg == 1) return base[0] + r * ld;
  P b = base[0];
#pragma unroll
  for (int k = 1; k < RH_MAX_SEG; ++k) {
    P bk = base[k];
    asm volatile("" : "+s"(bk));
    if (k < nseg && r >= seg) {
      r -= seg;
      b = bk;
    }
  }
  return b + r * ld;
}
template <typename T>
__device__ __forceinline__ const T* b_row(const GemmParams<T>& p, int64_t r) {
  if (p.b_nseg == 1) return p.B[0] + r * p.ldb;
  const int64_t s = r / p.b_seg;
  return p.B[s] + (r - s * p.b_seg) * p.ldb;
}
template <typename T>
__device__ __forceinline__ T* d_row(const GemmParams<T>& p, int64_t m) {
  return seg_row(p.D, p.d_nseg, p.d_seg, m, p.ldd);
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
  constexpr bool kBf16 = std::is_same<T, bf16_t>::value;  // bf16 results: fast GELU (see common.hpp)
  if (EPI == RH_EPI_GELU) {
    st_f32(p.aux_out + m * p.ldaux + n, v);
    v = kBf16 ? gelu_fast_f(v) : gelu_f(v);
  } else if (EPI == RH_EPI_GELU_DERIV) {
    st_f32(p.aux_out + m * p.ldaux + n, kBf16 ? gelu_grad_fast_f(v) : gelu_grad_f(v));
    v = kBf16 ? gelu_fast_f(v) : gelu_f(v);
  } else if (EPI == RH_EPI_GELU_GRAD) {
    const float a = ld_f32(p.aux + m * p.ldaux + n);
    v *= kBf16 ? gelu_grad_fast_f(a) : gelu_grad_f(a);
  } else if (EPI == RH_EPI_MUL_AUX) {
    v *= ld_f32(p.aux + m * p.ldaux + n);
  }
  st_f32(drow + n, v);
}

// The epilogue on 8 consecutive outputs of one row (bf16 storage): aux read/write and the
// GELU forms.  `xp` is the aux row pointer for this chunk (aux_out or aux by epilogue).
template <int EPI>
__device__ __forceinline__ void epi8_bf16(float (&v)[8], bf16_t* xp) {
  if (EPI == RH_EPI_GELU || EPI == RH_EPI_GELU_DERIV) {
    u16x8_t o;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const GeluParts g = gelu_parts_fast(v[t]);
      o[t] = f32_to_bf16(EPI == RH_EPI_GELU ? v[t] : g.cdf + v[t] * g.pdf);
      v[t] *= g.cdf;
    }
    *reinterpret_cast<u16x8_t*>(xp) = o;
  } else if (EPI == RH_EPI_GELU_GRAD || EPI == RH_EPI_MUL_AUX) {
    const u16x8_t a = *reinterpret_cast<const u16x8_t*>(xp);
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] *= EPI == RH_EPI_GELU_GRAD ? gelu_grad_fast_f(bf16_to_f32(a[t])) : bf16_to_f32(a[t]);
  }
}

template <int EPI>
constexpr bool epi_writes_aux() { return EPI == RH_EPI_GELU || EPI == RH_EPI_GELU_DERIV; }
template <int EPI>
constexpr bool epi_reads_aux() { return EPI == RH_EPI_GELU_GRAD || EPI == RH_EPI_MUL_AUX; }

// XCD-aware, GROUP_M-grouped tile coordinates of this workgroup.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int nwg = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int q = nwg / 8, r = nwg % 8;
  const int xcd = bid % 8, idx = bid / 8;
  const int logical = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + idx;
  const int per_group = group_m * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in = logical - g * per_group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

// ---------------------------------------------------------------------------
// bf16 MFMA kernel
// ---------------------------------------------------------------------------
constexpr int kBK = 64;

// element offset of (row r, 16-byte chunk c) in a k-contiguous [R][64] tile
__device__ __forceinline__ int kc_off(int r, int c) { return r * kBK + ((c ^ ((r >> 1) & 7)) << 3); }
// element offset of (k row, column col) in an m/n-contiguous [64][R] tile
template <int R>
__device__ __forceinline__ int mc_off(int k, int col) {
  return k * R + ((((col >> 5) ^ (k & 3))) << 5) + (col & 31);
}

// One operand tile (ROWS = m or n extent, 64 k), global -> registers -> LDS.
//   KC: global row r is k-contiguous: element (r, k) = rowptr(r)[k]
//   !KC: global row k is r-contiguous: element (r, k) = rowptr(k)[r]
template <int ROWS, bool KC, int NT>
struct TileIO {
  static constexpr int kChunks = ROWS * kBK / 8;
  static constexpr int kPer = kChunks / NT;
  static_assert(kChunks % NT == 0, "tile must split evenly over the threads");
  u16x8_t reg[kPer];

  template <typename RowFn>
  __device__ __forceinline__ void load(RowFn rowptr, int64_t o0, int64_t k0, int64_t outer_lim, int64_t k_lim,
                                       bool fast, bool aligned) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * NT;
      int64_t r, k;
      if (KC) {
        r = o0 + c / (kBK / 8);
        k = k0 + (c % (kBK / 8)) * 8;
      } else {
        k = k0 + c / (ROWS / 8);
        r = o0 + (c % (ROWS / 8)) * 8;
      }
      u16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (fast) {
        v = *reinterpret_cast<const u16x8_t*>(KC ? rowptr(r) + k : rowptr(k) + r);
      } else if (KC) {
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

  __device__ __forceinline__ void store(bf16_t* s) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * NT;
      if (KC) {
        const int r = c / (kBK / 8), ch = c % (kBK / 8);
        *reinterpret_cast<u16x8_t*>(s + kc_off(r, ch)) = reg[i];
      } else {
        const int k = c / (ROWS / 8), col = (c % (ROWS / 8)) * 8;
        *reinterpret_cast<u16x8_t*>(s + mc_off<ROWS>(k, col)) = reg[i];
      }
    }
  }
};

// MFMA fragment (32 rows/cols starting at rb, k-step ks) from an LDS tile.
template <int ROWS, bool KC>
__device__ __forceinline__ bf16x8_t load_frag(const bf16_t* s, int rb, int ks, int lane) {
  if (KC) {
    const int r = rb + (lane & 31);
    return *reinterpret_cast<const bf16x8_t*>(s + kc_off(r, ks * 2 + (lane >> 5)));
  } else {
    const int q = lane >> 4, i = lane & 15;
    const int col = rb + 16 * (q & 1) + 4 * (i & 3);
    const int k = ks * 16 + 8 * (q >> 1) + (i >> 2);
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(s + mc_off<ROWS>(k, col)));
    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(s + mc_off<ROWS>(k + 4, col)));
    s16x4_t both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8_t, both);
  }
}

// Interior-tile operand loader: every chunk in bounds and 16-byte aligned, per-thread
// pointers set up once; one k-tile advance is a pointer add (k-contiguous) or a
// scalar row-base computation (m/n-contiguous, where a k-tile never straddles a
// q/k/v segment).
template <int ROWS, bool KC, int NT>
struct FastIO {
  static constexpr int kChunks = ROWS * kBK / 8;
  static constexpr int kPer = kChunks / NT;
  u16x8_t reg[kPer];
  const bf16_t* ptr[kPer];  // KC: chunk pointers at k = kbeg
  int64_t off[kPer];        // !KC: element offset of each chunk from its k-tile's first row

  template <typename RowFn>
  __device__ __forceinline__ void setup(RowFn rowptr, int64_t o0, int64_t kbeg, int64_t ld) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * NT;
      if (KC) {
        ptr[i] = rowptr(o0 + c / (kBK / 8)) + kbeg + (c % (kBK / 8)) * 8;
      } else {
        off[i] = (int64_t)(c / (ROWS / 8)) * ld + o0 + (c % (ROWS / 8)) * 8;
      }
    }
  }

  // k-tile starting at k0 (= kbeg + kt*kBK); `base` is the row pointer of row k0 (!KC only)
  __device__ __forceinline__ void load(int kt, const bf16_t* base) {
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      reg[i] = KC ? *reinterpret_cast<const u16x8_t*>(ptr[i] + (int64_t)kt * kBK)
                  : *reinterpret_cast<const u16x8_t*>(base + off[i]);
  }

  __device__ __forceinline__ void store(bf16_t* s) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + i * NT;
      if (KC) {
        *reinterpret_cast<u16x8_t*>(s + kc_off(c / (kBK / 8), c % (kBK / 8))) = reg[i];
      } else {
        *reinterpret_cast<u16x8_t*>(s + mc_off<ROWS>(c / (ROWS / 8), (c % (ROWS / 8)) * 8)) = reg[i];
      }
    }
  }
};

template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC, int FM, int FN>
__device__ __forceinline__ void mma_ktile(const bf16_t* a_s, const bf16_t* b_s, floatx16_t (&acc)[FM][FN], int wm,
                                          int wn, int lane) {
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
    bf16x8_t af[FM], bfr[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = load_frag<BM, A_KC>(a_s, wm * WTM + i * 32, ks, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[j] = load_frag<BN, B_KC>(b_s, wn * WTN + j * 32, ks, lane);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  }
}

// Accumulate into AGPRs.  A 128x128 wave tile needs 256 accumulator registers, all of the
// architectural VGPRs, so they must live in the accumulation registers; with the builtin the
// register allocator keeps them in VGPRs and spills.  The compiler does not see this as an MFMA:
// the caller waits out the MFMA-result hazard (mfma_asm_drain) before reading the accumulators.
__device__ __forceinline__ void mfma_agpr(floatx16_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Volatile asm statements keep their order, so an empty statement that "modifies" every
// accumulator after the wait pins every later read of them behind it.
template <int FM, int FN>
__device__ __forceinline__ void agpr_fence(floatx16_t (&acc)[FM][FN]) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) asm volatile("" : "+a"(acc[i][j]));
}
// Before the first MFMA: the accumulators' zeroing (VALU writes) is done, plus 5 wait states.
template <int FM, int FN>
__device__ __forceinline__ void mfma_asm_begin(floatx16_t (&acc)[FM][FN]) {
  agpr_fence(acc);
  asm volatile("s_nop 4" ::: "memory");
}
// After the last MFMA: 24 wait states, more than a 32x32x16 MFMA's result latency for a VALU read.
template <int FM, int FN>
__device__ __forceinline__ void mfma_asm_drain(floatx16_t (&acc)[FM][FN]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  agpr_fence(acc);
}

// 4x4 transpose across the four lanes of each quad (DPP quad_perm, two exchange stages): on
// entry lane s = lane % 4 holds v[t] = element (t, s) of a 4x4 block, on exit element (s, t).
template <int CTRL>
__device__ __forceinline__ float quad_perm_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ void quad_transpose(float (&v)[4], int lane) {
  const bool b0 = lane & 1, b1 = lane & 2;
#pragma unroll
  for (int k = 0; k < 4; k += 2) {  // exchange bit 0 of (register, lane) with the neighbour lane ^ 1
    const float got = quad_perm_f32<0xB1>(b0 ? v[k] : v[k + 1]);  // quad_perm [1,0,3,2]
    if (b0) v[k] = got; else v[k + 1] = got;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {  // exchange bit 1 with lane ^ 2
    const float got = quad_perm_f32<0x4E>(b1 ? v[k] : v[k + 2]);  // quad_perm [2,3,0,1]
    if (b1) v[k] = got; else v[k + 2] = got;
  }
}

// Register epilogue, no LDS and no barrier: each wave finishes its own WTM x WTN sub-tile as soon
// as its last MFMA retires.  32x32 accumulator: register r of lane l holds row 8*(r/4) + 4*(l/32)
// + r%4, column l%32; a quad transpose turns every 4 registers into 4 consecutive columns of one
// row, so C / aux reads and D / aux / partial writes are 8-byte (fp32 partials: 16-byte) vectors,
// 64 contiguous bytes per row per instruction.  All C and aux reads are issued before any is
// used.  Sub-tiles that cross the matrix edge (or unaligned rows) take the per-element path.
template <int BM, int BN, int WGM, int WGN, int EPI, bool SPLIT, int FM, int FN>
__device__ __forceinline__ void epilogue_regs(const GemmParams<bf16_t>& p, floatx16_t (&acc)[FM][FN], int64_t m0,
                                              int64_t n0, int wm, int wn, int lane, int split) {
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  const int64_t wr0 = m0 + (int64_t)wm * WTM, wc0 = n0 + (int64_t)wn * WTN;
  const int g = lane >> 5;
  if (!(p.out_vec && wr0 + WTM <= p.M && wc0 + WTN <= p.N)) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const floatx16_t a = acc[i][j];  // a register copy: the rolled loop below indexes it by r
#pragma unroll 1
        for (int r = 0; r < 16; ++r) {
          const int64_t m = wr0 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3), n = wc0 + j * 32 + (lane & 31);
          if (m >= p.M || n >= p.N) continue;
          if (SPLIT)
            p.ws[(int64_t)split * p.M * p.N + m * p.N + n] = a[r];
          else
            epilogue_store<bf16_t, EPI>(p, m, n, a[r]);
        }
      }
    return;
  }
  // after the transpose: row wr0 + i*32 + 8*q + 4*g + lane%4, columns wc0 + j*32 + (lane & 28) + 0..3
  const int64_t rl = wr0 + 4 * g + (lane & 3);
  const int64_t cl = wc0 + (lane & 28);
  if (SPLIT) {
    float* ws = p.ws + (int64_t)split * p.M * p.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          quad_transpose(v, lane);
          const floatx4_t o = {v[0], v[1], v[2], v[3]};
          *reinterpret_cast<floatx4_t*>(ws + (rl + i * 32 + 8 * q) * p.N + cl + j * 32) = o;
        }
    return;
  }
  constexpr bool kReadAux = epi_reads_aux<EPI>(), kWriteAux = epi_writes_aux<EPI>();
  const bool has_c = p.beta != 0.f;
  if constexpr (kReadAux) {
    if (!has_c) {
      // aux-reading epilogue without C (the fc2 dgrad times gelu'): the whole sub-tile's aux
      // reads go out before the first is used (the main loop's registers are free by now)
      u16x4_t av[FM][4][FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            av[i][q][j] = *reinterpret_cast<const u16x4_t*>(p.aux + (rl + i * 32 + 8 * q) * p.ldaux + cl + j * 32);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t m = rl + i * 32 + 8 * q;
          bf16_t* drow = d_row(p, m);
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            quad_transpose(v, lane);
            u16x4_t o;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float a = bf16_to_f32(av[i][q][j][t]);
              o[t] = f32_to_bf16(p.alpha * v[t] * (EPI == RH_EPI_GELU_GRAD ? gelu_grad_fast_f(a) : a));
            }
            *reinterpret_cast<u16x4_t*>(drow + cl + j * 32) = o;
          }
        }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    // this row block's C and aux reads go out together, before any of them is used
    u16x4_t cv[4][FN], av[4][FN];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = rl + i * 32 + 8 * q;
      if (has_c) {
        const bf16_t* crow = p.C ? p.C + m * p.ldc : d_row(p, m);
#pragma unroll
        for (int j = 0; j < FN; ++j) cv[q][j] = *reinterpret_cast<const u16x4_t*>(crow + cl + j * 32);
      }
      if (kReadAux) {
#pragma unroll
        for (int j = 0; j < FN; ++j) av[q][j] = *reinterpret_cast<const u16x4_t*>(p.aux + m * p.ldaux + cl + j * 32);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = rl + i * 32 + 8 * q;
      bf16_t* drow = d_row(p, m);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        quad_transpose(v, lane);
        const int64_t n = cl + j * 32;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = has_c ? p.alpha * v[t] + p.beta * bf16_to_f32(cv[q][j][t]) : p.alpha * v[t];
        if (kWriteAux) {
          u16x4_t x;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const GeluParts gp = gelu_parts_fast(v[t]);
            x[t] = f32_to_bf16(EPI == RH_EPI_GELU ? v[t] : gp.cdf + v[t] * gp.pdf);
            v[t] *= gp.cdf;
          }
          *reinterpret_cast<u16x4_t*>(p.aux_out + m * p.ldaux + n) = x;
        } else if (kReadAux) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float a = bf16_to_f32(av[q][j][t]);
            v[t] *= EPI == RH_EPI_GELU_GRAD ? gelu_grad_fast_f(a) : a;
          }
        }
        u16x4_t o;
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = f32_to_bf16(v[t]);
        *reinterpret_cast<u16x4_t*>(drow + n) = o;
      }
    }
  }
}

// LM-head forward without logits: each wave reduces its WTM x 64 sub-tile of logits to one
// (max, sum of 2^(v log2 e - max)) pair per row in base-2 units, stored at
// part[m * ld_part + 2 * block] for the row's global 64-column block; the lane holding the row's
// target column stores that logit (natural units) to tgt[m].  Columns past N take no part.
template <int BM, int BN, int WGM, int WGN, int FM, int FN>
__device__ __forceinline__ void epilogue_lse(const GemmParams<bf16_t>& p, floatx16_t (&acc)[FM][FN], int64_t m0,
                                             int64_t n0, int wm, int wn, int lane) {
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static_assert(WTN == 64, "the row partials cover 64-column blocks: one per wave");
  constexpr float kL2e = 1.4426950408889634074f;
  const int64_t wr0 = m0 + (int64_t)wm * WTM, wc0 = n0 + (int64_t)wn * WTN;
  const int g = lane >> 5;
  const int64_t rl = wr0 + 4 * g + (lane & 3);
  const int64_t cl = wc0 + (lane & 28);
  const int64_t blk = (p.col_off + wc0) / 64;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = rl + i * 32 + 8 * q;
      float v[FN][4];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float t4[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        quad_transpose(t4, lane);
#pragma unroll
        for (int t = 0; t < 4; ++t) v[j][t] = p.alpha * t4[t];
      }
      // next-token id read unconditionally at a clamped (valid) index, then selected
      const bool scored = m < p.M && m % p.seq != p.seq - 1;
      const int64_t tn = p.tokens[min(m + 1, p.M - 1)];
      const int64_t tc = scored ? tn - p.col_off : -1;
      // Element loops without branches (columns past N are selected away; a per-element branch
      // around each exponential costs exec-mask bookkeeping on every row): the lane holding the
      // target column picks its logit by selects and stores it once.
      float mx = -INFINITY, tv = 0.f;
      bool has_t = false;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t n = cl + j * 32 + t;
          mx = fmaxf(mx, n < p.N ? v[j][t] * kL2e : -INFINITY);
          tv = n == tc ? v[j][t] : tv;
          has_t = has_t || n == tc;
        }
      if (has_t) p.tgt[m] = tv;
      mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      // (a row with every column past N has mx = -inf: each term is then 2^inf, all selected away)
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e = __builtin_amdgcn_exp2f(fmaf(v[j][t], kL2e, -mx));
          sum += cl + j * 32 + t < p.N ? e : 0.f;
        }
      sum += __shfl_xor(sum, 4, 64);
      sum += __shfl_xor(sum, 8, 64);
      sum += __shfl_xor(sum, 16, 64);
      if ((lane & 28) == 0 && m < p.M && wc0 < p.N) {
        p.part[m * p.ld_part + 2 * blk] = mx;
        p.part[m * p.ld_part + 2 * blk + 1] = sum;
      }
    }
}

// LM-head backward, one vocabulary chunk: the recomputed logits v of row m become
//   dS = (exp(v - lse[m]) - [col_off + n == target]) * grad * inv_n
// (0 on the unscored last position of every sequence), stored in bf16 for columns n < N and
// as zeros for N <= n < n_store (the padding the weight-gradient GEMM reads).
template <int BM, int BN, int WGM, int WGN, int FM, int FN>
__device__ __forceinline__ void epilogue_xent_grad(const GemmParams<bf16_t>& p, floatx16_t (&acc)[FM][FN], int64_t m0,
                                                   int64_t n0, int wm, int wn, int lane) {
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr float kL2e = 1.4426950408889634074f;
  const int64_t wr0 = m0 + (int64_t)wm * WTM, wc0 = n0 + (int64_t)wn * WTN;
  const int g = lane >> 5;
  const int64_t rl = wr0 + 4 * g + (lane & 3);
  const int64_t cl = wc0 + (lane & 28);
  const float scale = p.inv_n * *p.grad;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = rl + i * 32 + 8 * q;
      const bool scored = m < p.M && m % p.seq != p.seq - 1;
      // per-row values read unconditionally at clamped (valid) indices, then selected
      const int64_t mc = min(m, p.M - 1);
      const int64_t tn = p.tokens[min(m + 1, p.M - 1)];
      const float lr = p.lse[mc];
      const int64_t tc = scored ? tn - p.col_off : -1;
      const float l2 = scored ? lr * kL2e : 0.f;
      bf16_t* drow = m < p.M ? d_row(p, m) : nullptr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float t4[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        quad_transpose(t4, lane);
        const int64_t n = cl + j * 32;
        if (drow == nullptr || n >= p.n_store) continue;
        u16x4_t o;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          // computed for every element and selected (no branch per element; an unscored row's
          // exponential may overflow, and the select drops it)
          const float e = __builtin_amdgcn_exp2f(fmaf(p.alpha * t4[t], kL2e, -l2));
          const float d = (e - (n + t == tc ? 1.f : 0.f)) * scale;
          o[t] = f32_to_bf16(scored && n + t < p.N ? d : 0.f);
        }
        *reinterpret_cast<u16x4_t*>(drow + n) = o;
      }
    }
}

// Epilogue through LDS: the fp32 tile is written to LDS in row chunks, then every thread takes
// 8 consecutive columns at a time -- one rolled loop, 16-byte coalesced loads and stores.
// 32x32 accumulator: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
// `smem_elems` bf16 elements of LDS are free for it (the caller's stages, after a barrier).
template <int BM, int BN, int WGM, int WGN, int EPI, bool SPLIT, int SMEM_ELEMS, int FM, int FN>
__device__ __forceinline__ void epilogue_tile_impl(const GemmParams<bf16_t>& p, bf16_t* smem, floatx16_t (&acc)[FM][FN],
                                                   int64_t m0, int64_t n0, int wm, int wn, int lane, int split) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int CP = BN >= 256 ? BN : BN + 4;                 // fp32 row pitch in LDS
  constexpr int CH_MAX = (SMEM_ELEMS * (int)sizeof(bf16_t)) / (CP * 4);
  constexpr int CH = CH_MAX >= BM ? BM : (CH_MAX >= WTM ? (CH_MAX / WTM) * WTM : WTM);
  static_assert(CH * CP * 4 <= SMEM_ELEMS * (int)sizeof(bf16_t), "epilogue chunk must fit the LDS stages");
  float* cs = reinterpret_cast<float*>(smem);
  const int g = lane >> 5, c32 = lane & 31;
  for (int r0 = 0; r0 < BM; r0 += CH) {
    // waves whose rows fall in [r0, r0 + CH) deposit their accumulators
    if (wm * WTM >= r0 && wm * WTM < r0 + CH) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * WTM - r0 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            cs[row * CP + wn * WTN + j * 32 + c32] = acc[i][j][r];
          }
    }
    __syncthreads();
#pragma unroll 1
    for (int e = threadIdx.x; e < CH * (BN / 8); e += NT) {
      const int row = e / (BN / 8), col = (e % (BN / 8)) * 8;
      const int64_t m = m0 + r0 + row, n = n0 + col;
      if (m >= p.M || n >= p.N) continue;
      const floatx4_t lo = *reinterpret_cast<const floatx4_t*>(cs + row * CP + col);
      const floatx4_t hi = *reinterpret_cast<const floatx4_t*>(cs + row * CP + col + 4);
      float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      if (SPLIT) {
        float* w = p.ws + (int64_t)split * p.M * p.N + m * p.N + n;
        if (n + 8 <= p.N && p.N % 4 == 0) {
          *reinterpret_cast<floatx4_t*>(w) = lo;
          *reinterpret_cast<floatx4_t*>(w + 4) = hi;
        } else {
          for (int t = 0; t < 8 && n + t < p.N; ++t) w[t] = v[t];
        }
        continue;
      }
      bf16_t* dp = d_row(p, m) + n;
      const bf16_t* cp = p.C ? p.C + m * p.ldc + n : dp;
      const bf16_t* xp = epi_writes_aux<EPI>() ? p.aux_out + m * p.ldaux + n
                                                : (epi_reads_aux<EPI>() ? p.aux + m * p.ldaux + n : dp);
      const bool vec = n + 8 <= p.N && (((uintptr_t)dp | (uintptr_t)xp) & 15) == 0 &&
                       (p.beta == 0.f || ((uintptr_t)cp & 15) == 0);
      if (vec) {
        if (p.beta != 0.f) {
          const u16x8_t c = *reinterpret_cast<const u16x8_t*>(cp);
#pragma unroll
          for (int t = 0; t < 8; ++t) v[t] = p.alpha * v[t] + p.beta * bf16_to_f32(c[t]);
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) v[t] *= p.alpha;
        }
        epi8_bf16<EPI>(v, const_cast<bf16_t*>(xp));
        u16x8_t o;
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] = f32_to_bf16(v[t]);
        *reinterpret_cast<u16x8_t*>(dp) = o;
      } else {
        for (int t = 0; t < 8 && n + t < p.N; ++t) epilogue_store<bf16_t, EPI>(p, m, n + t, v[t]);
      }
    }
    __syncthreads();
  }
}

// Epilogue choice, measured per kernel inside the block's fwd+bwd step on MI355X: the LDS-staged
// epilogue is faster for unsplit bf16 results without an aux read (its stores are whole 512-byte
// row runs), the register epilogue for split-K partials and for the aux-reading forms.
template <int BM, int BN, int WGM, int WGN, int EPI, bool SPLIT, int SMEM_ELEMS, int FM, int FN>
__device__ __forceinline__ void epilogue_sel(const GemmParams<bf16_t>& p, bf16_t* smem, floatx16_t (&acc)[FM][FN],
                                             int64_t m0, int64_t n0, int wm, int wn, int lane, int split) {
  if constexpr (EPI == kEpiLsePartial) {
    epilogue_lse<BM, BN, WGM, WGN>(p, acc, m0, n0, wm, wn, lane);
    return;
  } else if constexpr (EPI == kEpiXentGrad) {
    epilogue_xent_grad<BM, BN, WGM, WGN>(p, acc, m0, n0, wm, wn, lane);
    return;
  }
  if constexpr (!SPLIT && !epi_reads_aux<EPI>()) {
    if (p.epi_lds) {
      __syncthreads();  // every wave is done reading the operand stages
      epilogue_tile_impl<BM, BN, WGM, WGN, EPI, SPLIT, SMEM_ELEMS>(p, smem, acc, m0, n0, wm, wn, lane, split);
      return;
    }
  }
  epilogue_regs<BM, BN, WGM, WGN, EPI, SPLIT>(p, acc, m0, n0, wm, wn, lane, split);
}

template <int BM, int BN, int WGM, int WGN, int L, int EPI, bool SPLIT>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bf16_mfma(GemmParams<bf16_t> p) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr bool A_KC = (L != RH_GEMM_TN);
  constexpr bool B_KC = (L == RH_GEMM_NT);
  constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 32, FN = WTN / 32;
  constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK, STAGE = A_ELEMS + B_ELEMS;

  // two stages, each [A tile | B tile]
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * STAGE];

  int tm, tn;
  tile_coords(p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t kbeg = (int64_t)blockIdx.z * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nk = (int)((kend - kbeg + kBK - 1) / kBK);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const bool aligned = p.aligned != 0;
  // interior: no bounds checks, 16-byte loads, and (for a segmented m/n-contiguous B) every
  // k-tile inside one segment
  const bool interior = aligned && m0 + BM <= p.M && n0 + BN <= p.N && (kend - kbeg) % kBK == 0 &&
                        (B_KC || p.b_nseg == 1 || p.b_seg % kBK == 0);

  floatx16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (interior) {
    FastIO<BM, A_KC, NT> fa;
    FastIO<BN, B_KC, NT> fb;
    fa.setup([&](int64_t r) { return p.A + r * p.lda; }, m0, kbeg, p.lda);
    fb.setup([&](int64_t r) { return b_row(p, r); }, n0, kbeg, p.ldb);
    // row-k base pointers of the m/n-contiguous operands (one scalar lookup per k-tile)
    auto a_base = [&](int kt) -> const bf16_t* { return A_KC ? nullptr : p.A + (kbeg + (int64_t)kt * kBK) * p.lda; };
    auto b_base = [&](int kt) -> const bf16_t* { return B_KC ? nullptr : b_row(p, kbeg + (int64_t)kt * kBK); };
    if (nk > 0) {
      fa.load(0, a_base(0));
      fb.load(0, b_base(0));
      fa.store(smem);
      fb.store(smem + A_ELEMS);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = (kt + 1) < nk;
      if (more) {
        fa.load(kt + 1, a_base(kt + 1));
        fb.load(kt + 1, b_base(kt + 1));
      }
      const bf16_t* a_s = smem + cur * STAGE;
      mma_ktile<BM, BN, WGM, WGN, A_KC, B_KC, FM, FN>(a_s, a_s + A_ELEMS, acc, wm, wn, lane);
      if (more) {
        bf16_t* nxt = smem + (cur ^ 1) * STAGE;
        fa.store(nxt);
        fb.store(nxt + A_ELEMS);
      }
      __syncthreads();
    }
  } else {
    auto a_row = [&](int64_t r) -> const bf16_t* { return p.A + r * p.lda; };
    auto bb_row = [&](int64_t r) -> const bf16_t* { return b_row(p, r); };
    TileIO<BM, A_KC, NT> ta;
    TileIO<BN, B_KC, NT> tb;
    if (nk > 0) {
      ta.load(a_row, m0, kbeg, p.M, kend, false, aligned);
      tb.load(bb_row, n0, kbeg, p.N, kend, false, aligned);
      ta.store(smem);
      tb.store(smem + A_ELEMS);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = (kt + 1) < nk;
      if (more) {
        const int64_t k0 = kbeg + (int64_t)(kt + 1) * kBK;
        ta.load(a_row, m0, k0, p.M, kend, false, aligned);
        tb.load(bb_row, n0, k0, p.N, kend, false, aligned);
      }
      const bf16_t* a_s = smem + cur * STAGE;
      mma_ktile<BM, BN, WGM, WGN, A_KC, B_KC, FM, FN>(a_s, a_s + A_ELEMS, acc, wm, wn, lane);
      if (more) {
        bf16_t* nxt = smem + (cur ^ 1) * STAGE;
        ta.store(nxt);
        tb.store(nxt + A_ELEMS);
      }
      __syncthreads();
    }
  }

  epilogue_sel<BM, BN, WGM, WGN, EPI, SPLIT, 2 * STAGE>(p, smem, acc, m0, n0, wm, wn, lane, (int)blockIdx.z);
}


// ---------------------------------------------------------------------------
// bf16 MFMA kernel fed by direct global->LDS loads
// ---------------------------------------------------------------------------
// The operand tiles go global->LDS with global_load_lds_dwordx4 (no staging registers, no LDS
// write instructions).  k-tiles are 64 deep so that every k-contiguous row piece a load fetches
// is a whole 128-byte cache line (measured on MI355X: the L2->CU path delivers ~1.5-2x more
// bytes per clock for whole lines than for 64-byte halves).  Two stages (128 KB at 256x256):
// tile t+1 is loaded while tile t is computed; each k-step's fragments are read during the
// previous k-step's MFMAs.  LDS layouts are the register-staged kernel's (kc_off / mc_off).
// Needs: 16-byte aligned rows, K and the K per split multiples of 64, m/n-contiguous operand
// extents multiples of 8, B segment boundaries multiples of 64 k-rows.  Rows / columns past
// the matrix edge are clamped onto the last valid ones (their results are never stored).
template <int ROWS, bool KC, int NWAVES>
struct DmaOperand {
  static constexpr int WIN = ROWS * kBK * 2 / 1024;
  static constexpr int PER = WIN / NWAVES;
  static_assert(WIN % NWAVES == 0, "tile windows must split evenly over the waves");
  static constexpr int KROWS = 512 / ROWS;  // !KC: k-rows per window
  const bf16_t* rowp[PER];
  int64_t off[PER];

  template <typename RowFn>
  __device__ __forceinline__ void setup(RowFn rowptr, int64_t o0, int64_t extent, int64_t kbeg, int64_t ld, int wave,
                                        int lane) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int win = wave + NWAVES * i;
      if (KC) {
        const int row = win * 8 + lane / 8;
        const int lchunk = (lane & 7) ^ ((row >> 1) & 7);  // inverse of kc_off's chunk swizzle
        const int64_t gr = min(o0 + row, extent - 1);
        rowp[i] = rowptr(gr) + kbeg + lchunk * 8;
      } else {
        const int kr = win * KROWS + lane / (ROWS / 8);
        const int pchunk = lane % (ROWS / 8);
        const int lunit = (pchunk >> 2) ^ (kr & 3);  // inverse of mc_off's unit swizzle
        const int64_t c = o0 + lunit * 32 + (pchunk & 3) * 8;
        off[i] = (int64_t)kr * ld + min(c, extent - 8);
      }
    }
  }
  // dst: the tile as a 32-bit LDS byte address (wave-uniform, scalar math)
  __device__ __forceinline__ void issue(uint32_t dst, int kt, const bf16_t* krow0, int wave) {
#pragma unroll
    for (int i = 0; i < PER; ++i) issue_one(i, dst, kt, krow0, wave);
  }
  __device__ __forceinline__ void issue_one(int i, uint32_t dst, int kt, const bf16_t* krow0, int wave) {
    const int win = wave + NWAVES * i;
    dma16(KC ? rowp[i] + (int64_t)kt * kBK : krow0 + off[i], dst + (uint32_t)win * 1024u);
  }
};

// DmaOperand with 32-bit per-lane byte offsets from a wave-uniform base (the saddr form of the
// load): half the VGPRs of 64-bit pointers.  KC: the base is the operand's first row at the
// k-tile (one allocation: rows r < extent at base + r*ld); !KC: the k-tile's first row.  The host
// keeps the offsets below 2^32 bytes (w4_addressable).
template <int ROWS, bool KC, int NWAVES>
struct DmaOperand32 {
  static constexpr int WIN = ROWS * kBK * 2 / 1024;
  static constexpr int PER = WIN / NWAVES;
  static_assert(WIN % NWAVES == 0, "tile windows must split evenly over the waves");
  static constexpr int KROWS = 512 / ROWS;  // !KC: k-rows per window
  uint32_t voff[PER];

  __device__ __forceinline__ void setup(int64_t o0, int64_t extent, int64_t kbeg, int64_t ld, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int win = wave + NWAVES * i;
      if (KC) {
        const int row = win * 8 + lane / 8;
        const int lchunk = (lane & 7) ^ ((row >> 1) & 7);  // inverse of kc_off's chunk swizzle
        const int64_t gr = min(o0 + row, extent - 1);
        voff[i] = (uint32_t)((gr * ld + kbeg + lchunk * 8) * 2);
      } else {
        const int kr = win * KROWS + lane / (ROWS / 8);
        const int pchunk = lane % (ROWS / 8);
        const int lunit = (pchunk >> 2) ^ (kr & 3);  // inverse of mc_off's unit swizzle
        const int64_t c = o0 + lunit * 32 + (pchunk & 3) * 8;
        voff[i] = (uint32_t)(((int64_t)kr * ld + min(c, extent - 8)) * 2);
      }
    }
  }
  // window i of the k-tile whose base is `base` (KC: operand base + kt*64; !KC: the k-tile's first row)
  __device__ __forceinline__ void issue_one(int i, uint32_t dst, const bf16_t* base, int wave) {
    const int win = wave + NWAVES * i;
    dma16s(base, voff[i], dst + (uint32_t)win * 1024u);
  }
};

// 256x256 tile on 4 waves (2 x 2, 128x128 per wave): a third fewer LDS fragment reads per MFMA
// than 8 waves of 128x64, and one wave per SIMD, so no two waves contend for one MFMA pipe.  The
// 256 accumulators per lane live in AGPRs (mfma_agpr).  One wave per SIMD cannot hide a stall
// behind another wave, so the k-tile is software-pipelined by hand; volatile asm statements keep
// their order and the LDS reads / DMA issues written between them stay where they are written:
//   k-steps 0..2: 16 MFMAs each, the next k-step's 8 fragments read one after each of the first
//     8 MFMAs (16 for transposing reads);
//   then wait for this wave's loads of tile kt+1 and the barrier (tile kt+1 visible everywhere,
//     every wave's reads of tile kt done: __syncthreads waits for them);
//   k-step 3: 16 MFMAs on fragments already in registers, with tile kt+1's k-step-0 fragments
//     read and tile kt+2's 16 DMA windows issued (into tile kt's stage) between them.
// So the only pipe bubble per k-tile is the barrier itself, which the waves reach together.
template <int BM, int BN, int L, int EPI, bool SPLIT>
__device__ __forceinline__ void gemm_dma_tile_w4(const GemmParams<bf16_t>& p, bf16_t* smem, int tm, int tn, int split) {
  constexpr int WGM = 2, WGN = 2, NW = 4;
  constexpr bool A_KC = (L != RH_GEMM_TN);
  constexpr bool B_KC = (L == RH_GEMM_NT);
  constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 32, FN = WTN / 32;
  constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK, STAGE = A_ELEMS + B_ELEMS;
  using DA = DmaOperand32<BM, A_KC, NW>;  // A: one allocation
  using DB = DmaOperand<BN, B_KC, NW>;    // B: k-contiguous rows may come from several segments
  using DB32 = DmaOperand32<BN, B_KC, NW>;
  static_assert(FM == 4 && FN == 4 && DA::PER + DB::PER == 16, "4-wave 256x256 tile");

  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nk = (int)((kend - kbeg) / kBK);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  DA da;
  std::conditional_t<B_KC, DB, DB32> db;
  da.setup(m0, p.M, kbeg, p.lda, wave, lane);
  if constexpr (B_KC) db.setup([&](int64_t r) { return b_row(p, r); }, n0, p.N, kbeg, p.ldb, wave, lane);
  else db.setup(n0, p.N, kbeg, p.ldb, wave, lane);
  const bf16_t* const bs0 = p.B[0];
  const bf16_t* const bs1 = p.B[1 % RH_MAX_SEG];
  const bf16_t* const bs2 = p.B[2 % RH_MAX_SEG];
  const bf16_t* const bs3 = p.B[3 % RH_MAX_SEG];
  const int bseg_rows = (!B_KC && p.b_nseg > 1) ? (int)p.b_seg : INT32_MAX;
  int iss_seg = 0, iss_row = (int)kbeg;
  if (!B_KC && p.b_nseg > 1) {
    iss_seg = (int)kbeg / bseg_rows;
    iss_row = (int)kbeg - iss_seg * bseg_rows;
  }
  // first k-row of the next m/n-contiguous B k-tile to issue (tiles are issued in order)
  auto next_b = [&]() -> const bf16_t* {
    if (B_KC) return nullptr;
    const bf16_t* base = iss_seg == 0 ? bs0 : iss_seg == 1 ? bs1 : iss_seg == 2 ? bs2 : bs3;
    const bf16_t* r = base + (int64_t)iss_row * p.ldb;
    iss_row += kBK;
    if (iss_row >= bseg_rows) {
      iss_row -= bseg_rows;
      ++iss_seg;
    }
    return r;
  };
  // A's base for k-tile kt (DmaOperand32: the offsets hold the rows and kbeg)
  auto a_krow = [&](int kt) -> const bf16_t* {
    return A_KC ? p.A + (int64_t)kt * kBK : p.A + (kbeg + (int64_t)kt * kBK) * p.lda;
  };
  auto b_issue = [&](int i, uint32_t dst, int kt, const bf16_t* bk) {
    if constexpr (B_KC) db.issue_one(i, dst, kt, nullptr, wave);
    else db.issue_one(i, dst, bk, wave);
  };
  // LDS: A in three stages (tile t in stage t % 3), B in two (t % 2), 160 KB in all.  The A stage
  // of tile kt+2 is free from tile kt-1's barrier on, so its loads spread over k-steps 0..2 of
  // tile kt; only B's wait for tile kt's own barrier.  (The DMA path moves about 64 B per clock
  // per CU, so a whole k-tile's 64 windows per CU take about half of the k-tile's MFMA time.)
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;  // a generic LDS pointer's low 32 bits
  constexpr uint32_t kABytes = A_ELEMS * 2, kBBytes = B_ELEMS * 2;
  auto a_lds = [&](int stage) { return lds0 + (uint32_t)stage * kABytes; };
  auto b_lds = [&](int stage) { return lds0 + 3u * kABytes + (uint32_t)stage * kBBytes; };
  auto a_ptr = [&](int stage) -> const bf16_t* { return smem + stage * A_ELEMS; };
  auto b_ptr = [&](int stage) -> const bf16_t* { return smem + 3 * A_ELEMS + stage * B_ELEMS; };
  auto issue_all = [&](int kt) {
    const bf16_t* ak = a_krow(kt);
    const bf16_t* bk = next_b();
#pragma unroll
    for (int i = 0; i < DA::PER; ++i) da.issue_one(i, a_lds(kt % 3), ak, wave);
#pragma unroll
    for (int i = 0; i < DB::PER; ++i) b_issue(i, b_lds(kt & 1), kt, bk);
  };

  floatx16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  mfma_asm_begin(acc);

  bf16x8_t fa[2][FM], fb[2][FN];
  auto frag = [&](int set, const bf16_t* sa, const bf16_t* sb, int ks, int f) {
    if (f < FM) fa[set][f] = load_frag<BM, A_KC>(sa, wm * WTM + f * 32, ks, lane);
    else fb[set][f - FM] = load_frag<BN, B_KC>(sb, wn * WTN + (f - FM) * 32, ks, lane);
  };

  if (nk > 0) {
    issue_all(0);
    if (nk > 1) {
      issue_all(1);
      wait_vm_le<DA::PER + DB::PER>();  // tile 0 has landed, tile 1 may be in flight
    } else {
      wait_vm_le<0>();
    }
    __syncthreads();
#pragma unroll
    for (int f = 0; f < FM + FN; ++f) frag(0, a_ptr(0), b_ptr(0), 0, f);
  }
  // Fragment reads, one every other MFMA, in the order the next k-step's MFMAs (row-major over
  // the 4 x 4 accumulator blocks) first need them: A0, B0..B3, A1, A2, A3.
  auto frag_order = [](int slot) { return slot == 0 ? 0 : slot < 5 ? FM + slot - 1 : slot - 4; };
  // one k-tile; MORE: a next tile exists (read its first fragments), REFILL: tile kt+2 exists.
  // sa3 = kt % 3 is carried by the caller (no division in the loop).
  static_assert(DA::PER == 8 && DB::PER == 8, "eight windows per wave and operand");
  auto ktile = [&](int kt, int sa3, auto more_c, auto refill_c) {
    constexpr bool MORE = decltype(more_c)::value, REFILL = decltype(refill_c)::value;
    const int na3 = sa3 == 2 ? 0 : sa3 + 1, fa3 = na3 == 2 ? 0 : na3 + 1;  // stages of kt+1, kt+2
    const bf16_t* sa = a_ptr(sa3);
    const bf16_t* sb = b_ptr(kt & 1);
    const bf16_t* ak = nullptr;
    if constexpr (REFILL) ak = a_krow(kt + 2);
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        mfma_agpr(acc[t / FN][t % FN], fa[ks & 1][t / FN], fb[ks & 1][t % FN]);
        if (t % 2 == 0) frag((ks + 1) & 1, sa, sb, ks + 1, frag_order(t / 2));
        if constexpr (REFILL) {
          const int g = ks * 16 + t;  // A windows of tile kt+2 at MFMA slots 3, 9, ..., 45
          if (g % 6 == 3) da.issue_one(g / 6, a_lds(fa3), ak, wave);
        }
      }
    }
    // this wave's loads of tile kt+1 have landed (the 8 A windows of tile kt+2 may be in flight)
    if constexpr (REFILL) wait_vm_le<DA::PER>();
    else wait_vm_le<0>();
    __syncthreads();
    const bf16_t* bk = nullptr;
    if constexpr (REFILL) bk = next_b();
#pragma unroll
    for (int t = 0; t < FM * FN; ++t) {
      mfma_agpr(acc[t / FN][t % FN], fa[1][t / FN], fb[1][t % FN]);
      if constexpr (MORE) {
        if (t % 2 == 0) frag(0, a_ptr(na3), b_ptr((kt + 1) & 1), 0, frag_order(t / 2));
      }
      if constexpr (REFILL) {
        if (t % 2 == 1) b_issue(t / 2, b_lds(kt & 1), kt + 2, bk);  // between the reads
      }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  int kt = 0, s3 = 0;
#pragma unroll 1
  for (; kt + 2 < nk; ++kt) {
    ktile(kt, s3, T_{}, T_{});
    s3 = s3 == 2 ? 0 : s3 + 1;
  }
  if (kt + 1 < nk) {
    ktile(kt++, s3, T_{}, F_{});
    s3 = s3 == 2 ? 0 : s3 + 1;
  }
  if (kt < nk) ktile(kt, s3, F_{}, F_{});
  mfma_asm_drain(acc);
  // the register epilogue: staging the tile through LDS makes the allocator spill accumulators
  epilogue_regs<BM, BN, WGM, WGN, EPI, SPLIT>(p, acc, m0, n0, wm, wn, lane, split);
}

// One output tile (tm, tn) of split `split` of a direct-to-LDS GEMM, on the workgroup's LDS `smem`
// (two stages of BM x 64 + BN x 64 bf16).
template <int BM, int BN, int WGM, int WGN, int L, int EPI, bool SPLIT>
__device__ __forceinline__ void gemm_dma_tile(const GemmParams<bf16_t>& p, bf16_t* smem, int tm, int tn, int split) {
  if constexpr (WGM * WGN == 4 && BM == 256 && BN == 256) {
    gemm_dma_tile_w4<BM, BN, L, EPI, SPLIT>(p, smem, tm, tn, split);
    return;
  }
  constexpr int NW = WGM * WGN;
  constexpr bool A_KC = (L != RH_GEMM_TN);
  constexpr bool B_KC = (L == RH_GEMM_NT);
  constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 32, FN = WTN / 32;
  constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK, STAGE = A_ELEMS + B_ELEMS;
  using DA = DmaOperand<BM, A_KC, NW>;
  using DB = DmaOperand<BN, B_KC, NW>;

  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nk = (int)((kend - kbeg) / kBK);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  DA da;
  DB db;
  da.setup([&](int64_t r) { return p.A + r * p.lda; }, m0, p.M, kbeg, p.lda, wave, lane);
  db.setup([&](int64_t r) { return b_row(p, r); }, n0, p.N, kbeg, p.ldb, wave, lane);
  const bf16_t* const bs0 = p.B[0];
  const bf16_t* const bs1 = p.B[1 % RH_MAX_SEG];
  const bf16_t* const bs2 = p.B[2 % RH_MAX_SEG];
  const bf16_t* const bs3 = p.B[3 % RH_MAX_SEG];
  const int bseg_rows = (!B_KC && p.b_nseg > 1) ? (int)p.b_seg : INT32_MAX;
  int iss_seg = 0, iss_row = (int)kbeg;
  if (!B_KC && p.b_nseg > 1) {
    iss_seg = (int)kbeg / bseg_rows;
    iss_row = (int)kbeg - iss_seg * bseg_rows;
  }
  // stages addressed as LDS byte offsets from one base converted once (a generic-to-LDS pointer
  // conversion per load costs a null check in scalar instructions)
  const uint32_t sbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem;
  auto issue = [&](int kt) {
    const uint32_t st = sbase + (uint32_t)((kt & 1) * STAGE * 2);
    const int64_t k0 = kbeg + (int64_t)kt * kBK;
    da.issue(st, kt, A_KC ? nullptr : p.A + k0 * p.lda, wave);
    if (B_KC) {
      db.issue(st + A_ELEMS * 2, kt, nullptr, wave);
    } else {
      const bf16_t* base = iss_seg == 0 ? bs0 : iss_seg == 1 ? bs1 : iss_seg == 2 ? bs2 : bs3;
      db.issue(st + A_ELEMS * 2, kt, base + (int64_t)iss_row * p.ldb, wave);
      iss_row += kBK;
      if (iss_row >= bseg_rows) {
        iss_row -= bseg_rows;
        ++iss_seg;
      }
    }
  };

  floatx16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  bf16x8_t fa[2][FM], fb[2][FN];
  auto read_frags = [&](int set, const bf16_t* st, int ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[set][i] = load_frag<BM, A_KC>(st, wm * WTM + i * 32, ks, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[set][j] = load_frag<BN, B_KC>(st + A_ELEMS, wn * WTN + j * 32, ks, lane);
  };
  constexpr int NREAD = FM * (A_KC ? 1 : 2) + FN * (B_KC ? 1 : 2);

  if (nk > 0) {
    issue(0);
    wait_vm_le<0>();
    __syncthreads();
  }
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) issue(kt + 1);
    const bf16_t* st = smem + (kt & 1) * STAGE;
    read_frags(0, st, 0);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      if (ks + 1 < kBK / 16) read_frags((ks + 1) & 1, st, ks + 1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks & 1][i], fb[ks & 1][j], acc[i][j], 0, 0, 0);
      if (ks + 1 < kBK / 16) {
        __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm_le<0>();  // tile kt+1 has landed
    __syncthreads();
  }

  epilogue_sel<BM, BN, WGM, WGN, EPI, SPLIT, 2 * STAGE>(p, smem, acc, m0, n0, wm, wn, lane, split);
}

// LDS of a direct-to-LDS tile: two stages of A and B; the 4-wave 256x256 tile keeps three of A
template <int BM, int BN, int WGM, int WGN>
constexpr int dma_smem_elems() {
  return (WGM * WGN == 4 && BM == 256 && BN == 256) ? (3 * BM + 2 * BN) * kBK : 2 * (BM + BN) * kBK;
}

template <int BM, int BN, int WGM, int WGN, int L, int EPI, bool SPLIT>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bf16_dma(GemmParams<bf16_t> p) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[dma_smem_elems<BM, BN, WGM, WGN>()];
  int tm, tn;
  tile_coords(p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  gemm_dma_tile<BM, BN, WGM, WGN, L, EPI, SPLIT>(p, smem, tm, tn, (int)blockIdx.z);
}

// ---------------------------------------------------------------------------
// Grouped launch: several GEMMs of one layout (the weight gradients of a decoder block, which
// share the token dimension as K) in ONE grid.  The workgroups are dealt over the problems in a
// logical order -- problem by problem, split-K slice by slice, tiles in GROUP_M order -- and each
// XCD takes one contiguous run of it, so the tiles sharing operand panels meet in one L2.
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 4;

struct GroupedParams {
  GemmParams<bf16_t> p[kMaxGroup];
  int first[kMaxGroup + 1];  // logical index of each problem's first workgroup (first[count] = total)
  int splits;
  int count;
};

// logical tile t of a tiles_m x tiles_n grid in GROUP_M order
__device__ __forceinline__ void group_order(int t, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int per_group = group_m * tiles_n;
  const int g = t / per_group;
  const int first_m = g * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in = t - g * per_group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

template <int BM, int BN, int WGM, int WGN, int L, bool SPLIT>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bf16_dma_grouped(GroupedParams gp) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[dma_smem_elems<BM, BN, WGM, WGN>()];
  const int nwg = gp.first[gp.count];
  const int bid = blockIdx.x;
  const int q = nwg / 8, r = nwg % 8;
  const int xcd = bid % 8, idx = bid / 8;
  const int logical = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + idx;
  int i = 0;
  while (i + 1 < gp.count && logical >= gp.first[i + 1]) ++i;
  const GemmParams<bf16_t>& p = gp.p[i];
  const int tiles = p.tiles_m * p.tiles_n;
  const int local = logical - gp.first[i];
  const int split = local / tiles;
  int tm, tn;
  group_order(local - split * tiles, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  gemm_dma_tile<BM, BN, WGM, WGN, L, RH_EPI_NONE, SPLIT>(p, smem, tm, tn, split);
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

// bf16, N % 8 == 0, 16-byte aligned rows: each thread reduces 8 consecutive outputs with
// 16-byte partial loads (the partials are read exactly once) and one 16-byte store.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_vec(GemmParams<bf16_t> p, int splits) {
  const int64_t total8 = p.M * p.N / 8;
  const int64_t n8 = p.N / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total8; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / n8, n = (i - m * n8) * 8;
    floatx4_t lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    for (int z = 0; z < splits; ++z) {
      const float* w = p.ws + (int64_t)z * p.M * p.N + m * p.N + n;
      lo += *reinterpret_cast<const floatx4_t*>(w);
      hi += *reinterpret_cast<const floatx4_t*>(w + 4);
    }
    float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    bf16_t* dp = d_row(p, m) + n;
    if (p.beta != 0.f) {
      const u16x8_t c = *reinterpret_cast<const u16x8_t*>(p.C ? p.C + m * p.ldc + n : dp);
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = p.alpha * v[t] + p.beta * bf16_to_f32(c[t]);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] *= p.alpha;
    }
    epi8_bf16<EPI>(v, epi_writes_aux<EPI>() ? p.aux_out + m * p.ldaux + n
                                            : const_cast<bf16_t*>(epi_reads_aux<EPI>() ? p.aux + m * p.ldaux + n : dp));
    u16x8_t o;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = f32_to_bf16(v[t]);
    *reinterpret_cast<u16x8_t*>(dp) = o;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
enum TileCfg { kT256x256 = 0, kT256x128 = 1, kT128x128 = 2, kT256x192 = 3, kTf32 = 4 };

struct TileShape {
  int bm, bn, threads;
};
constexpr TileShape kShapes[5] = {{256, 256, 512}, {256, 128, 512}, {128, 128, 256}, {256, 192, 512}, {fBM, fBN, 256}};
// waves (rows x columns) of each bf16 tile shape
constexpr int kWaves[5][2] = {{2, 4}, {4, 2}, {2, 2}, {4, 2}, {0, 0}};

struct Plan {
  int cfg;
  int splits;
  int64_t k_per_split;
  int64_t ws_bytes;
  int tiles_m, tiles_n;
  int64_t k_main = 0;  // K covered by the `splits` slices (a k-tile multiple when tail == 1)
  int tail = 0;        // 1: [k_main, K) is one more partial slice (register-staged kernel)
};

// Relative throughput of one CU on each tile shape (measured order of magnitude; bigger
// tiles re-read less of A and B per FLOP).  256x192 (NT only: both operands k-contiguous; the
// m/n-contiguous LDS swizzle needs power-of-two widths) exists for N = 1536-type outputs, where
// 256x256 tiles leave a quarter of the CUs idle.
constexpr double kTileEff[4] = {1.0, 0.85, 0.6, 0.95};

// Cost of one fp32 split-K partial element (written by the main kernel, re-read by the reduce) in
// the grouped planner's unit (one MAC of a tile's area over k).  Measured on MI355X with a decoder
// block's four weight gradients (K 8192, 192 tiles of 256x256) in one grouped launch: split 4 (3
// waves of 2048-deep tiles, 50 M partial elements) takes 270 us against 232 us unsplit (one wave of
// 8192); ~6 units per element reproduces both.
constexpr double kGroupSplitCost = 6.0;

inline Plan plan_gemm(const rh_gemm_desc* d) {
  Plan pl{kTf32, 1, 0, 0, 0, 0};
  if (d->dtype != RH_DTYPE_BF16) {
    pl.tiles_m = (int)rh_cdiv(d->M, fBM);
    pl.tiles_n = (int)rh_cdiv(d->N, fBN);
    pl.k_per_split = rh_cdiv(d->K, fBK) * fBK;
    pl.k_main = d->K;
    return pl;
  }
  const int64_t cus = rh_device_cus();
  // RESIHP_GEMM_TILE=0/1/2/3 pins the tile shape (256x256 / 256x128 / 128x128 / 256x192, the
  // last for NT only); tests use it to run every shape on every layout.
  int only = -1;
  if (const char* e = getenv("RESIHP_GEMM_TILE")) {
    if (e[0] >= '0' && e[0] <= '3' && e[1] == 0) only = e[0] - '0';
  }
  if (only == kT256x192 && d->layout != RH_GEMM_NT) only = -1;
  // Ragged K (e.g. the LM head's backward, K = vocab): the bulk, a multiple of the k-tile, runs
  // on the direct-to-LDS kernel and the last K % 64 as one extra fp32 partial slice on the
  // register-staged kernel; the ordered reduce adds every slice, so the result is rounded once.
  // (A k-row-segmented m/n-contiguous B keeps the one-kernel path.)
  const bool tail = d->K % kBK != 0 && d->K >= 8 * kBK && (d->layout == RH_GEMM_NT || d->b_nseg == 1);
  const int64_t Kp = tail ? d->K - d->K % kBK : d->K;
  // estimated time ~ (tiles resident per CU over the whole run) x tile area x k / efficiency;
  // split K when one wave of tiles leaves CUs idle
  double best = 1e300;
  for (int c = 0; c < 4; ++c) {
    if (only >= 0 && c != only) continue;
    const double eff = kTileEff[c];
    if (c == kT256x192 && d->layout != RH_GEMM_NT) continue;
    const int64_t tm = rh_cdiv(d->M, kShapes[c].bm), tn = rh_cdiv(d->N, kShapes[c].bn);
    const int64_t tiles = tm * tn;
    const int64_t per_cu = c == kT128x128 ? 2 : 1;  // co-resident workgroups (LDS-bound)
    const int64_t slots = cus * per_cu;
    for (int64_t splits = 1; splits <= 8; ++splits) {
      if (splits > 1 && (Kp / splits < 512 || tiles * (splits - 1) >= slots)) break;
      const int64_t kps = rh_cdiv(rh_cdiv(Kp, splits), kBK) * kBK;
      const int64_t waves = rh_cdiv(tiles * splits, slots);
      double t = (double)waves * per_cu * kShapes[c].bm * kShapes[c].bn * (double)kps / eff;
      // partial write + reduce: measured on MI355X, a split-4 2048x2048 reduce costs ~1/4 of a
      // 256x256x2048 tile wave, i.e. ~2 units per partial element (the fc2 forward of GPT-2-small,
      // M 8192 N 768 K 3072, is faster split in two than unsplit on 256x128 tiles)
      if (splits > 1) t += 2.0 * (double)splits * d->M * d->N;
      if (t < best * 0.98) {
        best = t;
        pl.cfg = c;
        pl.splits = (int)rh_cdiv(Kp, kps);
        pl.k_per_split = kps;
        pl.tiles_m = (int)tm;
        pl.tiles_n = (int)tn;
      }
    }
  }
  pl.k_main = Kp;
  pl.tail = tail ? 1 : 0;
  const int64_t slices = pl.splits + pl.tail;
  pl.ws_bytes = slices > 1 ? slices * d->M * d->N * (int64_t)sizeof(float) : 0;
  return pl;
}

inline int validate(const rh_gemm_desc* d) {
  RH_REQUIRE(d != nullptr, "rh_gemm: null descriptor");
  RH_REQUIRE(d->dtype == RH_DTYPE_F32 || d->dtype == RH_DTYPE_BF16, "rh_gemm: unknown dtype %d", d->dtype);
  RH_REQUIRE(d->layout >= RH_GEMM_NT && d->layout <= RH_GEMM_TN, "rh_gemm: unknown layout %d", d->layout);
  RH_REQUIRE(d->epilogue >= RH_EPI_NONE && d->epilogue <= RH_EPI_MUL_AUX, "rh_gemm: unknown epilogue %d",
             d->epilogue);
  RH_REQUIRE(d->M >= 0 && d->N >= 0 && d->K >= 0, "rh_gemm: negative extent M=%lld N=%lld K=%lld",
             (long long)d->M, (long long)d->N, (long long)d->K);
  RH_REQUIRE(d->M <= INT32_MAX / 2 && d->N <= INT32_MAX / 2, "rh_gemm: M or N too large");
  RH_REQUIRE(d->b_nseg >= 1 && d->b_nseg <= RH_MAX_SEG && d->d_nseg >= 1 && d->d_nseg <= RH_MAX_SEG,
             "rh_gemm: segment count out of range (b %d, d %d)", d->b_nseg, d->d_nseg);
  if (d->M == 0 || d->N == 0) return RH_OK;
  RH_REQUIRE(d->A || d->K == 0, "rh_gemm: null A");
  RH_REQUIRE(d->D[0], "rh_gemm: null D");
  const int64_t a_cols = d->layout == RH_GEMM_TN ? d->M : d->K;
  const int64_t b_rows = d->layout == RH_GEMM_NT ? d->N : d->K;
  const int64_t b_cols = d->layout == RH_GEMM_NT ? d->K : d->N;
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
    if (d->epilogue == RH_EPI_GELU || d->epilogue == RH_EPI_GELU_DERIV)
      RH_REQUIRE(d->aux_out, "rh_gemm: epilogue %d needs aux_out", d->epilogue);
    if (d->epilogue == RH_EPI_GELU_GRAD || d->epilogue == RH_EPI_MUL_AUX)
      RH_REQUIRE(d->aux, "rh_gemm: epilogue %d needs aux", d->epilogue);
  }
  return RH_OK;
}

// Which kernel runs a 256x256 direct-to-LDS tile: the 4-wave one (gemm_dma_tile_w4) for grouped
// launches and split-K slices (the weight gradients and the LM head's dgrad: long K, fp32 partials
// or no epilogue; the GPT-2-small head dgrad runs 0.64 ms instead of 0.87), the 8-wave one for unsplit
// single GEMMs, whose epilogues (GELU, residual) it finishes faster through LDS (measured inside the
// block's step).  RESIHP_GEMM_WAVES=4 or 8 pins one for all (tests run both).
inline bool four_wave_256(bool long_k) {
  const char* e = getenv("RESIHP_GEMM_WAVES");
  if (e && (e[0] == '4' || e[0] == '8') && e[1] == 0) return e[0] == '4';
  return long_k;
}

// The 4-wave kernel addresses A (and an m/n-contiguous B) with 32-bit byte offsets from a
// wave-uniform base (DmaOperand32): every offset it forms must stay below 2^32 bytes.
inline bool w4_addressable(const rh_gemm_desc* d) {
  constexpr int64_t kLim = (int64_t)1 << 31;  // elements
  const bool a_kc = d->layout != RH_GEMM_TN, b_kc = d->layout == RH_GEMM_NT;
  const int64_t a_span = a_kc ? d->M * d->lda + d->K : (int64_t)kBK * d->lda + d->M;
  const int64_t b_span = b_kc ? 0 : (int64_t)kBK * d->ldb + d->N;
  return a_span < kLim && b_span < kLim;
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
  const int64_t vec = 16 / (int64_t)sizeof(T);
  bool al = rh_aligned(d->A, 16) && d->lda % vec == 0 && d->ldb % vec == 0;
  for (int s = 0; s < d->b_nseg; ++s) al = al && rh_aligned(d->B[s], 16);
  // segment boundaries must not split a 16-byte chunk of the k-contiguous B or a k-tile row
  if (d->b_nseg > 1) al = al && d->b_seg_rows % 8 == 0;
  p.aligned = al ? 1 : 0;
  // the register epilogue's vector path: 4-element bf16 groups of D / C / aux rows, 4-element
  // fp32 groups of the [splits][M][N] partials
  bool ov = d->ldd % 4 == 0 && (pl.splits + pl.tail == 1 || (d->N % 4 == 0 && rh_aligned(ws, 16)));
  for (int s = 0; s < d->d_nseg; ++s) ov = ov && rh_aligned(d->D[s], 8);
  if (d->beta != 0.f && d->C) ov = ov && rh_aligned(d->C, 8) && d->ldc % 4 == 0;
  if (d->epilogue != RH_EPI_NONE) ov = ov && d->ldaux % 4 == 0;
  if (d->aux) ov = ov && rh_aligned(d->aux, 8);
  if (d->aux_out) ov = ov && rh_aligned(d->aux_out, 8);
  if (d->d_nseg > 1) ov = ov && d->d_seg_rows % 4 == 0;
  p.out_vec = ov ? 1 : 0;
  // (epilogue_tile_impl checks the alignment of each 8-element chunk itself)
  const bool lds = pl.splits + pl.tail == 1 && d->epilogue != RH_EPI_GELU_GRAD && d->epilogue != RH_EPI_MUL_AUX;
  p.epi_lds = lds ? 1 : 0;
  p.w4 = w4_addressable(d) ? 1 : 0;
  p.tiles_m = pl.tiles_m;
  p.tiles_n = pl.tiles_n;
  // Each XCD receives a contiguous run of ~tiles/8 logical tiles (tile_coords); grouping that
  // many tiles into a square-ish block of GROUP_M rows x (run/GROUP_M) columns minimises the A and
  // B panels one XCD's L2 has to fetch (2 x 4 blocks of the 2048x2048 weight-gradient tiles need
  // 6 panels where 8 x 1 blocks need 9).
  const int64_t per_xcd = rh_cdiv((int64_t)pl.tiles_m * pl.tiles_n, 8);
  int gm = 1;
  while ((int64_t)(2 * gm) * (2 * gm) <= per_xcd && 2 * gm <= pl.tiles_m) gm *= 2;
  p.group_m = gm;
  return p;
}

template <int BM, int BN, int WGM, int WGN, int L, int EPI, bool SPLIT>
void launch_bf16(const GemmParams<bf16_t>& p, bool dma, dim3 grid, hipStream_t st) {
  if (dma) hipLaunchKernelGGL((gemm_bf16_dma<BM, BN, WGM, WGN, L, EPI, SPLIT>), grid, dim3(64 * WGM * WGN), 0, st, p);
  else hipLaunchKernelGGL((gemm_bf16_mfma<BM, BN, WGM, WGN, L, EPI, SPLIT>), grid, dim3(64 * WGM * WGN), 0, st, p);
}


template <int L, int EPI, bool SPLIT>
void launch_cfg(int cfg, const GemmParams<bf16_t>& p, bool dma, dim3 grid, hipStream_t st) {
  switch (cfg) {
    case kT256x256:
      if (dma && four_wave_256(SPLIT) && p.w4)
        hipLaunchKernelGGL((gemm_bf16_dma<256, 256, 2, 2, L, EPI, SPLIT>), grid, dim3(256), 0, st, p);
      else launch_bf16<256, 256, 2, 4, L, EPI, SPLIT>(p, dma, grid, st);
      break;
    case kT256x128: launch_bf16<256, 128, 4, 2, L, EPI, SPLIT>(p, dma, grid, st); break;
    case kT256x192:
      if constexpr (L == RH_GEMM_NT) launch_bf16<256, 192, 4, 2, L, EPI, SPLIT>(p, dma, grid, st);
      break;
    default: launch_bf16<128, 128, 2, 2, L, EPI, SPLIT>(p, dma, grid, st); break;
  }
}

// The direct-to-LDS kernel covers every call whose operands it can address without bounds
// checks (see gemm_bf16_dma); RESIHP_GEMM_DMA=0 forces the register-staged kernel.
inline bool dma_ok(const rh_gemm_desc* d, const Plan& pl, const GemmParams<bf16_t>& p) {
  static const int enabled = [] {
    const char* e = getenv("RESIHP_GEMM_DMA");
    return (e && e[0] == '0' && e[1] == 0) ? 0 : 1;
  }();
  if (!enabled || !p.aligned || pl.k_main % kBK || pl.k_per_split % kBK) return false;
  const bool a_kc = d->layout != RH_GEMM_TN, b_kc = d->layout == RH_GEMM_NT;
  if (!a_kc && (d->M < 8 || d->M % 8)) return false;
  if (!b_kc && (d->N < 8 || d->N % 8)) return false;
  if (!b_kc && d->b_nseg > 1 && d->b_seg_rows % kBK) return false;
  return true;
}

template <typename T, int L, int EPI, bool SPLIT>
void launch_main(int cfg, const GemmParams<T>& p, bool dma, dim3 grid, hipStream_t st) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    launch_cfg<L, EPI, SPLIT>(cfg, p, dma, grid, st);
  } else {
    hipLaunchKernelGGL((gemm_f32_fma<L, EPI, SPLIT>), grid, dim3(256), 0, st, p);
  }
}

// Sum `slices` fp32 partial slices of p.ws in slice order and apply the epilogue.
template <typename T, int EPI>
int launch_reduce(const rh_gemm_desc* d, const GemmParams<T>& p, int slices, const void* ws, hipStream_t st) {
  const int64_t total = d->M * d->N;
  if constexpr (std::is_same<T, bf16_t>::value) {
    // every output row and the partials are 16-byte aligned when N % 8 == 0 (the partials
    // are [splits][M][N] fp32); D/C/aux rows need ld % 8 == 0 and aligned bases as well
    bool vec = d->N % 8 == 0 && d->ldd % 8 == 0 && rh_aligned(ws, 16);
    for (int q = 0; q < d->d_nseg; ++q) vec = vec && rh_aligned(d->D[q], 16);
    if (d->beta != 0.f && d->C) vec = vec && rh_aligned(d->C, 16) && d->ldc % 8 == 0;
    if (d->epilogue != RH_EPI_NONE) {
      const bool writes = d->epilogue == RH_EPI_GELU || d->epilogue == RH_EPI_GELU_DERIV;
      vec = vec && rh_aligned(writes ? d->aux_out : d->aux, 16) && d->ldaux % 8 == 0;
    }
    if (vec) {
      int64_t blocks = rh_cdiv(total / 8, 256);
      if (blocks > 8 * 1024) blocks = 8 * 1024;
      hipLaunchKernelGGL((gemm_splitk_reduce_vec<EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, slices);
      return rh_check_launch("rh_gemm split-k reduce");
    }
  }
  int64_t blocks = rh_cdiv(total, 256);
  if (blocks > 4 * 1024) blocks = 4 * 1024;
  hipLaunchKernelGGL((gemm_splitk_reduce<T, EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, slices);
  return rh_check_launch("rh_gemm split-k reduce");
}

template <typename T, int L, int EPI>
int launch_layout(const rh_gemm_desc* d, const Plan& pl, void* ws, hipStream_t st, int stage) {
  GemmParams<T> p = make_params<T>(d, pl, ws);
  const int64_t tiles = (int64_t)pl.tiles_m * pl.tiles_n;
  if (tiles > INT32_MAX) return rh_set_error(RH_ERR_INVALID, "rh_gemm: too many tiles (%lld)", (long long)tiles);
  dim3 grid((unsigned)tiles, 1, (unsigned)pl.splits);
  const int slices = pl.splits + pl.tail;
  p.K = pl.k_main;  // the split slices cover [0, k_main); a tail slice covers the rest
  bool dma = false;
  if constexpr (std::is_same<T, bf16_t>::value) dma = dma_ok(d, pl, p);
  if (slices > 1) {
    if (stage != RH_GEMM_STAGE_REDUCE) {
      // split slices write raw fp32 partials whatever the epilogue (the reduce applies it), so
      // every epilogue shares the RH_EPI_NONE main kernels
      launch_main<T, L, RH_EPI_NONE, true>(pl.cfg, p, dma, grid, st);
      int rc = rh_check_launch("rh_gemm");
      if (rc) return rc;
      if (pl.tail) {
        // [k_main, K) into partial slice `splits`, operands offset by k_main along K
        GemmParams<T> pt = p;
        pt.K = d->K - pl.k_main;
        pt.k_per_split = pt.K;
        pt.A = L == RH_GEMM_TN ? p.A + pl.k_main * p.lda : p.A + pl.k_main;
        for (int s = 0; s < RH_MAX_SEG; ++s)
          pt.B[s] = L == RH_GEMM_NT ? p.B[s] + pl.k_main : p.B[s] + pl.k_main * p.ldb;
        pt.ws = p.ws + (int64_t)pl.splits * d->M * d->N;
        launch_main<T, L, RH_EPI_NONE, true>(pl.cfg, pt, false, dim3((unsigned)tiles, 1, 1), st);
        rc = rh_check_launch("rh_gemm (K tail)");
        if (rc) return rc;
      }
      if (stage == RH_GEMM_STAGE_MAIN) return RH_OK;
    }
    return launch_reduce<T, EPI>(d, p, slices, ws, st);
  }
  if (stage == RH_GEMM_STAGE_REDUCE) return RH_OK;  // unsplit: the main kernel did everything
  launch_main<T, L, EPI, false>(pl.cfg, p, dma, grid, st);
  return rh_check_launch("rh_gemm");
}

// ---------------------------------------------------------------------------
// grouped GEMMs (rh_gemm_grouped)
// ---------------------------------------------------------------------------
struct GroupPlan {
  int ok = 0;       // 0: the group runs as separate rh_gemm calls
  int splits = 1;
  int64_t kps[kMaxGroup] = {};
  int64_t ws_off[kMaxGroup + 1] = {};  // byte offset of each problem's partials; ws_off[n] = total
};

// One launch for the whole group needs bf16, one layout, no epilogue, K a multiple of the k-tile
// and operands the direct-to-LDS kernel can address; the split-K count (1, 2 or 4, shared by the
// group) minimises waves x K per split plus the partial traffic, as plan_gemm does.
inline GroupPlan plan_grouped(const rh_gemm_desc* d, int n) {
  GroupPlan g;
  if (n < 1 || n > kMaxGroup) return g;
  for (int i = 0; i < n; ++i) {
    if (d[i].dtype != RH_DTYPE_BF16 || d[i].layout != d[0].layout || d[i].epilogue != RH_EPI_NONE) return g;
    if (d[i].M == 0 || d[i].N == 0 || d[i].K == 0 || d[i].K % kBK) return g;
  }
  const int64_t cus = rh_device_cus();
  double best = 1e300;
  for (int s : {1, 2, 4}) {
    int64_t wgs = 0, kmax = 0, partial = 0;
    bool fits = true;
    for (int i = 0; i < n; ++i) {
      const int64_t kps = rh_cdiv(rh_cdiv(d[i].K, s), kBK) * kBK;
      if (s > 1 && (d[i].K / s < 512 || rh_cdiv(d[i].K, kps) != s)) fits = false;
      wgs += rh_cdiv(d[i].M, 256) * rh_cdiv(d[i].N, 256) * s;
      kmax = std::max(kmax, kps);
      partial += s > 1 ? s * d[i].M * d[i].N : 0;
    }
    if (!fits || wgs > INT32_MAX) continue;
    const double t = (double)rh_cdiv(wgs, cus) * 256.0 * 256.0 * (double)kmax + kGroupSplitCost * (double)partial;
    if (t < best * 0.98) {
      best = t;
      g.splits = s;
    }
  }
  int64_t off = 0;
  for (int i = 0; i < n; ++i) {
    Plan pl{kT256x256, g.splits, 0, 0, (int)rh_cdiv(d[i].M, 256), (int)rh_cdiv(d[i].N, 256)};
    pl.k_per_split = rh_cdiv(rh_cdiv(d[i].K, g.splits), kBK) * kBK;
    pl.k_main = d[i].K;
    const GemmParams<bf16_t> p = make_params<bf16_t>(&d[i], pl, nullptr);
    if (!dma_ok(&d[i], pl, p)) return GroupPlan{};
    g.kps[i] = pl.k_per_split;
    g.ws_off[i] = off;
    if (g.splits > 1) off += rh_cdiv(g.splits * d[i].M * d[i].N * (int64_t)sizeof(float), 256) * 256;
  }
  g.ws_off[n] = off;
  g.ok = 1;
  return g;
}

template <int L>
int launch_grouped(const rh_gemm_desc* d, int n, const GroupPlan& g, void* ws, hipStream_t st) {
  GroupedParams gp{};
  int total = 0;
  for (int i = 0; i < n; ++i) {
    Plan pl{kT256x256, g.splits, g.kps[i], 0, (int)rh_cdiv(d[i].M, 256), (int)rh_cdiv(d[i].N, 256)};
    pl.k_main = d[i].K;
    gp.p[i] = make_params<bf16_t>(&d[i], pl, static_cast<char*>(ws) + g.ws_off[i]);
    gp.first[i] = total;
    total += pl.tiles_m * pl.tiles_n * g.splits;
  }
  gp.first[n] = total;
  gp.count = n;
  gp.splits = g.splits;
  const unsigned grid = (unsigned)total;
  bool w4 = four_wave_256(true);
  for (int i = 0; i < n; ++i) w4 = w4 && w4_addressable(&d[i]);
  if (w4) {
    if (g.splits > 1)
      hipLaunchKernelGGL((gemm_bf16_dma_grouped<256, 256, 2, 2, L, true>), dim3(grid), dim3(256), 0, st, gp);
    else
      hipLaunchKernelGGL((gemm_bf16_dma_grouped<256, 256, 2, 2, L, false>), dim3(grid), dim3(256), 0, st, gp);
  } else if (g.splits > 1)
    hipLaunchKernelGGL((gemm_bf16_dma_grouped<256, 256, 2, 4, L, true>), dim3(grid), dim3(512), 0, st, gp);
  else
    hipLaunchKernelGGL((gemm_bf16_dma_grouped<256, 256, 2, 4, L, false>), dim3(grid), dim3(512), 0, st, gp);
  int rc = rh_check_launch("rh_gemm_grouped");
  if (rc) return rc;
  if (g.splits > 1) {
    for (int i = 0; i < n; ++i) {
      rc = launch_reduce<bf16_t, RH_EPI_NONE>(&d[i], gp.p[i], g.splits, gp.p[i].ws, st);
      if (rc) return rc;
    }
  }
  return RH_OK;
}

}  // namespace rh_gemm_impl
