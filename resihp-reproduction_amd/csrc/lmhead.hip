// LM head fused with the next-token cross-entropy: logits = x . W^T and
// loss = mean over scored rows of (lse - logit[target]) without the [tokens, vocab] logits or
// their gradient ever reaching HBM as whole tensors.
//
// Forward: the NT GEMM's epilogue reduces every 64-column block of a row to a base-2
// (max, sum-exp) pair and picks out the target logit (epilogue_lse); a combine kernel folds the
// blocks of each row into its log-sum-exp and loss, and a single block takes the mean in a fixed
// order (deterministic).
// Backward, vocabulary chunk by chunk (8192 ids): the logits of the chunk are recomputed by the
// same GEMM with the gradient epilogue (epilogue_xent_grad), which stores
//   dS = (softmax - onehot) * dloss / N
// in bf16 into a chunk buffer (134 MB at 8192 tokens, reused by every chunk); the chunk's rows of
// dW = dS^T . x go straight into the weight gradient (rh_gemm), and dX's share dS . W_chunk is
// written as one fp32 slice; after the last chunk one ordered reduce sums the slices into dX.
// One extra GEMM (the recompute) buys the absence of both 823 MB logits tensors at GPT-2-small.
#include "gemm_impl.hpp"

using namespace rh_gemm_impl;

namespace {

constexpr int64_t kChunk = 8192;  // vocabulary ids per backward chunk

__global__ __launch_bounds__(256) void lse_combine_kernel(int64_t rows, int S, int64_t V, int nblk, int64_t ld_part,
                                                          const float* __restrict__ part, const float* __restrict__ tgt,
                                                          const int64_t* __restrict__ tokens, float* __restrict__ lse,
                                                          float* __restrict__ loss_rows) {
  __shared__ float scratch[16];
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  const float* pr = part + row * ld_part;
  float m = -INFINITY;
  for (int b = threadIdx.x; b < nblk; b += 256) m = fmaxf(m, pr[2 * b]);
  const float M = block_max(m, scratch);
  float s = 0.f;
  for (int b = threadIdx.x; b < nblk; b += 256) {
    const float mb = pr[2 * b];
    if (mb != -INFINITY) s += pr[2 * b + 1] * __builtin_amdgcn_exp2f(mb - M);
  }
  const float tot = block_sum(s, scratch + 8);
  if (threadIdx.x == 0) {
    const float l = (M + log2f(tot)) * 0.69314718055994530942f;
    const bool scored = row % S != S - 1;
    lse[row] = scored ? l : 0.f;
    float lr = 0.f;
    if (scored) {
      const int64_t t = tokens[row + 1];
      lr = (t >= 0 && t < V) ? l - tgt[row] : NAN;  // an id outside the vocabulary poisons the loss
    }
    loss_rows[row] = lr;
  }
}

__global__ __launch_bounds__(1024) void mean_rows_kernel(int64_t n, const float* __restrict__ rows, float inv_n,
                                                         float* __restrict__ out) {
  __shared__ float scratch[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += rows[i];
  const float tot = block_sum(s, scratch);
  if (threadIdx.x == 0) out[0] = tot * inv_n;
}

struct FwdLayout {
  int64_t nblk, ld_part, part_bytes, tgt_off, rows_off, total;
};
FwdLayout fwd_layout(int64_t rows, int64_t V) {
  FwdLayout f;
  f.nblk = rh_cdiv(V, 64);
  f.ld_part = 2 * f.nblk;
  f.part_bytes = rh_cdiv(rows * f.ld_part * (int64_t)sizeof(float), 256) * 256;
  f.tgt_off = f.part_bytes;
  f.rows_off = f.tgt_off + rh_cdiv(rows * (int64_t)sizeof(float), 256) * 256;
  f.total = f.rows_off + rh_cdiv(rows * (int64_t)sizeof(float), 256) * 256;
  return f;
}

// The chunk GEMMs of the backward as rh_gemm descriptors.
rh_gemm_desc chunk_wgrad_desc(int64_t rows, int64_t dim, int64_t n_valid, int64_t n_store, const void* dS,
                              int64_t ld_s, const void* x, void* dw_rows, void* pad_rows, float beta) {
  rh_gemm_desc d{};
  d.dtype = RH_DTYPE_BF16;
  d.layout = RH_GEMM_TN;
  d.epilogue = RH_EPI_NONE;
  d.b_nseg = 1;
  d.M = n_store;
  d.N = dim;
  d.K = rows;
  d.A = dS;
  d.lda = ld_s;
  d.B[0] = x;
  d.ldb = dim;
  d.alpha = 1.f;
  d.beta = beta;
  d.ldd = dim;
  if (n_store > n_valid) {  // rows past the vocabulary land in a scratch segment
    d.d_nseg = 2;
    d.d_seg_rows = n_valid;
    d.D[0] = dw_rows;
    d.D[1] = pad_rows;
  } else {
    d.d_nseg = 1;
    d.D[0] = dw_rows;
  }
  return d;
}

struct BwdLayout {
  int64_t ld_s, nchunks, slices, ds_bytes, slice_off, slice_bytes, pad_off, gemm_off, gemm_bytes, total;
};
BwdLayout bwd_layout(int64_t rows, int64_t V, int64_t dim) {
  BwdLayout b;
  const int64_t wmax = std::min(V, kChunk);
  b.ld_s = rh_cdiv(wmax, 64) * 64;
  b.nchunks = rh_cdiv(V, kChunk);
  const int64_t last = V - (b.nchunks - 1) * kChunk;
  b.slices = b.nchunks + (last % 64 ? 1 : 0);  // a ragged last chunk adds a K-tail slice
  b.ds_bytes = rh_cdiv(rows * b.ld_s * 2, 256) * 256;
  b.slice_off = b.ds_bytes;
  b.slice_bytes = rows * dim * (int64_t)sizeof(float);
  b.pad_off = b.slice_off + rh_cdiv(b.slices * b.slice_bytes, 256) * 256;
  b.gemm_off = b.pad_off + rh_cdiv(8 * dim * 2, 256) * 256;
  // split-K workspace of the chunk weight-gradient GEMMs (full and last chunk)
  int64_t most = 0;
  for (int64_t w : {wmax, last}) {
    const int64_t store = rh_cdiv(w, 8) * 8;
    rh_gemm_desc d = chunk_wgrad_desc(rows, dim, w, store, (void*)256, b.ld_s, (void*)256, (void*)256, (void*)256, 1.f);
    const Plan pl = plan_gemm(&d);
    most = std::max(most, pl.ws_bytes);
  }
  b.gemm_bytes = most;
  b.total = b.gemm_off + rh_cdiv(most, 256) * 256;
  return b;
}

int check_lmhead(const char* who, int64_t B, int64_t S, int64_t V, int64_t dim) {
  RH_REQUIRE(B >= 1 && S >= 2, "%s: need batch >= 1 and seq >= 2", who);
  RH_REQUIRE(V >= 1 && V < (1ll << 31), "%s: vocabulary of %lld ids", who, (long long)V);
  RH_REQUIRE(dim >= 64 && dim % 64 == 0, "%s: model_dim %lld must be a positive multiple of 64", who, (long long)dim);
  RH_REQUIRE(B * S <= INT32_MAX / 2, "%s: too many tokens", who);
  return RH_OK;
}

// NT GEMM x[rows, dim] . W[c0 : c0 + n, :]^T with one of the cross-entropy epilogues.
template <int EPI>
int launch_xent_gemm(GemmParams<bf16_t> p, hipStream_t st) {
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL((gemm_bf16_dma<256, 256, 2, 4, RH_GEMM_NT, EPI, false>), dim3((unsigned)tiles), dim3(512), 0, st,
                     p);
  return rh_check_launch("rh_lmhead_xent (GEMM)");
}

GemmParams<bf16_t> nt_params(int64_t rows, int64_t n, int64_t dim, const void* x, const void* w_rows) {
  rh_gemm_desc d{};
  d.dtype = RH_DTYPE_BF16;
  d.layout = RH_GEMM_NT;
  d.epilogue = RH_EPI_NONE;
  d.b_nseg = d.d_nseg = 1;
  d.M = rows;
  d.N = n;
  d.K = dim;
  d.A = x;
  d.lda = dim;
  d.B[0] = w_rows;
  d.ldb = dim;
  d.alpha = 1.f;
  d.D[0] = (void*)x;  // unused by the cross-entropy epilogues
  d.ldd = n;
  Plan pl{kT256x256, 1, dim, 0, (int)rh_cdiv(rows, 256), (int)rh_cdiv(n, 256)};
  pl.k_main = dim;
  return make_params<bf16_t>(&d, pl, nullptr);
}

}  // namespace

extern "C" int rh_lmhead_xent_workspace_bytes(int64_t batch, int64_t seq, int64_t vocab, int64_t dim,
                                              int64_t* fwd_bytes, int64_t* bwd_bytes) {
  int rc = check_lmhead("rh_lmhead_xent_workspace_bytes", batch, seq, vocab, dim);
  if (rc) return rc;
  RH_REQUIRE(fwd_bytes && bwd_bytes, "rh_lmhead_xent_workspace_bytes: null output");
  *fwd_bytes = fwd_layout(batch * seq, vocab).total;
  *bwd_bytes = bwd_layout(batch * seq, vocab, dim).total;
  return RH_OK;
}

extern "C" int rh_lmhead_xent_fwd(int64_t batch, int64_t seq, int64_t vocab, int64_t dim, const void* x,
                                  const void* w, const int64_t* tokens, float* row_lse, float* loss,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_lmhead("rh_lmhead_xent_fwd", batch, seq, vocab, dim);
  if (rc) return rc;
  RH_REQUIRE(x && w && tokens && row_lse && loss, "rh_lmhead_xent_fwd: null pointer");
  RH_REQUIRE(rh_aligned(x, 16) && rh_aligned(w, 16), "rh_lmhead_xent_fwd: x and W must be 16-byte aligned");
  const int64_t rows = batch * seq;
  const FwdLayout f = fwd_layout(rows, vocab);
  RH_REQUIRE(workspace && workspace_bytes >= f.total && rh_aligned(workspace, 256),
             "rh_lmhead_xent_fwd: workspace of %lld bytes is too small (%lld needed, 256-byte aligned)",
             (long long)workspace_bytes, (long long)f.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws);
  float* tgt = reinterpret_cast<float*>(ws + f.tgt_off);
  float* loss_rows = reinterpret_cast<float*>(ws + f.rows_off);
  GemmParams<bf16_t> p = nt_params(rows, vocab, dim, x, w);
  p.tokens = tokens;
  p.part = part;
  p.tgt = tgt;
  p.seq = seq;
  p.col_off = 0;
  p.ld_part = f.ld_part;
  rc = launch_xent_gemm<kEpiLsePartial>(p, st);
  if (rc) return rc;
  hipLaunchKernelGGL(lse_combine_kernel, dim3((unsigned)rows), dim3(256), 0, st, rows, (int)seq, vocab, (int)f.nblk,
                     f.ld_part, part, tgt, tokens, row_lse, loss_rows);
  rc = rh_check_launch("rh_lmhead_xent_fwd (combine)");
  if (rc) return rc;
  hipLaunchKernelGGL(mean_rows_kernel, dim3(1), dim3(1024), 0, st, rows, loss_rows, 1.0f / (float)(batch * (seq - 1)),
                     loss);
  return rh_check_launch("rh_lmhead_xent_fwd (mean)");
}

extern "C" int rh_lmhead_xent_bwd(int64_t batch, int64_t seq, int64_t vocab, int64_t dim, const void* x,
                                  const void* w, const int64_t* tokens, const float* row_lse, const float* grad_loss,
                                  void* dx, void* dw, int accumulate, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  int rc = check_lmhead("rh_lmhead_xent_bwd", batch, seq, vocab, dim);
  if (rc) return rc;
  RH_REQUIRE(x && w && tokens && row_lse && grad_loss && dx && dw, "rh_lmhead_xent_bwd: null pointer");
  RH_REQUIRE(rh_aligned(x, 16) && rh_aligned(w, 16) && rh_aligned(dx, 16) && rh_aligned(dw, 16),
             "rh_lmhead_xent_bwd: x, W, dx and dW must be 16-byte aligned");
  const int64_t rows = batch * seq;
  const BwdLayout b = bwd_layout(rows, vocab, dim);
  RH_REQUIRE(workspace && workspace_bytes >= b.total && rh_aligned(workspace, 256),
             "rh_lmhead_xent_bwd: workspace of %lld bytes is too small (%lld needed, 256-byte aligned)",
             (long long)workspace_bytes, (long long)b.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  bf16_t* dS = reinterpret_cast<bf16_t*>(ws);
  float* slices = reinterpret_cast<float*>(ws + b.slice_off);
  bf16_t* pad = reinterpret_cast<bf16_t*>(ws + b.pad_off);
  void* gemm_ws = b.gemm_bytes ? ws + b.gemm_off : nullptr;
  const bf16_t* W = static_cast<const bf16_t*>(w);
  bf16_t* dW = static_cast<bf16_t*>(dw);
  const float inv_n = 1.0f / (float)(batch * (seq - 1));
  int slice = 0;
  for (int64_t c = 0; c < b.nchunks; ++c) {
    const int64_t c0 = c * kChunk;
    const int64_t n_valid = std::min(kChunk, vocab - c0);
    const int64_t n_store = rh_cdiv(n_valid, 8) * 8;
    // 1. recompute the chunk's logits; store its softmax gradient dS
    GemmParams<bf16_t> p = nt_params(rows, n_valid, dim, x, W + c0 * dim);
    p.D[0] = dS;
    p.ldd = b.ld_s;
    p.tokens = tokens;
    p.lse = row_lse;
    p.grad = grad_loss;
    p.inv_n = inv_n;
    p.seq = seq;
    p.col_off = c0;
    p.n_store = n_store;
    rc = launch_xent_gemm<kEpiXentGrad>(p, st);
    if (rc) return rc;
    // 2. the chunk's rows of dW = dS^T . x
    rh_gemm_desc dwd = chunk_wgrad_desc(rows, dim, n_valid, n_store, dS, b.ld_s, x, dW + c0 * dim, pad,
                                        accumulate ? 1.f : 0.f);
    rc = rh_gemm(&dwd, gemm_ws, b.gemm_bytes, stream);
    if (rc) return rc;
    // 3. dX's share dS . W_chunk as fp32 slice(s): the 64-aligned bulk of the chunk width on the
    //    direct-to-LDS kernel, a ragged remainder on the bounds-checked one
    rh_gemm_desc nd{};
    nd.dtype = RH_DTYPE_BF16;
    nd.layout = RH_GEMM_NN;
    nd.epilogue = RH_EPI_NONE;
    nd.b_nseg = nd.d_nseg = 1;
    nd.M = rows;
    nd.N = dim;
    nd.K = n_valid;
    nd.A = dS;
    nd.lda = b.ld_s;
    nd.B[0] = W + c0 * dim;
    nd.ldb = dim;
    nd.alpha = 1.f;
    nd.D[0] = dx;
    nd.ldd = dim;
    const int64_t kb = n_valid / 64 * 64;
    Plan pl{kT256x128, 1, kb, 0, (int)rh_cdiv(rows, 256), (int)rh_cdiv(dim, 128)};
    pl.k_main = kb;
    GemmParams<bf16_t> pn = make_params<bf16_t>(&nd, pl, slices);
    const dim3 grid((unsigned)((int64_t)pl.tiles_m * pl.tiles_n));
    if (kb > 0) {
      pn.K = kb;
      pn.ws = slices + (int64_t)slice * rows * dim;
      hipLaunchKernelGGL((gemm_bf16_dma<256, 128, 4, 2, RH_GEMM_NN, RH_EPI_NONE, true>), grid, dim3(512), 0, st, pn);
      rc = rh_check_launch("rh_lmhead_xent_bwd (dX slice)");
      if (rc) return rc;
      ++slice;
    }
    if (n_valid > kb) {
      GemmParams<bf16_t> pt = pn;
      pt.K = n_valid - kb;
      pt.k_per_split = pt.K;
      pt.A = static_cast<const bf16_t*>(nd.A) + kb;
      for (int s = 0; s < RH_MAX_SEG; ++s) pt.B[s] = W + (c0 + kb) * dim;
      pt.ws = slices + (int64_t)slice * rows * dim;
      hipLaunchKernelGGL((gemm_bf16_mfma<256, 128, 4, 2, RH_GEMM_NN, RH_EPI_NONE, true>), grid, dim3(512), 0, st, pt);
      rc = rh_check_launch("rh_lmhead_xent_bwd (dX tail slice)");
      if (rc) return rc;
      ++slice;
    }
  }
  // 4. dX = the slices summed in order, rounded once
  rh_gemm_desc rd{};
  rd.dtype = RH_DTYPE_BF16;
  rd.layout = RH_GEMM_NN;
  rd.epilogue = RH_EPI_NONE;
  rd.b_nseg = rd.d_nseg = 1;
  rd.M = rows;
  rd.N = dim;
  rd.K = 1;
  rd.alpha = 1.f;
  rd.D[0] = dx;
  rd.ldd = dim;
  Plan pr{kT256x256, slice, 1, 0, 1, 1};
  GemmParams<bf16_t> prm = make_params<bf16_t>(&rd, pr, slices);
  return launch_reduce<bf16_t, RH_EPI_NONE>(&rd, prm, slice, slices, st);
}
