/*
 * resihp_hip.h -- C ABI of the MI355X (gfx950) kernels behind the decoder-LM
 * forward/backward step of resihp/model.py and the shard math of
 * resihp/parallel/tp.py, plus the on-device TP re-slice of
 * resihp/parallel/reshard.py.
 *
 * Conventions shared by every entry point:
 *   - plain device pointers, element counts and leading dimensions in
 *     ELEMENTS (not bytes) unless a name says *_bytes;
 *   - `stream` is a hipStream_t passed as void*; work is only enqueued, no
 *     entry point synchronises the device or allocates device memory;
 *   - scratch space comes from the caller (`workspace`, sized by the matching
 *     *_workspace_bytes query);
 *   - return value 0 = success; otherwise an RH_ERR_* code and a message
 *     available from rh_last_error() (thread-local).
 *
 * Storage dtypes: RH_DTYPE_F32 (IEEE fp32) and RH_DTYPE_BF16 (bfloat16,
 * round-to-nearest-even).  Every kernel accumulates in fp32.
 *
 * The reference (ksqbxm/resihp-reproduction) is pure Python on PyTorch; it has
 * no foreign-function interface of its own.  Each entry point below names the
 * reference call site(s) whose ATen op it replaces.
 */
#ifndef RESIHP_HIP_H
#define RESIHP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status / dtype codes ------------------------------------------------ */
#define RH_OK 0
#define RH_ERR_INVALID 1     /* bad shape / pointer / argument (maps to ValueError) */
#define RH_ERR_HIP 2         /* HIP runtime or launch failure                       */
#define RH_ERR_UNSUPPORTED 3 /* valid request this build does not implement         */

#define RH_DTYPE_F32 0
#define RH_DTYPE_BF16 1

/* Library version (major*10000 + minor*100 + patch). */
int rh_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* rh_last_error(void);

/* ---- GEMM ------------------------------------------------------------------
 * Replaces F.linear / nn.Linear (bias-free, weight [out,in]) and the matmuls of
 * its autograd backward:
 *   q/k/v projections   resihp/model.py:55-57,63-65   resihp/parallel/tp.py:235-237
 *   out_proj            resihp/model.py:58,71         resihp/parallel/tp.py:243
 *   fc1 / fc2           resihp/model.py:77-78,81      resihp/parallel/tp.py:247-248
 *   lm_head             resihp/model.py:116,133       resihp/parallel/tp.py:272
 * All matrices are row-major.  Layouts:
 *   RH_GEMM_NT : D[M,N] = A[M,K] . B[N,K]^T   (forward  y  = x . W^T)
 *   RH_GEMM_NN : D[M,N] = A[M,K] . B[K,N]     (dgrad    dx = dy . W)
 *   RH_GEMM_TN : D[M,N] = A[K,M]^T . B[K,N]   (wgrad    dW = dy^T . x)
 * then  v = alpha*acc + beta*C  and the epilogue:
 *   RH_EPI_NONE      D = v
 *   RH_EPI_GELU      aux_out = v, D = gelu(v)            (fc1 + exact-erf GELU,
 *                                                       model.py:81, tp.py:247)
 *   RH_EPI_GELU_GRAD D = v * gelu'(aux)                  (GELU backward fused
 *                                                       into the fc2 dgrad)
 *   RH_EPI_GELU_DERIV aux_out = gelu'(v), D = gelu(v)    (fc1 forward keeping the
 *                                                       derivative for backward)
 *   RH_EPI_MUL_AUX   D = v * aux                         (fc2 dgrad times the kept
 *                                                       derivative)
 * bf16 results evaluate gelu / gelu' with Abramowitz & Stegun 7.1.26 for the normal
 * CDF (|error| <= 7e-8, far below bf16 resolution); fp32 results use erff/expf.
 * Segmented operands let three separate q/k/v weights act as one [3*d_l, d]
 * matrix without a copy: row r of the *stored* B lives at
 * B[r / b_seg_rows] + (r % b_seg_rows)*ldb, and row m of D lives at
 * D[m / d_seg_rows] + (m % d_seg_rows)*ldd.  With b_nseg == 1 (d_nseg == 1)
 * only B[0] (D[0]) is used.  C == NULL with beta != 0 reads C from D
 * (in-place accumulation, e.g. into a parameter's .grad).
 */
#define RH_GEMM_NT 0
#define RH_GEMM_NN 1
#define RH_GEMM_TN 2

#define RH_EPI_NONE 0
#define RH_EPI_GELU 1
#define RH_EPI_GELU_GRAD 2
#define RH_EPI_GELU_DERIV 3
#define RH_EPI_MUL_AUX 4

#define RH_MAX_SEG 4

typedef struct rh_gemm_desc {
  int32_t dtype;
  int32_t layout;
  int32_t epilogue;
  int32_t b_nseg;
  int32_t d_nseg;
  int32_t reserved;
  int64_t M, N, K;
  const void* A;
  int64_t lda;
  const void* B[RH_MAX_SEG];
  int64_t ldb;
  int64_t b_seg_rows;
  float alpha;
  float beta;
  const void* C;
  int64_t ldc;
  void* D[RH_MAX_SEG];
  int64_t ldd;
  int64_t d_seg_rows;
  const void* aux;
  void* aux_out;
  int64_t ldaux;
} rh_gemm_desc;

/* Workspace (bytes) rh_gemm would use for split-K on this device; 0 if none. */
int rh_gemm_workspace_bytes(const rh_gemm_desc* desc, int64_t* bytes);
/* A smaller workspace than requested is legal: the call then runs unsplit. */
int rh_gemm(const rh_gemm_desc* desc, void* workspace, int64_t workspace_bytes, void* stream);
/* rh_gemm in two enqueued halves: RH_GEMM_STAGE_MAIN runs the main kernel (for a split-K
 * plan it writes the fp32 partials to the workspace), RH_GEMM_STAGE_REDUCE then sums the
 * partials and applies the epilogue (a no-op for an unsplit plan); RH_GEMM_STAGE_ALL is
 * rh_gemm.  Both halves must see the same descriptor, workspace and stream order.  No
 * counterpart in the reference: it lets profilers time the two kernels apart and callers
 * schedule other work between them. */
#define RH_GEMM_STAGE_ALL 0
#define RH_GEMM_STAGE_MAIN 1
#define RH_GEMM_STAGE_REDUCE 2
int rh_gemm_stage(const rh_gemm_desc* desc, void* workspace, int64_t workspace_bytes, int stage, void* stream);
/* Name of the main-kernel instantiation rh_gemm launches for this descriptor with the queried
 * workspace (as rocprof prints it, e.g. "gemm_bf16_dma<256, 256, 2, 4, 0, 0, false>"), for
 * attributing profiler records.  No counterpart in the reference (profiling support). */
int rh_gemm_kernel_name(const rh_gemm_desc* desc, char* buf, int64_t len);

/* Grouped GEMMs: up to 4 problems of one layout in ONE launch -- the weight gradients of a
 * decoder block (fc2, fc1, out_proj and the fused q/k/v: dW = dY^T X with the token count
 * as K, resihp/parallel/tp.py:235-248 and their autograd backward), so the block's wgrads
 * fill the chip together instead of each needing a split-K pass of its own.  Every
 * descriptor is an ordinary rh_gemm descriptor (beta/C accumulation into .grad and
 * segmented D included); each problem's result equals rh_gemm's up to the order of the
 * split-K partial sums.  The group runs in one launch (plus one reduce per problem when
 * the planner splits K) when all are bf16, of one layout, RH_EPI_NONE, K a multiple of 64
 * and the operands 16-byte aligned; otherwise, or with a smaller workspace than queried,
 * the problems run as consecutive rh_gemm calls.  rh_gemm_grouped_plan reports the split
 * count the single launch would use (0: consecutive calls).  No counterpart in the
 * reference beyond the GEMMs themselves. */
#define RH_GEMM_MAX_GROUP 4
int rh_gemm_grouped_workspace_bytes(const rh_gemm_desc* descs, int n, int64_t* bytes);
int rh_gemm_grouped(const rh_gemm_desc* descs, int n, void* workspace, int64_t workspace_bytes,
                    void* stream);
int rh_gemm_grouped_plan(const rh_gemm_desc* descs, int n, int* splits);
/* The kernel the single launch would run (its template name, as profilers print it), or "none"
 * when the group runs as consecutive rh_gemm calls.  No counterpart in the reference
 * (profiling support). */
int rh_gemm_grouped_kernel_name(const rh_gemm_desc* descs, int n, char* buf, int64_t len);

/* ---- causal self-attention core ---------------------------------------------
 * Replaces  scores = q @ k^T / sqrt(Dh); masked_fill(triu(ones,1), -inf);
 * softmax(-1); @ v   (resihp/model.py:62-70, resihp/parallel/tp.py:231-242)
 * and its autograd backward, as one fused online-softmax kernel that never
 * materialises the [S,S] scores.
 * Token t = b*seq + s; element (t, head h, d) of q/k/v/o/do/dq/dk/dv is at
 * ptr + t*ld + h*head_dim + d.  lse is [batch, heads, seq] fp32, natural log of
 * the softmax denominator of each query row (saved by forward for backward).
 * `causal` = 1 masks keys after the query (the diagonal is kept), as the
 * reference always does; 0 attends to every key.  `scale` must be positive
 * (the reference's 1/sqrt(head_dim)); other values are rejected (RH_ERR_INVALID).
 * o_lo (bf16 only, may be NULL; same layout as o): the forward writes the rounding
 * residual o - bf16(o), and the backward forms delta_i = do_i.o_i from o + o_lo.
 * delta must equal sum_j P_ij dP_ij for every row of dS to sum to zero; from the
 * rounded o alone it does not, and dq / dk pick up that error times the common
 * component of the keys / queries (about 2 % of the q/k projection gradients of a
 * 12-layer GPT-2-small at random init, against 0.3 % with o_lo).
 */
int rh_attn_fwd(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                const void* q, const void* k, const void* v, int64_t ld_qkv,
                void* o, void* o_lo, int64_t ld_o, float* lse, float scale, int causal, void* stream);
int rh_attn_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t heads, int64_t* bytes);
int rh_attn_bwd(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                const void* q, const void* k, const void* v, int64_t ld_qkv,
                const void* o, const void* o_lo, int64_t ld_o, const void* dout, int64_t ld_do,
                const float* lse, void* dq, void* dk, void* dv, int64_t ld_dqkv, float scale,
                int causal, void* workspace, int64_t workspace_bytes, void* stream);

/* rh_attn_bwd_noalloc: rh_attn_bwd with no workspace argument and no allocation of any
 * kind -- for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The backward's scratch (delta, one fp32 per query row) lives in a static device array
 * of RH_ATTN_NOALLOC_MAX_ROWS floats (8 MiB, held by every GPU the library runs on until
 * the process ends); batch*seq*heads above that limit is rejected (RH_ERR_INVALID).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must not be issued; calls in one stream's order are
 * safe.  Results equal rh_attn_bwd's bit for bit. */
#define RH_ATTN_NOALLOC_MAX_ROWS 2097152
int rh_attn_bwd_noalloc(int dtype, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                        const void* q, const void* k, const void* v, int64_t ld_qkv,
                        const void* o, const void* o_lo, int64_t ld_o, const void* dout, int64_t ld_do,
                        const float* lse, void* dq, void* dk, void* dv, int64_t ld_dqkv, float scale,
                        int causal, void* stream);

/* ---- LayerNorm ----------------------------------------------------------------
 * Replaces nn.LayerNorm / F.layer_norm over the last dim, eps default 1e-5,
 * biased variance (resihp/model.py:89,91,95-96,115,132;
 * resihp/parallel/tp.py:262,264,268) and its backward.  x/y/dy/dx are
 * [rows, dim] contiguous; gamma/beta [dim]; mean/rstd [rows] fp32.
 * Backward: dx = LN_bwd(dy) (+ dresidual when non-NULL: the residual-branch
 * gradient of x + sublayer(LN(x)), model.py:95-96, fused here);
 * dgamma/dbeta (either may be NULL) are written, or added to when
 * accumulate != 0 (gradient accumulation into .grad).
 */
int rh_layernorm_fwd(int dtype, int64_t rows, int64_t dim, const void* x, const void* gamma,
                     const void* beta, float eps, void* y, float* mean, float* rstd, void* stream);
int rh_layernorm_bwd_workspace_bytes(int64_t rows, int64_t dim, int64_t* bytes);
int rh_layernorm_bwd(int dtype, int64_t rows, int64_t dim, const void* dy, const void* x,
                     const float* mean, const float* rstd, const void* gamma,
                     const void* dresidual, void* dx, void* dgamma, void* dbeta, int accumulate,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* ---- elementwise ----------------------------------------------------------------
 * rh_gelu_fwd/bwd : F.gelu, approximate='none' (model.py:81, tp.py:247).
 * rh_add          : out = a + b, the residual add x + sublayer(.)
 *                   (model.py:95-96, tp.py:263,265) when not fused.
 * rh_scale_by     : x[r, c] *= *scalar for a [rows, cols] view with row
 *                   stride ld; a no-op when *scalar == 1 (device scalar, read
 *                   on the device).
 */
int rh_gelu_fwd(int dtype, int64_t n, const void* x, void* y, void* stream);
int rh_gelu_bwd(int dtype, int64_t n, const void* x, const void* dy, void* dx, void* stream);
int rh_add(int dtype, int64_t n, const void* a, const void* b, void* out, void* stream);
int rh_scale_by(int dtype, int64_t rows, int64_t cols, int64_t ld, void* x, const float* scalar,
                void* stream);

/* ---- optimizer steps ------------------------------------------------------------
 * rh_sgd_step   : p <- p - lr*(g + weight_decay*p)   (plain SGD; the cfg1 step)
 * rh_adamw_step : torch.optim.AdamW update with the reference's constants
 *                 (resihp/reference.py:20-38): decoupled decay
 *                 p *= 1 - lr*wd; m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g^2;
 *                 p -= (lr/bias_c1) * m / (sqrt(v)/sqrt(bias_c2) + eps).
 *                 exp_avg / exp_avg_sq have the parameter's dtype.
 */
int rh_sgd_step(int dtype, int64_t n, void* param, const void* grad, float lr,
                float weight_decay, void* stream);
int rh_adamw_step(int dtype, int64_t n, void* param, const void* grad, void* exp_avg,
                  void* exp_avg_sq, float lr, float beta1, float beta2, float eps,
                  float weight_decay, float bias_c1, float bias_c2, void* stream);

/* rh_adamw_multi : the same AdamW update for every tensor of a list -- the whole of
 *                  adamw(params).step() (resihp/reference.py:29-38; the stage optimizer
 *                  stepped once per iteration at resihp/parallel/pp.py:428-451) -- in one
 *                  launch per 64 tensors plus one single-workgroup launch that increments
 *                  the step counters.  Each tensor carries its own fp32 step counter in
 *                  device memory (torch's capturable form of state["step"]); the call adds
 *                  1 to it and forms the bias corrections 1 - beta^step on the device, in
 *                  double precision like torch's scalar arithmetic, so no host sync and no
 *                  host-side step value is needed.  Every tensor has `dtype` storage
 *                  (moments in the parameter's dtype); step counters must be distinct. */
typedef struct rh_adamw_tensor {
  void* param;
  const void* grad;
  void* exp_avg;
  void* exp_avg_sq;
  float* step;
  int64_t numel;
} rh_adamw_tensor;

int rh_adamw_multi(int dtype, int n_tensors, const rh_adamw_tensor* tensors, double lr, double beta1,
                   double beta2, double eps, double weight_decay, void* stream);

/* ---- next-token cross-entropy ---------------------------------------------------
 * Replaces next_token_loss = F.cross_entropy(logits[:, :-1].reshape(-1, V),
 * tokens[:, 1:].reshape(-1)) (resihp/reference.py:41-50; called at
 * resihp/parallel/pp.py:379-383) without materialising the shifted copy.
 * logits [batch, seq, vocab] with row stride ld (>= vocab); tokens int64
 * [batch, seq].  Rows s < seq-1 are scored against tokens[b, s+1]; the mean is
 * over N = batch*(seq-1) rows.  Outputs: row_lse [batch*seq] fp32 (log-sum-exp
 * of each row), loss [1] fp32 (the mean).  When dlogits != NULL the gradient
 * of the mean is written too:  (softmax - onehot)/N on scored rows, 0 on the
 * last position of every sequence and in pad columns [vocab, ld_d).
 * Token ids outside [0, vocab) are rejected on the device: the row's loss
 * becomes NaN.
 * rh_xent_bwd recomputes the same gradient scaled by *grad_loss.
 */
int rh_xent_workspace_bytes(int64_t batch, int64_t seq, int64_t* bytes);
int rh_xent_fwd(int dtype, int64_t batch, int64_t seq, int64_t vocab, const void* logits,
                int64_t ld, const int64_t* tokens, float* row_lse, float* loss, void* dlogits,
                int64_t ld_d, void* workspace, int64_t workspace_bytes, void* stream);
int rh_xent_bwd(int dtype, int64_t batch, int64_t seq, int64_t vocab, const void* logits,
                int64_t ld, const int64_t* tokens, const float* row_lse, const float* grad_loss,
                void* dlogits, int64_t ld_d, void* stream);

/* ---- LM head fused with the next-token cross-entropy -------------------------------
 * Replaces  logits = lm_head(final_norm(x))  (resihp/model.py:116,133; the vocab-parallel
 * head and its gather, resihp/parallel/tp.py:92-110,269-273) followed by next_token_loss
 * (resihp/reference.py:41-50), bf16 only, without materialising the [batch*seq, vocab]
 * logits or their gradient.  x [batch*seq, dim] (the final LayerNorm's output) and
 * W [vocab, dim] row-major, dim a multiple of 64; tokens int64 [batch, seq].
 * rh_lmhead_xent_fwd: loss [1] = mean over the batch*(seq-1) scored rows of
 *   lse - logit[target]; row_lse [batch*seq] (0 on each sequence's last position).  The
 *   GEMM's epilogue keeps only per-row (max, sum-exp) partials of each 64-column block.
 * rh_lmhead_xent_bwd: dx [batch*seq, dim] = dS . W and dW (+)= dS^T . x (accumulate != 0
 *   adds to dW, e.g. a parameter's .grad) for dS = (softmax - onehot) * *grad_loss / N,
 *   recomputing the logits vocabulary chunk by chunk (8192 ids): each chunk's dS lives in
 *   a reused workspace buffer, dx is summed over the chunks in fp32 and rounded once.
 * Workspace sizes come from rh_lmhead_xent_workspace_bytes (256-byte aligned). */
int rh_lmhead_xent_workspace_bytes(int64_t batch, int64_t seq, int64_t vocab, int64_t dim,
                                   int64_t* fwd_bytes, int64_t* bwd_bytes);
int rh_lmhead_xent_fwd(int64_t batch, int64_t seq, int64_t vocab, int64_t dim, const void* x,
                       const void* w, const int64_t* tokens, float* row_lse, float* loss,
                       void* workspace, int64_t workspace_bytes, void* stream);
int rh_lmhead_xent_bwd(int64_t batch, int64_t seq, int64_t vocab, int64_t dim, const void* x,
                       const void* w, const int64_t* tokens, const float* row_lse,
                       const float* grad_loss, void* dx, void* dw, int accumulate,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* ---- embeddings ------------------------------------------------------------------
 * Forward: out[b,s,:] = tok[ids[b,s] - vocab_start, :] (zero row when the id is
 * outside [vocab_start, vocab_start + vocab_rows): the vocab-parallel lookup
 * of resihp/parallel/tp.py:222-228) + pos[s, :] (pos may be NULL;
 * resihp/model.py:128-129, resihp/parallel/tp.py:256-257).
 * Backward: dtok[id - vocab_start] (+)= sum of dout rows with that id, and
 * dpos[s] (+)= sum over batch of dout[b, s].  Either gradient may be NULL.  Any
 * token count below 2^31: the rows of one id are summed in ascending token order
 * within chunks of 32 sorted rows and the chunk sums in chunk order, so the result
 * is deterministic (no atomics) and a heavily repeated id is summed in parallel.
 * The workspace holds the sort keys and fp32 chunk sums; its size depends on dim.
 */
int rh_embedding_fwd(int dtype, int64_t batch, int64_t seq, int64_t dim, const int64_t* tokens,
                     const void* tok, int64_t vocab_start, int64_t vocab_rows, const void* pos,
                     void* out, void* stream);
int rh_embedding_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t dim, int64_t* bytes);
int rh_embedding_bwd(int dtype, int64_t batch, int64_t seq, int64_t dim, const int64_t* tokens,
                     const void* dout, int64_t vocab_start, int64_t vocab_rows, void* dtok,
                     void* dpos, int accumulate, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* ---- TP re-slice (bit-exact byte movement) -----------------------------------------
 * rh_reshard_pack   : dst = torch.cat(src[0..n_src), dim=shard_dim)
 *                     (reconstruct_full, resihp/parallel/reshard.py:84-104; with
 *                     consecutive old shards this is the TP4->TP2 new shard
 *                     cat(old[2r], old[2r+1]) without building the full tensor).
 *                     dim 0: src i is [extent[i], cols], dst [sum extent, cols];
 *                     dim 1: src i is [rows, extent[i]], dst [rows, sum extent].
 * rh_reshard_unpack : dst[i] = torch.chunk(src, ., dim=shard_dim)[i].contiguous()
 *                     for the given extents (local_slice / shard_logical_state,
 *                     reshard.py:107-123).
 * Sources and destinations are contiguous; elem_bytes is the element size.
 * A NULL destination in rh_reshard_unpack skips that extent (so one call can
 * cut out a single new shard).
 *
 * rh_copy2d_batch   : n independent strided byte copies
 *                     dst[r*dst_ld + c] = src[r*src_ld + c], r < rows,
 *                     c < row_bytes -- the general re-slice for shard ranges
 *                     that straddle old shards (old_size % new_size != 0).
 */
typedef struct rh_copy2d {
  const void* src;
  void* dst;
  int64_t src_ld_bytes;
  int64_t dst_ld_bytes;
  int64_t rows;
  int64_t row_bytes;
} rh_copy2d;

int rh_copy2d_batch(const rh_copy2d* segs, int n, void* stream);
int rh_reshard_pack(const void* const* src, const int64_t* extent, int n_src, int64_t rows,
                    int64_t cols, int shard_dim, int64_t elem_bytes, void* dst, void* stream);
int rh_reshard_unpack(const void* src, int64_t rows, int64_t cols, int shard_dim,
                      int64_t elem_bytes, int n_dst, void* const* dst, const int64_t* extent,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RESIHP_HIP_H */
