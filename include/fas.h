/*
 * fas.h -- C ABI of the MI355X (gfx950) fused flash-attention-forward family
 * ("flash attention with scores").
 *
 * One entry point per launcher of the reference package.  Each takes the
 * shared attention description (fas_attn_args: q/k/v/out device pointers,
 * element strides, sizes, dtype, causal flag, softmax scale) plus the side
 * output of that variant, and enqueues its kernels asynchronously, in order,
 * on the given HIP stream.  Nothing here allocates or frees device memory:
 * every output and every workspace is owned by the caller, and no call
 * synchronises with the host.
 *
 * Conventions shared by every entry point (they restate the reference's
 * Triton launchers; citations are to the reference checkout):
 *   - q is (B, Hq, M, D); k and v are (B, Hk, N, D); out is like q.  Only the
 *     innermost stride must be 1 (flash.py:23-26, maybe_contiguous); rows
 *     must be 16-byte aligned (pointer and strides[0..2] multiples of 8),
 *     and one (batch, head) slice of any tensor must span < 2^31 bytes.
 *   - D in {16, 32, 64, 128}, Hq % Hk == 0; query head h reads KV head
 *     h / (Hq/Hk) (attention_with_scores.py:57).
 *   - Causal masking keeps (i, j) iff (N - M) + i >= j (bottom-right
 *     aligned, attention_with_scores.py:136) except in the cross-token
 *     QK-sum, which keeps i >= j (attention_cross_token_qk_sum.py:138).
 *   - Softmax is computed in base 2 on raw scores with
 *     qk_scale = sm_scale * log2(e) (attention_with_scores.py:53-54,165-183).
 *   - Query rows with no admissible key (causal, M > N) produce out = 0 and
 *     zero sums (attention_with_scores.py:192-195).
 *   - Column-type sums are per KV head: the Hq/Hk query heads of a group are
 *     folded into one (B, Hk, *) vector (attention_with_col_sum.py:72,370).
 *   - Every element of every output is written by the call; outputs need no
 *     zero-fill (the reference zero-fills with torch.zeros).
 *   - Column sums are deterministic: each column is reduced by one
 *     workgroup in a fixed order (the reference uses fp32 atomics).
 *   - Short query ranges against long key ranges (fewer row blocks than the
 *     chip has CUs) split each row block's keys over several workgroups;
 *     the variants whose forward can split then need a workspace for the
 *     fp32 partials, which fas_workspace_bytes includes.
 *
 * Return value: FAS_OK (0) or a negative fas_status; fas_last_error() then
 * returns a thread-local message naming the entry point and the cause.
 */
#ifndef FAS_H_
#define FAS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAS_ABI_VERSION 8

typedef enum fas_dtype {
  FAS_DTYPE_F16 = 0,
  FAS_DTYPE_BF16 = 1
} fas_dtype;

typedef enum fas_status {
  FAS_OK = 0,
  FAS_ERR_INVALID = -1,     /* bad shape, pointer, stride or alignment */
  FAS_ERR_UNSUPPORTED = -2, /* valid request this build does not implement */
  FAS_ERR_WORKSPACE = -3,   /* caller-provided workspace too small */
  FAS_ERR_HIP = -4          /* the HIP runtime rejected a launch */
} fas_status;

/* Variant selector for fas_workspace_bytes. */
typedef enum fas_variant {
  FAS_VARIANT_SCORES = 0,
  FAS_VARIANT_ROW_SUM = 1,
  FAS_VARIANT_COL_SUM = 2,
  FAS_VARIANT_COL_SUM_SEQUENTIAL = 3,
  FAS_VARIANT_SOFTMAX_COL_SUM = 4,
  FAS_VARIANT_CROSS_QK_SUM = 5,
  FAS_VARIANT_CROSS_SOFTMAX_SUM = 6,
  FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED = 7,
  FAS_VARIANT_ATTENTION_BACKWARD = 8,
  FAS_VARIANT_ATTENTION_FORWARD = 9,
  /* Not a workspace: the size of the keep_bits buffer below. */
  FAS_VARIANT_KEEP_BITS = 10
} fas_variant;

/* The attention problem shared by every entry point.  Strides are in
 * elements, ordered (batch, head, row, dim); stride[3] must be 1. */
typedef struct fas_attn_args {
  int32_t dtype;   /* fas_dtype of q, k, v and out */
  int32_t causal;  /* 0 or 1 */
  float sm_scale;  /* softmax scale applied to q.k (1/sqrt(D) by default) */
  int32_t reserved;
  int64_t batch, heads_q, heads_k, seqlen_q, seqlen_k, head_dim;
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  /* Dropout of the attention weights, 0 <= dropout_p < 1 (0: none).  With
   * the reference's random stream: element (b, h, i, j) is kept iff
   * Triton's tl.rand(dropout_seed, dropout_offset + ((b*Hq + h)*M + i)*N
   * + j, n_rounds=6) > dropout_p, the index taken mod 2^32
   * (attention_with_scores.py:70-75, 173-176); seed and offset are the pair
   * dropout.py:5-15 takes from the device generator.  Weights are dropped
   * after the row normaliser has summed them.  Which outputs see the mask
   * follows the reference entry point by entry point: O everywhere
   * (rescaled by 1/(1 - dropout_p) only by fas_attention_with_scores and
   * fas_attention_forward), the column sums of
   * fas_attention_with_softmax_col_sum, nothing else.  The buffered cross
   * softmax sum, the scores-only call, the total attention and the score and
   * raw-sum outputs ignore it.  Offsets >= 2^31 with B*Hq*M*N >= 2^31 return
   * FAS_ERR_UNSUPPORTED.  fas_attention_backward takes the forward's dropout
   * fields and regenerates the same mask, or reads it from keep_bits. */
  float dropout_p;
  int32_t reserved2;
  uint64_t dropout_seed;
  uint64_t dropout_offset;
  /* Optional, with dropout: a device buffer of
   * fas_workspace_bytes(FAS_VARIANT_KEEP_BITS, ...) bytes, 256-byte aligned,
   * owned by the caller.  fas_attention_forward stores the mask in it (one
   * bit per pair, key-major for the dK/dV kernel, plus row blocks for the
   * dQ kernel that recomputes S and dP when the backward cannot store dS);
   * fas_attention_backward given the same buffer and dropout fields reads
   * it instead of evaluating the random stream again.  NULL: both evaluate
   * the stream.  The other entry points ignore it.  This build's own
   * addition: the reference's backward regenerates the mask. */
  void* keep_bits;
} fas_attn_args;

int fas_abi_version(void);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* fas_last_error(void);

/* Device workspace (bytes, 256-byte aligned) an entry point of `variant`
 * needs for this problem; 0 when it needs none.  split is ignored by the
 * variants without one, except FAS_VARIANT_ATTENTION_BACKWARD: there a
 * nonzero split asks for the size without the stored dS (the smallest
 * workspace the backward accepts).  Returns (size_t)-1 for an invalid
 * request. */
size_t fas_workspace_bytes(int variant, const fas_attn_args* a, int64_t split);

/* Replaces attention_with_scores.py:214-333 (+ _fwd_kernel_with_scores
 * :23-211).  scores is (B, Hq, M, N) in the input dtype with element strides
 * scores_stride (innermost 1); it receives (q.k) * sm_scale, with masked
 * positions (causal, upper triangle) written as 0 by the kernel itself.
 * Workspace: fas_workspace_bytes(FAS_VARIANT_SCORES, ...), non-zero only
 * for short query ranges, which run the key-split forward plus the
 * scores-only kernel instead of the fused writer. */
int fas_attention_with_scores(const fas_attn_args* a, void* scores,
                              const int64_t scores_stride[4], void* workspace,
                              size_t workspace_bytes, void* stream);

/* Replaces attention_scores.py:154-223 (compute_attention_scores + kernel
 * :55-151): scores (B, Hq, M, N) in the input dtype receives
 * (q . k) * sm_scale for every pair, with no mask (the reference ignores
 * causal there).  Only a->q and a->k are read. */
int fas_attention_scores(const fas_attn_args* a, void* scores, const int64_t scores_stride[4],
                         void* stream);

/* Replaces attention_with_row_sum.py:204-326 (+ kernel :22-202).
 * row_sum is (B, Hq, M) fp32: sum over admissible keys of (q.k)*sm_scale.
 * The workspace (fas_workspace_bytes(FAS_VARIANT_ROW_SUM, ...), often 0)
 * holds key-split partials for short query ranges. */
int fas_attention_with_row_sum(const fas_attn_args* a, float* row_sum,
                               const int64_t row_sum_stride[3], void* workspace,
                               size_t workspace_bytes, void* stream);

/* Replaces attention_with_col_sum.py:297-419 (+ kernel :22-294): col_sum is
 * (B, Hk, N) fp32, sum over admissible queries and group heads of
 * (q.k)*sm_scale.  The reference's reverse / round-robin key orders only
 * change its atomic summation order; this result is order-independent. */
int fas_attention_with_col_sum(const fas_attn_args* a, float* col_sum,
                               const int64_t col_sum_stride[3], void* workspace,
                               size_t workspace_bytes, void* stream);

/* Replaces attention_with_col_sum_sequential.py:214-341 (+ kernel :23-211):
 * same output as fas_attention_with_col_sum. */
int fas_attention_with_col_sum_sequential(const fas_attn_args* a, float* col_sum,
                                          const int64_t col_sum_stride[3], void* workspace,
                                          size_t workspace_bytes, void* stream);

/* Replaces attention_with_col_softmax_sum.py:274-401 (+ kernel :23-270):
 * col_sum is (B, Hk, N) fp32, sum over queries and group heads of the final
 * softmax weights P = exp(s - m) / l.  Second pass key-block outer. */
int fas_attention_with_softmax_col_sum(const fas_attn_args* a, float* col_sum,
                                       const int64_t col_sum_stride[3], void* workspace,
                                       size_t workspace_bytes, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same computation and kernels as
 * fas_attention_with_softmax_col_sum, with the workspace taken from a
 * file-scope device array of the library instead of a caller buffer.  The
 * caller still passes the inputs and outputs; nothing is allocated or freed,
 * here or in any library routine this call makes.
 * Limits: the array holds 64 MiB per GPU (B*Hq*M*4 bytes of row normalizers,
 * + B*Hq*N*4 of group partials when Hq > Hk, + key-split partials, which
 * shrink to fit); larger problems return FAS_ERR_WORKSPACE.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller.
 * No part of the array needs to start at zero; each call writes what it
 * reads. */
int fas_attention_with_softmax_col_sum_noalloc(const fas_attn_args* a, float* col_sum,
                                               const int64_t col_sum_stride[3], void* stream);

/* Replaces attention_cross_token_qk_sum.py:255-408 (+ kernel :17-252):
 * cross is (B, Hk, split) fp32, sum over queries i >= split of (q.k)*sm_scale
 * for keys j < split.  Causal masking here (and for out) is top-left:
 * i >= j.  0 < split <= N. */
int fas_attention_cross_token_qk_sum(const fas_attn_args* a, int64_t split, float* cross,
                                     const int64_t cross_stride[3], void* workspace,
                                     size_t workspace_bytes, void* stream);

/* Replaces attention_cross_token_softmax_sum.py:735-863 (+ fused kernel
 * :24-268): cross is (B, Hk, split) fp32, sum over queries i >= split of the
 * softmax weights exp(s - m) / (l + 1e-12) for keys j < split. */
int fas_attention_cross_token_softmax_sum(const fas_attn_args* a, int64_t split, float* cross,
                                          const int64_t cross_stride[3], void* workspace,
                                          size_t workspace_bytes, void* stream);

/* Replaces attention_cross_token_softmax_sum.py:639-732 (+ buffered kernel
 * :434-636): same output as fas_attention_cross_token_softmax_sum, but the
 * first pass stores the scores of the region (rows >= split, keys < split)
 * in the workspace and the second pass reloads them instead of recomputing
 * q.k.  The reference keeps raw fp32 scores in a B*Hq*M*N*4-byte buffer
 * (attention_cross_token_softmax_sum.py:704-705); only the region is ever
 * re-read, so only it is kept, as fp16 base-2 exponents relative to each
 * row's maximum over the region keys of a 64-key tile plus that maximum:
 * B*Hq*(M - split)*(split*2 + ceil(split/64)*4) bytes. */
int fas_attention_cross_token_softmax_sum_buffered(const fas_attn_args* a, int64_t split,
                                                   float* cross, const int64_t cross_stride[3],
                                                   void* workspace, size_t workspace_bytes,
                                                   void* stream);

/* Replaces the forward half of flash.py:264-297 (attention ->
 * FlashAttention.forward :34-170, _fwd_kernel :335-500), with dropout as
 * fas_attn_args describes (flash.py:459-466, 488-491):
 * out = softmax(mask(q k^T sm_scale)) v, and lse (B, Hq, M) fp32 with
 * element strides lse_stride receives the natural-log normalizer
 * m * sm_scale + ln(l), -inf for rows that see no key (flash.py:477-483).
 * Causal masking is bottom-right, as everywhere but the cross QK sum.  The
 * workspace is fas_workspace_bytes(FAS_VARIANT_ATTENTION_FORWARD, ...). */
int fas_attention_forward(const fas_attn_args* a, float* lse, const int64_t lse_stride[3],
                          void* workspace, size_t workspace_bytes, void* stream);

/* Replaces total.py:9-48 (+ _total_attention_kernel :51-143), which
 * flash.py:141-156 runs for return_total_attention: total (B, Hq, N) fp32
 * receives, per query head and key, the sum over query rows of the softmax
 * weights exp(q.k * sm_scale - lse) of the admissible pairs.  lse is a
 * normalizer as fas_attention_forward writes it.  Only a->q and a->k are
 * read (a->v and a->out may be NULL). */
int fas_total_attention(const fas_attn_args* a, const float* lse, const int64_t lse_stride[3],
                        float* total, const int64_t total_stride[3], void* stream);

/* Replaces FlashAttention.backward (flash.py:172-261, kernels :532-918)
 * with the forward's dropout (flash.py:653-731, 843-895).  a->out is the
 * forward output O and lse its normalizer;
 * dout is dL/dO (shaped like out).  Writes dq (like q) and dk, dv
 * (B, Hk, N, D) in the input dtype, dk and dv summed over the Hq/Hk query
 * heads of each KV head.  The full workspace, fas_workspace_bytes(
 * FAS_VARIANT_ATTENTION_BACKWARD, a, 0), includes dS in the input dtype for
 * every 32 x 32 block of (query, key) pairs that holds a visible pair (2 KiB
 * per block, rows padded to Mpad = M rounded up to 128; about B*Hq*M*N bytes
 * causal): the dK/dV kernel stores it and the dQ kernel reads it instead of
 * recomputing S and dP.  It is left out when it would pass 16 GiB or 2 GiB
 * in one head, or when the workspace given is smaller than the full size but
 * at least fas_workspace_bytes(FAS_VARIANT_ATTENTION_BACKWARD, a, 1); dk and
 * dv are the same bits either way, dq agrees within rounding.  Without the
 * stored dS, with dropout and no keep_bits, that smaller size includes
 * B*Hq*Mpad*ceil(N/32)*4 bytes (256-byte aligned) of keep bits passed from
 * the dK/dV kernel to the dQ kernel; a workspace short of them (at least the
 * rest) makes both kernels evaluate the random stream, with the same
 * result. */
int fas_attention_backward(const fas_attn_args* a, const void* dout,
                           const int64_t dout_stride[4], const float* lse,
                           const int64_t lse_stride[3], void* dq, const int64_t dq_stride[4],
                           void* dk, const int64_t dk_stride[4], void* dv,
                           const int64_t dv_stride[4], void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAS_H_ */
