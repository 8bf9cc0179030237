// C ABI of the gfx950 fused attention family (declared in include/fas.h).
//
// Validates a request, packs the kernel parameter block and enqueues the
// launches on the caller's stream.  No device memory is allocated here and
// nothing is synchronised.
#include "fas.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "fas_launch.hpp"
#include "fas_params.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fn, const char* fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  g_last_error = std::string(fn) + ": " + msg;
  return code;
}

int hip_status(const char* fn, hipError_t e) {
  if (e == hipSuccess) return FAS_OK;
  return fail(FAS_ERR_HIP, fn, "HIP launch failed: %s", hipGetErrorString(e));
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Checks one (B, H, L, D)-shaped 16-bit tensor: innermost stride 1 and
// 16-byte aligned rows, which the kernels' vector loads/stores require.
int check_tensor(const char* fn, const char* name, const void* ptr, const int64_t* st) {
  if (ptr == nullptr) return fail(FAS_ERR_INVALID, fn, "%s is NULL", name);
  if (st[3] != 1) return fail(FAS_ERR_INVALID, fn, "%s innermost stride must be 1 (got %lld)", name,
                              (long long)st[3]);
  if (!aligned16(ptr) || st[0] % 8 || st[1] % 8 || st[2] % 8)
    return fail(FAS_ERR_INVALID, fn,
                "%s rows must be 16-byte aligned (pointer and outer strides multiples of 8 elements)",
                name);
  return FAS_OK;
}

// Fills the fields of the parameter block common to every variant.
// top_left selects the cross-token QK-sum's causal alignment (i >= j)
// instead of the bottom-right one ((N - M) + i >= j) used elsewhere.
int fill_common(const char* fn, const fas_attn_args* a, fas::KParams* p, bool top_left) {
  if (a == nullptr) return fail(FAS_ERR_INVALID, fn, "args is NULL");
  if (a->dtype != FAS_DTYPE_F16 && a->dtype != FAS_DTYPE_BF16)
    return fail(FAS_ERR_UNSUPPORTED, fn, "dtype %d is not fp16 (0) or bf16 (1)", (int)a->dtype);
  if (a->causal != 0 && a->causal != 1)
    return fail(FAS_ERR_INVALID, fn, "causal must be 0 or 1");
  const int64_t D = a->head_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail(FAS_ERR_UNSUPPORTED, fn, "head_dim %lld not in {16, 32, 64, 128}", (long long)D);
  if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_k < 0 || a->heads_q <= 0 || a->heads_k <= 0)
    return fail(FAS_ERR_INVALID, fn, "negative or zero size");
  if (a->heads_q % a->heads_k != 0)
    return fail(FAS_ERR_INVALID, fn, "heads_q (%lld) is not a multiple of heads_k (%lld)",
                (long long)a->heads_q, (long long)a->heads_k);
  if (a->seqlen_q > (1 << 30) || a->seqlen_k > (1 << 30) || a->batch * a->heads_q > (1 << 30))
    return fail(FAS_ERR_UNSUPPORTED, fn, "sizes exceed the 32-bit index range of the kernels");
  if (!std::isfinite(a->sm_scale)) return fail(FAS_ERR_INVALID, fn, "sm_scale is not finite");
  const int64_t nrb = (a->seqlen_q + fas::kBMHost - 1) / fas::kBMHost;
  if (nrb * a->batch * a->heads_q > 0xffffffffLL)
    return fail(FAS_ERR_UNSUPPORTED, fn, "grid too large");

  *p = fas::KParams{};
  p->q = static_cast<const uint16_t*>(a->q);
  p->k = static_cast<const uint16_t*>(a->k);
  p->v = static_cast<const uint16_t*>(a->v);
  p->o = static_cast<uint16_t*>(a->out);
  p->lse = a->lse;
  p->sq0 = a->q_stride[0]; p->sq1 = a->q_stride[1]; p->sq2 = a->q_stride[2];
  p->sk0 = a->k_stride[0]; p->sk1 = a->k_stride[1]; p->sk2 = a->k_stride[2];
  p->sv0 = a->v_stride[0]; p->sv1 = a->v_stride[1]; p->sv2 = a->v_stride[2];
  p->so0 = a->out_stride[0]; p->so1 = a->out_stride[1]; p->so2 = a->out_stride[2];
  p->sl0 = a->lse_stride[0]; p->sl1 = a->lse_stride[1]; p->sl2 = a->lse_stride[2];
  p->B = (int)a->batch;
  p->H = (int)a->heads_q;
  p->G = (int)(a->heads_q / a->heads_k);
  p->M = (int)a->seqlen_q;
  p->N = (int)a->seqlen_k;
  p->split = 0;
  p->causal = a->causal;
  p->causal_off = top_left ? 0 : (int)(a->seqlen_k - a->seqlen_q);
  p->order = fas::kOrderForward;
  p->order2 = fas::kOrderForward;
  p->nrb = (int)nrb;
  p->sm_scale = a->sm_scale;
  p->qk_scale = (float)((double)a->sm_scale * 1.4426950408889634);

  if (a->batch * a->heads_q * a->seqlen_q == 0) return FAS_OK;  // nothing to read
  int rc;
  if ((rc = check_tensor(fn, "q", a->q, a->q_stride))) return rc;
  if ((rc = check_tensor(fn, "out", a->out, a->out_stride))) return rc;
  if (a->seqlen_k > 0) {
    if ((rc = check_tensor(fn, "k", a->k, a->k_stride))) return rc;
    if ((rc = check_tensor(fn, "v", a->v, a->v_stride))) return rc;
  }
  return FAS_OK;
}

bool empty_launch(const fas::KParams& p) { return (int64_t)p.B * p.H * p.M == 0; }

int set_aux(const char* fn, fas::KParams* p, float* aux, const int64_t* st, const char* name) {
  if (aux == nullptr) return fail(FAS_ERR_INVALID, fn, "%s is NULL", name);
  if (st == nullptr) return fail(FAS_ERR_INVALID, fn, "%s strides are NULL", name);
  p->aux = aux;
  p->sa0 = st[0];
  p->sa1 = st[1];
  p->sa2 = st[2];
  return FAS_OK;
}

int zero_aux(const char* fn, const fas::KParams& p, int64_t n1, int64_t n2, hipStream_t s) {
  return hip_status(fn, fas::launch_fill_zero(p.aux, p.sa0, p.sa1, p.sa2, p.B, n1, n2, s));
}

int check_split(const char* fn, const fas_attn_args* a, int64_t split) {
  if (!(split > 0 && split <= a->seqlen_k))
    return fail(FAS_ERR_INVALID, fn, "split %lld outside (0, %lld]", (long long)split,
                (long long)a->seqlen_k);
  return FAS_OK;
}

using Launcher = hipError_t (*)(const fas::KParams&, int, int, hipStream_t);

// Column-type sum over (B, Hk, n2): zero, then launch.
int run_col(const char* fn, const fas_attn_args* a, float* out, const int64_t* st, int64_t n2,
            fas::KParams* p, Launcher launch, void* stream) {
  int rc;
  if ((rc = set_aux(fn, p, out, st, "sum output"))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = zero_aux(fn, *p, a->heads_k, n2, s))) return rc;
  if (empty_launch(*p)) return FAS_OK;
  return hip_status(fn, launch(*p, a->dtype, (int)a->head_dim, s));
}

}  // namespace

extern "C" {

int fas_abi_version(void) { return FAS_ABI_VERSION; }

const char* fas_last_error(void) { return g_last_error.c_str(); }

int fas_attention_with_scores(const fas_attn_args* a, void* scores, const int64_t scores_stride[4],
                              void* stream) {
  static const char* fn = "fas_attention_with_scores";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  if (empty_launch(p) || a->seqlen_k == 0) return FAS_OK;
  if (scores == nullptr || scores_stride == nullptr)
    return fail(FAS_ERR_INVALID, fn, "scores is NULL");
  if (scores_stride[3] != 1) return fail(FAS_ERR_INVALID, fn, "scores innermost stride must be 1");
  if (reinterpret_cast<uintptr_t>(scores) & 1u)
    return fail(FAS_ERR_INVALID, fn, "scores is not 2-byte aligned");
  p.scores = static_cast<uint16_t*>(scores);
  p.ss0 = scores_stride[0];
  p.ss1 = scores_stride[1];
  p.ss2 = scores_stride[2];
  p.vec_scores = aligned16(scores) && p.ss0 % 8 == 0 && p.ss1 % 8 == 0 && p.ss2 % 8 == 0;
  return hip_status(fn, fas::launch_scores(p, a->dtype, (int)a->head_dim,
                                           static_cast<hipStream_t>(stream)));
}

int fas_attention_with_row_sum(const fas_attn_args* a, float* row_sum, const int64_t st[3],
                               void* stream) {
  static const char* fn = "fas_attention_with_row_sum";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  if (empty_launch(p)) return FAS_OK;
  if ((rc = set_aux(fn, &p, row_sum, st, "row_sum"))) return rc;
  // Every row is written by the kernel; no zero-fill needed.
  return hip_status(fn, fas::launch_row_sum(p, a->dtype, (int)a->head_dim,
                                            static_cast<hipStream_t>(stream)));
}

int fas_attention_with_col_sum(const fas_attn_args* a, float* col_sum, const int64_t st[3],
                               void* stream) {
  static const char* fn = "fas_attention_with_col_sum";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  p.order = a->causal ? fas::kOrderReverse : fas::kOrderRoundRobin;
  return run_col(fn, a, col_sum, st, a->seqlen_k, &p, fas::launch_col_sum, stream);
}

int fas_attention_with_col_sum_sequential(const fas_attn_args* a, float* col_sum,
                                          const int64_t st[3], void* stream) {
  static const char* fn = "fas_attention_with_col_sum_sequential";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  p.order = fas::kOrderRoundRobin;
  return run_col(fn, a, col_sum, st, a->seqlen_k, &p, fas::launch_col_sum, stream);
}

int fas_attention_with_softmax_col_sum(const fas_attn_args* a, float* col_sum, const int64_t st[3],
                                       void* stream) {
  static const char* fn = "fas_attention_with_softmax_col_sum";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  p.order = fas::kOrderRoundRobin;
  p.order2 = a->causal ? fas::kOrderReverse : fas::kOrderRoundRobin;
  return run_col(fn, a, col_sum, st, a->seqlen_k, &p, fas::launch_col_softmax, stream);
}

int fas_attention_cross_token_qk_sum(const fas_attn_args* a, int64_t split, float* cross,
                                     const int64_t st[3], void* stream) {
  static const char* fn = "fas_attention_cross_token_qk_sum";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, true))) return rc;
  if ((rc = check_split(fn, a, split))) return rc;
  p.split = (int)split;
  return run_col(fn, a, cross, st, split, &p, fas::launch_cross_qk, stream);
}

int fas_attention_cross_token_softmax_sum(const fas_attn_args* a, int64_t split, float* cross,
                                          const int64_t st[3], void* stream) {
  static const char* fn = "fas_attention_cross_token_softmax_sum";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  if ((rc = check_split(fn, a, split))) return rc;
  p.split = (int)split;
  p.order = fas::kOrderRoundRobin;
  return run_col(fn, a, cross, st, split, &p, fas::launch_cross_softmax, stream);
}

size_t fas_cross_token_softmax_sum_buffered_workspace_bytes(const fas_attn_args* a, int64_t split) {
  if (a == nullptr || split <= 0) return 0;
  const int64_t rows = a->seqlen_q > split ? a->seqlen_q - split : 0;
  return (size_t)(a->batch * a->heads_q * rows * split) * sizeof(float);
}

int fas_attention_cross_token_softmax_sum_buffered(const fas_attn_args* a, int64_t split,
                                                   float* cross, const int64_t st[3],
                                                   void* workspace, size_t workspace_bytes,
                                                   void* stream) {
  static const char* fn = "fas_attention_cross_token_softmax_sum_buffered";
  fas::KParams p;
  int rc;
  if ((rc = fill_common(fn, a, &p, false))) return rc;
  if ((rc = check_split(fn, a, split))) return rc;
  p.split = (int)split;
  const size_t need = fas_cross_token_softmax_sum_buffered_workspace_bytes(a, split);
  if (need > 0) {
    if (workspace == nullptr || workspace_bytes < need)
      return fail(FAS_ERR_WORKSPACE, fn, "workspace of %zu bytes needed, %zu given", need,
                  workspace_bytes);
    if (!aligned16(workspace)) return fail(FAS_ERR_INVALID, fn, "workspace not 16-byte aligned");
  }
  const int64_t rows = a->seqlen_q > split ? a->seqlen_q - split : 0;
  p.buf = static_cast<float*>(workspace);
  p.sb2 = split;
  p.sb1 = rows * split;
  p.sb0 = a->heads_q * rows * split;
  return run_col(fn, a, cross, st, split, &p, fas::launch_cross_softmax_buf, stream);
}

}  // extern "C"
