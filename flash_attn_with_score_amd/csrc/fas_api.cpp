// C ABI of the gfx950 fused attention family (declared in include/fas.h).
//
// Validates a request, packs the kernel parameter blocks and enqueues the
// launches on the caller's stream.  No device memory is allocated here and
// nothing is synchronised.
#include "fas.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <vector>
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

constexpr int64_t kMaxSliceBytes = (int64_t)1 << 31;
// Largest batch or head stride (elements): 2^46 two-byte elements span 128
// TiB, beyond any device's address space, and keep every offset product of
// the kernels (index * stride, index < 2^24) inside int64.
constexpr int64_t kMaxOuterStride = (int64_t)1 << 46;

// Checks one (B, H, L, D)-shaped 16-bit tensor: innermost stride 1, 16-byte
// aligned rows, and a (batch, head) slice addressable with 32-bit offsets
// (including the tile overhang the kernels read past the last row).  Each
// bound is tested before the product that uses it, so no arithmetic here
// can overflow whatever strides the caller passes.
int check_tensor(const char* fn, const char* name, const void* ptr, const int64_t* st, int64_t rows,
                 int64_t D) {
  if (ptr == nullptr) return fail(FAS_ERR_INVALID, fn, "%s is NULL", name);
  if (st[3] != 1)
    return fail(FAS_ERR_INVALID, fn, "%s innermost stride must be 1 (got %lld)", name,
                (long long)st[3]);
  if (st[0] < 0 || st[1] < 0 || st[2] < 0)
    return fail(FAS_ERR_INVALID, fn, "%s has a negative stride", name);
  if (!aligned16(ptr) || st[0] % 8 || st[1] % 8 || st[2] % 8)
    return fail(FAS_ERR_INVALID, fn,
                "%s rows must be 16-byte aligned (pointer and outer strides multiples of 8)", name);
  if (st[2] < D) return fail(FAS_ERR_INVALID, fn, "%s rows overlap (row stride < head_dim)", name);
  if (st[0] >= kMaxOuterStride || st[1] >= kMaxOuterStride)
    return fail(FAS_ERR_UNSUPPORTED, fn, "%s batch or head stride exceeds 2^46 elements", name);
  // rows <= 2^28 (check_shape), so with st[2] < 2^31 the product fits.
  if (st[2] >= kMaxSliceBytes || (rows + 512) * st[2] * 2 >= kMaxSliceBytes)
    return fail(FAS_ERR_UNSUPPORTED, fn, "%s (batch, head) slice exceeds 2 GiB", name);
  return FAS_OK;
}

// Compute units of the current device (cached per device; 256 if the query
// fails).
int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((size_t)dev >= cache.size()) cache.resize((size_t)dev + 1, 0);
  if (cache[(size_t)dev] == 0) {
    int n = 0;
    cache[(size_t)dev] =
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
            ? n
            : 256;
  }
  return cache[(size_t)dev];
}

uint32_t slice_bytes(int64_t rows, int64_t row_stride, int64_t D) {
  return rows <= 0 ? 0u : (uint32_t)(((rows - 1) * row_stride + D) * 2);
}

struct Problem {
  int B, H, Hk, G, M, N, D, dtype, causal;
  bool dropout;  // dropout_p > 0
  bool keep;     // dropout with a caller keep-bit buffer (fas_attn_args.keep_bits)
  float sm_scale;
  int pack;  // query heads per forward workgroup (GQA packing): G, or 1
};

// Bytes a 16-bit (B, H, L, D) tensor spans over `heads` consecutive heads of
// one batch entry, including the tile overhang the kernels may address past
// the last row.
int64_t head_span_bytes(const int64_t* st, int64_t heads, int64_t rows) {
  return ((heads - 1) * st[1] + (rows + 512) * st[2]) * 2;
}

// GQA packing: a forward workgroup serves all G query heads of a KV head
// when the G heads of q and out can be addressed with 32-bit offsets from
// the first (the kernels mark invalid rows with offset 2^31).
int choose_pack(const fas_attn_args* a, int G, int M) {
  // Launches with dropout keep one head per workgroup (no packed dropout
  // instances are built).
  if (G <= 1 || a->dropout_p > 0.f) return 1;
  if (head_span_bytes(a->q_stride, G, M) >= kMaxSliceBytes ||
      head_span_bytes(a->out_stride, G, M) >= kMaxSliceBytes)
    return 1;
  return G;
}

// Sizes, dtype and flags only (no pointers): enough to size a workspace.
int check_shape(const char* fn, const fas_attn_args* a, Problem* pr) {
  if (a == nullptr) return fail(FAS_ERR_INVALID, fn, "args is NULL");
  if (a->dtype != FAS_DTYPE_F16 && a->dtype != FAS_DTYPE_BF16)
    return fail(FAS_ERR_UNSUPPORTED, fn, "dtype %d is not fp16 (0) or bf16 (1)", (int)a->dtype);
  if (a->causal != 0 && a->causal != 1) return fail(FAS_ERR_INVALID, fn, "causal must be 0 or 1");
  const int64_t D = a->head_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail(FAS_ERR_UNSUPPORTED, fn, "head_dim %lld not in {16, 32, 64, 128}", (long long)D);
  if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_k < 0 || a->heads_q <= 0 || a->heads_k <= 0)
    return fail(FAS_ERR_INVALID, fn, "negative or zero size");
  if (a->heads_q % a->heads_k != 0)
    return fail(FAS_ERR_INVALID, fn, "heads_q (%lld) is not a multiple of heads_k (%lld)",
                (long long)a->heads_q, (long long)a->heads_k);
  // Bounds that keep every index of the kernels inside 32 bits and every
  // size and offset product of the host code inside 64 (heads_q is tested
  // alone first so that batch * heads_q cannot overflow).
  if (a->seqlen_q > (1 << 28) || a->seqlen_k > (1 << 28) || a->heads_q > (1 << 24) ||
      a->batch > (1 << 24) || a->batch * a->heads_q > (1 << 24))
    return fail(FAS_ERR_UNSUPPORTED, fn, "sizes exceed the index range of the kernels");
  // The largest workspace term is 4 bytes per (query, key) pair (the
  // buffered cross softmax sum's region): past 2^58 pairs its size would
  // not fit a size_t.
  if ((unsigned __int128)a->batch * a->heads_q * a->seqlen_q * a->seqlen_k >
      ((unsigned __int128)1 << 58))
    return fail(FAS_ERR_UNSUPPORTED, fn, "B*Hq*M*N exceeds 2^58 (query, key) pairs");
  if (!std::isfinite(a->sm_scale)) return fail(FAS_ERR_INVALID, fn, "sm_scale is not finite");
  if (!(a->dropout_p >= 0.f && a->dropout_p < 1.f))
    return fail(FAS_ERR_INVALID, fn, "dropout_p %g outside [0, 1)", (double)a->dropout_p);
  if (a->dropout_p > 0.f && a->dropout_offset >= (1ull << 31) &&
      (uint64_t)a->batch * a->heads_q * a->seqlen_q * a->seqlen_k >= (1ull << 31))
    return fail(FAS_ERR_UNSUPPORTED, fn,
                "dropout offset >= 2^31 with B*Hq*M*N >= 2^31 (the reference's element "
                "index then depends on its block sizes)");
  pr->B = (int)a->batch;
  pr->H = (int)a->heads_q;
  pr->Hk = (int)a->heads_k;
  pr->G = pr->H / pr->Hk;
  pr->M = (int)a->seqlen_q;
  pr->N = (int)a->seqlen_k;
  pr->D = (int)D;
  pr->dtype = a->dtype;
  pr->causal = a->causal;
  pr->dropout = a->dropout_p > 0.f;
  pr->keep = pr->dropout && a->keep_bits != nullptr;
  pr->sm_scale = a->sm_scale;
  pr->pack = choose_pack(a, pr->G, pr->M);
  return FAS_OK;
}

int check_args(const char* fn, const fas_attn_args* a, Problem* pr) {
  int rc;
  if ((rc = check_shape(fn, a, pr))) return rc;
  const int64_t D = pr->D;
  if ((int64_t)pr->B * pr->H * pr->M == 0) return FAS_OK;  // nothing is read
  if ((rc = check_tensor(fn, "q", a->q, a->q_stride, pr->M, D))) return rc;
  if ((rc = check_tensor(fn, "out", a->out, a->out_stride, pr->M, D))) return rc;
  if (pr->N > 0) {
    if ((rc = check_tensor(fn, "k", a->k, a->k_stride, pr->N, D))) return rc;
    if ((rc = check_tensor(fn, "v", a->v, a->v_stride, pr->N, D))) return rc;
  }
  return FAS_OK;
}

// Exponent scale of the base-2 softmax, |sm_scale| * log2(e).  For
// sm_scale == 0 the weights are uniform over the admissible keys; a zero
// scale would turn the masked scores' -inf into NaN (-inf * 0) and the
// column pass's starting value -lse2 / qk_scale into a division by zero, so
// a tiny positive scale stands in: finite scores then contribute exp2(~0) = 1
// exactly in fp32, masked ones exp2(-inf) = 0.
float qk_scale_of(float sm_scale) {
  if (sm_scale == 0.f) return 1e-30f;
  return (float)((double)std::fabs(sm_scale) * 1.4426950408889634);
}

// Dropout threshold: the largest y in [0, 2^31 - 1] whose uniform
// float(y) * 4.6566127342e-10 (Triton's uint_to_uniform_float, fp32) is
// <= p, so that "u > p" is "y > thresh".  u is non-decreasing in y.
int32_t dropout_thresh(float p) {
  auto u = [](int64_t y) { return (float)y * 4.6566127342e-10f; };
  int64_t lo = 0, hi = INT32_MAX;  // u(lo) <= p
  if (u(hi) <= p) return INT32_MAX;
  while (hi - lo > 1) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (u(mid) <= p)
      lo = mid;
    else
      hi = mid;
  }
  return (int32_t)lo;
}

fas::DropParams drop_params(const fas_attn_args* a, const Problem& pr) {
  fas::DropParams d{};
  d.scale = 1.f;
  if (!(a->dropout_p > 0.f)) return d;
  const uint64_t off = a->dropout_offset;
  const bool wide = off >= (1ull << 31);  // a 64-bit offset fills counter word 1
  d.k0 = (uint32_t)a->dropout_seed;
  d.k1 = (uint32_t)(a->dropout_seed >> 32);
  d.off_lo = (uint32_t)off;
  // Index sums below 2^32 - off_lo do not carry into word 1; the element
  // index stays below 2^31 with a 64-bit offset (the argument check rejects
  // larger problems).
  d.carry_lim = wide ? d.off_lo : 0u;
  const uint32_t w1 = wide ? (uint32_t)(off >> 32) : 0u;
  uint32_t hi[2], lo[2];
  for (int c = 0; c < 2; ++c) {
    const uint64_t pa = (uint64_t)fas::kPhiloxMulA * ((w1 + (uint32_t)c) ^ d.k0);
    hi[c] = (uint32_t)(pa >> 32) ^ (d.k1 + fas::kPhiloxWeylB);
    lo[c] = (uint32_t)pa;
  }
  d.r1_hi = hi[0];
  d.r1_hi_carry = hi[0] ^ hi[1];
  d.r1_lo = lo[0];
  d.r1_lo_carry = lo[0] ^ lo[1];
  // y = x ^ (x >> 31) > t (x the word as int32, t in [0, 2^31 - 1]) holds
  // for x mod 2^32 in [t + 1, 2^32 - t - 2]: t + 1 .. 2^31 - 1 as x >= 0,
  // 2^31 .. 2^32 - t - 2 as x <= -t - 2.  Empty for t = 2^31 - 1.
  const uint32_t t = (uint32_t)dropout_thresh(a->dropout_p);
  d.keep_lo = t + 1u;
  d.keep_span = 0xFFFFFFFEu - 2u * t;
  d.n = pr.N;
  return d;
}

// O multiplier of the entry points that rescale kept weights (the reference
// computes 1.0 / (1.0 - dropout_p) in fp32, attention_with_scores.py:200-203).
void rescale_dropout(fas::FwdParams& p, const fas_attn_args* a) {
  if (p.dropout) p.drop.scale = 1.f / (1.f - a->dropout_p);
}

// Fills the forward parameter block.  top_left selects the cross-token
// QK-sum's causal alignment (i >= j) instead of (N - M) + i >= j.
fas::FwdParams fwd_params(const fas_attn_args* a, const Problem& pr, bool top_left, int rows_per_block) {
  fas::FwdParams p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->out);
  p.sq0 = a->q_stride[0]; p.sq1 = a->q_stride[1]; p.sq2 = a->q_stride[2];
  p.sk0 = a->k_stride[0]; p.sk1 = a->k_stride[1]; p.sk2 = a->k_stride[2];
  p.sv0 = a->v_stride[0]; p.sv1 = a->v_stride[1]; p.sv2 = a->v_stride[2];
  p.so0 = a->out_stride[0]; p.so1 = a->out_stride[1]; p.so2 = a->out_stride[2];
  // q and out are addressed from the first head of a packed group.
  p.q_bytes = slice_bytes(pr.M, p.sq2, pr.D) + (uint32_t)((pr.pack - 1) * p.sq1 * 2);
  p.o_bytes = slice_bytes(pr.M, p.so2, pr.D) + (uint32_t)((pr.pack - 1) * p.so1 * 2);
  p.k_bytes = slice_bytes(pr.N, p.sk2, pr.D);
  p.v_bytes = slice_bytes(pr.N, p.sv2, pr.D);
  p.qneg = pr.sm_scale < 0.f ? 0x80008000u : 0u;
  p.B = pr.B;
  p.H = pr.H;
  p.G = pr.G;
  p.M = pr.M;
  p.N = pr.N;
  p.causal = pr.causal;
  p.causal_off = top_left ? 0 : pr.N - pr.M;
  p.pack = pr.pack;
  p.pack_shift = pr.pack == 1 ? 0 : pr.pack == 2 ? 1 : pr.pack == 4 ? 2 : pr.pack == 8 ? 3 : -1;
  p.nrb = (int)(((int64_t)pr.M * pr.pack + rows_per_block - 1) / rows_per_block);
  p.bm = rows_per_block;
  p.nsplit = 1;
  p.sm_scale = std::fabs(pr.sm_scale);
  p.qk_scale = qk_scale_of(pr.sm_scale);
  p.dropout = a->dropout_p > 0.f ? 1 : 0;
  p.drop = drop_params(a, pr);
  return p;
}

int run_fwd(const char* fn, fas::FwdParams& p, const Problem& pr, int mode, void* stream) {
  if (p.nrb == 0 || (int64_t)pr.B * pr.H == 0) return FAS_OK;
  return hip_status(fn, fas::launch_fwd(p, mode, pr.dtype, pr.D, static_cast<hipStream_t>(stream)));
}

// Whether one of the first n strides is negative or past kMaxOuterStride.
bool strides_out_of_range(const int64_t* st, int n) {
  for (int i = 0; i < n; ++i)
    if (st[i] < 0 || st[i] >= kMaxOuterStride) return true;
  return false;
}

int check_out3(const char* fn, const char* name, const float* out, const int64_t* st) {
  if (out == nullptr) return fail(FAS_ERR_INVALID, fn, "%s is NULL", name);
  if (st == nullptr) return fail(FAS_ERR_INVALID, fn, "%s strides are NULL", name);
  if (strides_out_of_range(st, 3))
    return fail(FAS_ERR_INVALID, fn, "%s strides must lie in [0, 2^46)", name);
  return FAS_OK;
}

int zero_out3(const char* fn, float* out, const int64_t* st, int64_t n0, int64_t n1, int64_t n2,
              void* stream) {
  return hip_status(fn, fas::launch_fill_zero(out, st[0], st[1], st[2], n0, n1, n2,
                                              static_cast<hipStream_t>(stream)));
}

// ---------------------------------------------------------------- workspace

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SplitPlan {
  int nsplit = 1, tps = 0;
  int64_t mpad = 0;
};

// Head split of the softmax column pass (ColsmParams.fold / nsplit): one
// workgroup per (unit, split, output group), a unit being a mirror pair of
// 256-key blocks (colsm64_kernel) or one key block (the buffered pass).
// With fold heads per output column, nsplit workgroups share a unit's heads
// (heads s, s + nsplit, ...) and fold their column sums through partials and
// a ticket per unit; nsplit is the smallest of least cost, cost = rounds of
// `slots` concurrent workgroups x heads per workgroup, so a problem with few
// output groups still fills the chip (B1 with 4 KV heads of 7 query heads:
// 7 splits, 224 workgroups), and one that fills it walks all of a KV head's
// query heads per workgroup with its keys resident (8 KV heads of 4 query
// heads at 16K keys: 256 workgroups, no split).
struct ColPlan {
  int fold = 1, nsplit = 1;
  int64_t nunits = 0, ngroups = 0;
};
constexpr int64_t kCus = 256;  // MI355X compute units
ColPlan col_plan(const Problem& pr, bool buffered, int64_t ncols, bool fold_heads) {
  ColPlan c;
  c.fold = fold_heads ? pr.G : 1;
  c.ngroups = (int64_t)pr.B * (pr.H / c.fold);
  int64_t slots = kCus;  // colsm64_kernel: one 8-wave workgroup per CU
  if (buffered) {
    const int64_t bk = ncols % 4 == 0 ? 256 : 64;  // keys per workgroup (VEC or not)
    c.nunits = (ncols + bk - 1) / bk;
    slots = 8 * kCus;  // 4-wave workgroups, eight per CU
  } else {
    c.nunits = ((ncols + 255) / 256 + 1) / 2;
  }
  int64_t best = INT64_MAX;
  for (int ns = 1; ns <= c.fold; ++ns) {
    const int64_t wgs = c.nunits * ns * c.ngroups;
    const int64_t cost = ((wgs + slots - 1) / slots) * ((c.fold + ns - 1) / ns);
    if (cost < best) {
      best = cost;
      c.nsplit = ns;
    }
  }
  return c;
}

struct Workspace {
  size_t lse = 0, part = 0, bsum = 0, region = 0, region_m = 0, total = 0;  // byte offsets / total
  size_t ticket = 0;                                            // column-pass tickets
  ColPlan cp;                                                   // column-pass head split
  size_t bits = 0;                                              // dropout keep bits
  bool has_bits = false;
  size_t nl = 0, delta = 0;                                     // backward row values
  size_t ds = 0;                                                // backward dS blocks
  int64_t ds_head = 0;
  bool has_ds = false;
  size_t so = 0, sm = 0, sl = 0, sr = 0;                        // key-split partials
  bool has_lse = false, has_part = false, has_bsum = false, has_region = false;
  bool has_split = false;
  SplitPlan sp;  // the forward's key split (nsplit 1: none)
};

// Key split of the plain / row-sum forward.  When the row blocks of the
// whole problem give fewer workgroups than the chip has CUs (short query
// ranges against long key ranges: decode, last-window scoring), each row
// block's key tiles are dealt to nsplit workgroups of at least 8 tiles,
// aiming at ~512 workgroups in all.  Depends on sizes only, so the workspace
// query and the launch agree.  The scores variant splits only up to 64 row
// blocks, 128 when the key range is at least 8 times the query range, 256
// at 64 times: its split route writes the scores in a second kernel, which
// the fused writer beats while it still has a quarter of the CUs busy, or
// half or all of them over keys not much longer than its rows (B2 H32 M512
// N16384: 0.607 against 0.734 ms fused; B1 H32 M1024 N16384: 0.547 against
// 0.592; B8 H32 M256 N16384: 1.27 against 1.58; but B4 H32 M512 N16384:
// 1.19 against 1.16 fused; B1 H32 M = N = 1024 stays fused).
constexpr int64_t kScoresSplitMaxWgs = 64;
static int64_t scores_split_max_wgs(const Problem& pr) {
  const int64_t m = pr.M;
  return pr.N >= 64 * m ? 4 * kScoresSplitMaxWgs
         : pr.N >= 8 * m ? 2 * kScoresSplitMaxWgs
                         : kScoresSplitMaxWgs;
}
// Bytes of the fp32 partials of a plan (O, offset, weight sum, row sum).
size_t split_bytes(const Problem& pr, const SplitPlan& sp) {
  const size_t rows = (size_t)pr.B * pr.H * sp.nsplit * sp.mpad;
  return align256(rows * pr.D * 4) + 3 * align256(rows * 4);
}
// max_bytes bounds the partials (the no-allocation entry point's scratch):
// the plan then takes fewer, longer splits, or none.
SplitPlan split_plan(const Problem& pr, bool top_left, int64_t max_wgs = 255,
                     size_t max_bytes = SIZE_MAX) {
  SplitPlan sp;
  // Virtual row blocks of each group of pack heads (the forward's grid).
  const int64_t nrb = ((int64_t)pr.M * pr.pack + fas::kFwdRows - 1) / fas::kFwdRows;
  const int64_t wgs = (int64_t)pr.B * (pr.H / pr.pack) * nrb;
  if (wgs == 0 || wgs > max_wgs) return sp;
  const int64_t off = top_left ? 0 : (int64_t)pr.N - pr.M;
  int64_t hi = pr.N;
  if (pr.causal) hi = std::min<int64_t>(pr.N, std::max<int64_t>(0, off + pr.M));
  const int64_t nt = (hi + 63) / 64;
  for (int64_t want = std::min<int64_t>((512 + wgs - 1) / wgs, nt / 8); want >= 2; --want) {
    const int64_t tps = (nt + want - 1) / want;
    const int64_t ns = (nt + tps - 1) / tps;
    if (ns < 2) break;
    SplitPlan c;
    c.nsplit = (int)ns;
    c.tps = (int)tps;
    // Partials are indexed by (head, split, position): M rounded up.
    c.mpad = (((int64_t)pr.M + fas::kFwdRows - 1) / fas::kFwdRows) * fas::kFwdRows;
    if (split_bytes(pr, c) <= max_bytes) return c;
  }
  return sp;
}

// Whether a variant's forward pass is the plain or row-sum kernel (the ones
// that can split), and its causal alignment.
// The scores variant takes this route too: for a split plan it runs the
// plain forward plus the scores-only kernel instead of the fused writer.
bool forward_can_split(int variant) {
  return variant != FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED &&
         variant != FAS_VARIANT_ATTENTION_BACKWARD;
}

// Backward: rows padded to whole 128-row blocks.
int64_t bwd_mpad(const Problem& pr) {
  return (((int64_t)pr.M + fas::kBwdBlock - 1) / fas::kBwdBlock) * fas::kBwdBlock;
}
int64_t bwd_nkb(const Problem& pr) { return ((int64_t)pr.N + fas::kBwdBlock - 1) / fas::kBwdBlock; }
// The dK/dV kernel walks a KV head's whole query-head group per workgroup
// unless that leaves fewer workgroups than the chip has CUs; then it takes
// one query head per workgroup and writes fp32 partials.
bool bwd_partial(const Problem& pr) {
  return pr.G > 1 && (int64_t)pr.B * pr.Hk * bwd_nkb(pr) < 256;
}
// The backward's stored dS (BwdParams.ds): 32-row block r sees 32-key blocks
// [0, clamp(r + a, 0, ceil(N/32))): a = floor((N - M + 31) / 32) + 1 under the
// causal mask (block (r, j) holds a visible pair iff (N - M) + 32 r + 31 >=
// 32 j), every block without it.
int64_t bwd_ds_a(const Problem& pr) {
  const int64_t n32 = ((int64_t)pr.N + 31) / 32;
  if (!pr.causal) return n32;
  const int64_t x = (int64_t)pr.N - pr.M + 31;
  return (x >= 0 ? x / 32 : -((-x + 31) / 32)) + 1;
}
int64_t bwd_ds_head(const Problem& pr) {
  return fas::ds_block_start(bwd_mpad(pr) / 32, bwd_ds_a(pr), ((int64_t)pr.N + 31) / 32);
}
// Largest dS workspace the backward takes (all heads); past it, and when one
// head's blocks reach 2 GiB, the dQ kernel recomputes S and dP instead.
constexpr size_t kBwdDsMaxBytes = (size_t)16 << 30;
size_t bwd_ds_bytes(const Problem& pr) {
  return align256((size_t)pr.B * pr.H * (size_t)bwd_ds_head(pr) * 2048);
}
// Whether the backward stores dS when the caller's workspace has room.
bool bwd_ds_fits(const Problem& pr) {
  return pr.M > 0 && pr.N > 0 && bwd_ds_head(pr) * 2048 < ((int64_t)1 << 31) &&
         bwd_ds_bytes(pr) <= kBwdDsMaxBytes;
}

// The caller's keep-bit buffer (fas_attn_args.keep_bits) of attention's
// forward and backward: key-major words for the dK/dV kernel (word
// ((b*H + h) * ceil(M/32) + i/32) * N + j, bit i % 32), then, only when the
// backward cannot store dS, 32-row blocks of row-major words for the dQ
// kernel that recomputes S and dP (the backward's own layout, rows padded
// to Mpad).  Each head's part must stay below 2 GiB (32-bit buffer
// offsets); otherwise no buffer (key-major part) or no row blocks.
struct KeepLayout {
  size_t keys = 0, rows = 0, total = 0;  // byte offsets / total
  bool ok = false;
  bool has_rows = false;
};
KeepLayout keep_layout(const Problem& pr) {
  KeepLayout k;
  const size_t head_keys = (size_t)((pr.M + 31) / 32) * pr.N * 4;
  const size_t head_rows = (size_t)bwd_mpad(pr) * ((pr.N + 31) / 32) * 4;
  if (!pr.dropout || head_keys >= ((size_t)1 << 31)) return k;
  k.keys = 0;
  k.total = align256((size_t)pr.B * pr.H * head_keys);
  k.ok = true;
  // The row blocks serve only the dQ kernel that recomputes S and dP: none
  // when the backward can store dS (a backward that then takes the recompute
  // route anyway evaluates the random stream for dQ, with the same result).
  if (!bwd_ds_fits(pr) && head_rows < ((size_t)1 << 31)) {
    k.rows = k.total;
    k.total += align256((size_t)pr.B * pr.H * head_rows);
    k.has_rows = true;
  }
  return k;
}

int check_keep(const char* fn, const fas_attn_args* a, const Problem& pr, KeepLayout* kl) {
  *kl = keep_layout(pr);
  if (!pr.keep) return FAS_OK;
  if (!kl->ok)
    return fail(FAS_ERR_UNSUPPORTED, fn, "keep_bits given, but a head's bits exceed 2 GiB");
  if ((reinterpret_cast<uintptr_t>(a->keep_bits) & 255u) != 0)
    return fail(FAS_ERR_INVALID, fn, "keep_bits must be 256-byte aligned");
  return FAS_OK;
}

// Column count of a variant's side output.
int64_t ncols_of(int variant, const Problem& pr, int64_t split) {
  switch (variant) {
    case FAS_VARIANT_CROSS_QK_SUM:
    case FAS_VARIANT_CROSS_SOFTMAX_SUM:
    case FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED: return split;
    default: return pr.N;
  }
}

// budget: largest total the caller can provide (SIZE_MAX: any); only the
// key-split partials adapt to it, by a smaller split.
Workspace layout(int variant, const Problem& pr, int64_t split, size_t budget = SIZE_MAX) {
  Workspace w;
  size_t off = 0;
  const int64_t ncols = ncols_of(variant, pr, split);
  const bool softmax = variant == FAS_VARIANT_SOFTMAX_COL_SUM ||
                       variant == FAS_VARIANT_CROSS_SOFTMAX_SUM ||
                       variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED;
  const bool raw = variant == FAS_VARIANT_COL_SUM || variant == FAS_VARIANT_COL_SUM_SEQUENTIAL ||
                   variant == FAS_VARIANT_CROSS_QK_SUM;
  if (softmax) {
    w.has_lse = true;
    w.lse = off;
    off += align256((size_t)pr.B * pr.H * pr.M * 4);
    w.cp = col_plan(pr, variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED, ncols, true);
    if (w.cp.nsplit > 1) {
      // The splits' column sums and one ticket per (output group, unit).
      w.has_part = true;
      w.part = off;
      off += align256((size_t)w.cp.ngroups * w.cp.nsplit * ncols * 4);
      w.ticket = off;
      off += align256((size_t)w.cp.ngroups * w.cp.nunits * 4);
    }
  }
  // The softmax column sum with dropout: the forward stores its keep
  // decisions (one bit per pair, 32-row words) for the column pass, which
  // would otherwise evaluate the Philox stream again, when they fit the
  // budget and a head's words stay below 2 GiB (32-bit buffer offsets).
  if (variant == FAS_VARIANT_SOFTMAX_COL_SUM && pr.dropout) {
    const size_t head_bytes = (size_t)((pr.M + 31) / 32) * pr.N * 4;
    const size_t bytes = align256((size_t)pr.B * pr.H * head_bytes);
    if (head_bytes < ((size_t)1 << 31) && off + bytes <= budget) {
      w.has_bits = true;
      w.bits = off;
      off += bytes;
    }
  }
  if (variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED) {
    // The region's fp16 exponents, then one fp32 offset per 64-key tile and
    // region row (tile-major).
    w.has_region = true;
    w.region = off;
    const int64_t rows = pr.M > split ? pr.M - split : 0;
    off += align256((size_t)pr.B * pr.H * rows * split * 2);
    w.region_m = off;
    off += align256((size_t)pr.B * pr.H * rows * ((split + 63) / 64) * 4);
  }
  if (variant == FAS_VARIANT_ATTENTION_BACKWARD) {
    const size_t rows = (size_t)pr.B * pr.H * bwd_mpad(pr) * 4;
    w.nl = off;
    off += align256(rows);
    w.delta = off;
    off += align256(rows);
    if (bwd_partial(pr)) {
      w.has_part = true;
      w.part = off;
      off += align256((size_t)pr.B * pr.H * pr.N * 2 * pr.D * 4);
    }
    // dS for the dQ kernel (2 bytes per visible pair, in 32 x 32 blocks),
    // when a head's blocks stay below 2 GiB, all of them within
    // kBwdDsMaxBytes and the caller's workspace has room for them
    // (fas_workspace_bytes includes them unless asked with split != 0).
    const size_t ds_bytes = bwd_ds_bytes(pr);
    if (split == 0 && bwd_ds_fits(pr) && off + ds_bytes <= budget) {
      w.has_ds = true;
      w.ds = off;
      w.ds_head = bwd_ds_head(pr);
      off += ds_bytes;
    }
    // Without stored dS, with dropout, the dK/dV kernel stores its keep
    // decisions (one bit per pair) for the dQ kernel, when a head's words
    // stay below 2 GiB and the caller's workspace has room for them
    // (fas_workspace_bytes includes them); otherwise the dQ kernel evaluates
    // the Philox stream again.
    const size_t head_bytes = (size_t)bwd_mpad(pr) * ((pr.N + 31) / 32) * 4;
    const size_t bits = align256((size_t)pr.B * pr.H * head_bytes);
    if (!w.has_ds && pr.dropout && !pr.keep && head_bytes < ((size_t)1 << 31) &&
        off + bits <= budget) {
      w.has_bits = true;
      w.bits = off;
      off += bits;
    }
  }
  if (raw) {
    const int64_t row_lo = variant == FAS_VARIANT_CROSS_QK_SUM ? split : 0;
    const int64_t rows = pr.M > row_lo ? pr.M - row_lo : 0;
    const int64_t nblk = (rows + 63) / 64;
    w.has_bsum = true;
    w.bsum = off;
    off += align256((size_t)pr.B * pr.Hk * (nblk + 1) * pr.D * 4);
  }
  if (forward_can_split(variant) && off <= budget) {
    const SplitPlan sp = split_plan(pr, variant == FAS_VARIANT_CROSS_QK_SUM,
                                    variant == FAS_VARIANT_SCORES ? scores_split_max_wgs(pr) : 255,
                                    budget - off);
    if (sp.nsplit > 1) {
      const size_t rows = (size_t)pr.B * pr.H * sp.nsplit * sp.mpad;
      w.has_split = true;
      w.sp = sp;
      w.so = off;
      off += align256(rows * pr.D * 4);
      w.sm = off;
      off += align256(rows * 4);
      w.sl = off;
      off += align256(rows * 4);
      w.sr = off;
      off += align256(rows * 4);
    }
  }
  w.total = off;
  return w;
}

int check_workspace(const char* fn, const Workspace& w, void* ws, size_t bytes) {
  if (w.total == 0) return FAS_OK;
  if (ws == nullptr || bytes < w.total)
    return fail(FAS_ERR_WORKSPACE, fn, "workspace of %zu bytes needed, %zu given", w.total, bytes);
  if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
    return fail(FAS_ERR_INVALID, fn, "workspace must be 256-byte aligned");
  return FAS_OK;
}

template <class T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

// Points the forward at its key-split partials when the plan splits.
void apply_split(fas::FwdParams& p, const Workspace& w, void* ws) {
  if (!w.has_split) return;
  const SplitPlan& sp = w.sp;
  p.nsplit = sp.nsplit;
  p.tps = sp.tps;
  p.Mpad = (int)sp.mpad;
  p.part_o = at<float>(ws, w.so);
  p.part_m = at<float>(ws, w.sm);
  p.part_l = at<float>(ws, w.sl);
  p.part_r = at<float>(ws, w.sr);
}

// ---------------------------------------------------------------- variants

// Raw-score column sums (col_sum, col_sum_sequential, cross_qk).
int run_raw(const char* fn, int variant, const fas_attn_args* a, int64_t split, float* out,
            const int64_t* st, void* ws, size_t ws_bytes, void* stream) {
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  const bool cross = variant == FAS_VARIANT_CROSS_QK_SUM;
  if (cross && !(split > 0 && split <= pr.N))
    return fail(FAS_ERR_INVALID, fn, "split %lld outside (0, %d]", (long long)split, pr.N);
  if ((rc = check_out3(fn, "sum output", out, st))) return rc;
  const int64_t ncols = ncols_of(variant, pr, split);
  if ((int64_t)pr.B * pr.Hk * ncols == 0) {
    fas::FwdParams p = fwd_params(a, pr, cross, fas::kFwdRows);
    return run_fwd(fn, p, pr, fas::kFwdPlain, stream);
  }
  const Workspace w = layout(variant, pr, split);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;

  // Attention output.
  fas::FwdParams p = fwd_params(a, pr, cross, fas::kFwdRows);
  apply_split(p, w, ws);
  if ((rc = run_fwd(fn, p, pr, fas::kFwdPlain, stream))) return rc;
  if (pr.M == 0) return zero_out3(fn, out, st, pr.B, pr.Hk, ncols, stream);

  fas::RawParams r{};
  r.q = p.q;
  r.k = p.k;
  r.bsum = at<float>(ws, w.bsum);
  r.out = out;
  r.sq0 = p.sq0; r.sq1 = p.sq1; r.sq2 = p.sq2;
  r.sk0 = p.sk0; r.sk1 = p.sk1; r.sk2 = p.sk2;
  r.so0 = st[0]; r.so1 = st[1]; r.so2 = st[2];
  r.B = pr.B; r.H = pr.H; r.G = pr.G; r.Hk = pr.Hk; r.M = pr.M; r.N = pr.N; r.D = pr.D;
  r.row_lo = cross ? (int)split : 0;
  r.nblk = pr.M > r.row_lo ? (pr.M - r.row_lo + 63) / 64 : 0;
  r.ncols = (int)ncols;
  r.causal = pr.causal;
  r.causal_off = pr.N - pr.M;
  // Cross-token sums see every (i >= split, j < split) pair under the
  // top-left mask, so only the bottom-right causal column sum needs the
  // per-key suffix.
  const bool suffix = !cross && pr.causal;
  r.nextra = suffix && r.causal_off > 0 ? (std::min(r.ncols, r.causal_off) + 63) / 64 : 0;
  r.sm_scale = pr.sm_scale;
  return hip_status(fn, fas::launch_rawsum(r, pr.dtype, suffix, static_cast<hipStream_t>(stream)));
}

// Softmax-weight column sums (softmax col sum, cross softmax, buffered).
int run_softmax(const char* fn, int variant, const fas_attn_args* a, int64_t split, float* out,
                const int64_t* st, void* ws, size_t ws_bytes, void* stream,
                size_t budget = SIZE_MAX) {
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  const bool cross = variant != FAS_VARIANT_SOFTMAX_COL_SUM;
  const bool buffered = variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED;
  if (cross && !(split > 0 && split <= pr.N))
    return fail(FAS_ERR_INVALID, fn, "split %lld outside (0, %d]", (long long)split, pr.N);
  if ((rc = check_out3(fn, "sum output", out, st))) return rc;
  const int64_t ncols = ncols_of(variant, pr, split);
  const Workspace w = layout(variant, pr, split, budget);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;

  fas::FwdParams p = fwd_params(a, pr, false, fas::kFwdRows);
  p.lse2 = at<float>(ws, w.lse);
  if (w.has_bits) p.drop_bits = at<uint32_t>(ws, w.bits);
  if (w.cp.nsplit > 1) {
    // The forward clears the column pass's tickets.
    p.zero_words = at<uint32_t>(ws, w.ticket);
    p.n_zero_words = (int)(w.cp.ngroups * w.cp.nunits);
  }
  if (!buffered) apply_split(p, w, ws);
  if (buffered) {
    p.region = at<uint16_t>(ws, w.region);
    p.region_m = at<float>(ws, w.region_m);
    p.region_rows = (int64_t)pr.B * pr.H * (pr.M > split ? pr.M - split : 0);
    p.split = (int)split;
    p.vec_region = (split % 8 == 0) ? 1 : 0;
  }
  const int mode = buffered ? fas::kFwdRegion : w.has_bits ? fas::kFwdPlainKeepBits : fas::kFwdPlain;
  if ((rc = run_fwd(fn, p, pr, mode, stream))) return rc;
  if ((int64_t)pr.B * pr.Hk * ncols == 0) return FAS_OK;
  if ((int64_t)pr.B * pr.H * pr.M == 0) return zero_out3(fn, out, st, pr.B, pr.Hk, ncols, stream);

  fas::ColsmParams c{};
  c.q = p.q;
  c.k = p.k;
  c.lse2 = p.lse2;
  c.region = p.region;
  c.region_m = p.region_m;
  c.region_rows = p.region_rows;
  c.sq0 = p.sq0; c.sq1 = p.sq1; c.sq2 = p.sq2;
  c.sk0 = p.sk0; c.sk1 = p.sk1; c.sk2 = p.sk2;
  c.q_bytes = p.q_bytes;
  c.k_bytes = p.k_bytes;
  c.qneg = p.qneg;
  c.B = pr.B; c.H = pr.H; c.G = pr.G; c.M = pr.M; c.N = pr.N;
  c.row_lo = cross ? (int)split : 0;
  c.ncols = (int)ncols;
  c.split = (int)split;
  c.causal = pr.causal;
  c.causal_off = pr.N - pr.M;
  c.nkb = (int)((ncols + 255) / 256);
  c.qk_scale = p.qk_scale;
  // Only the softmax column sum masks its weights; the cross-token pass
  // does not (attention_cross_token_softmax_sum.py has no dropout there).
  c.dropout = variant == FAS_VARIANT_SOFTMAX_COL_SUM && p.dropout ? (w.has_bits ? 2 : 1) : 0;
  c.drop = p.drop;
  c.drop_bits = p.drop_bits;
  c.out = out;
  c.so0 = st[0]; c.so1 = st[1]; c.so2 = st[2];
  // The column sums of a KV head's query heads, folded inside the pass.
  c.fold = w.cp.fold;
  c.nsplit = w.cp.nsplit;
  if (w.cp.nsplit > 1) {
    c.part = at<float>(ws, w.part);
    c.ticket = at<uint32_t>(ws, w.ticket);
  }
  return hip_status(fn, fas::launch_colsm(c, pr.dtype, pr.D, buffered,
                                          static_cast<hipStream_t>(stream)));
}

// ------------------------------------------------- no-allocation scratch
//
// fas_attention_with_softmax_col_sum_noalloc takes its workspace from this
// file-scope device array instead of a caller buffer, for callers that
// cannot allocate.  Every GPU the library runs on holds its own copy for the
// life of the process.  Host code must never pass `scratch` itself to a
// kernel or copy: on the host the name is only a stand-in.  Its device
// address is looked up once per device, with that device current, and kept
// in g_scratch_ptr.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch, resolved on the first
// call on each device.
int scratch_of_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(fn, e);
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FAS_ERR_UNSUPPORTED, fn, "device %d beyond the %d this build tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(FAS_ERR_HIP, fn, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FAS_OK;
}

}  // namespace

extern "C" {

int fas_abi_version(void) { return FAS_ABI_VERSION; }

const char* fas_last_error(void) { return g_last_error.c_str(); }

size_t fas_workspace_bytes(int variant, const fas_attn_args* a, int64_t split) {
  static const char* fn = "fas_workspace_bytes";
  Problem pr;
  if (variant < FAS_VARIANT_SCORES || variant > FAS_VARIANT_KEEP_BITS) {
    fail(FAS_ERR_INVALID, fn, "variant %d unknown", variant);
    return (size_t)-1;
  }
  if (check_shape(fn, a, &pr)) return (size_t)-1;
  if (variant == FAS_VARIANT_KEEP_BITS) return keep_layout(pr).total;
  const bool has_split = variant == FAS_VARIANT_CROSS_QK_SUM ||
                         variant == FAS_VARIANT_CROSS_SOFTMAX_SUM ||
                         variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED;
  if (has_split && !(split > 0 && split <= pr.N)) {
    fail(FAS_ERR_INVALID, fn, "split %lld outside (0, %d]", (long long)split, pr.N);
    return (size_t)-1;
  }
  // The backward: split != 0 asks for the size without the stored dS.
  const bool bwd = variant == FAS_VARIANT_ATTENTION_BACKWARD;
  // The key-split plan depends on the GQA packing, which a launch picks
  // from the strides; the size covers both choices, so a query made with
  // placeholder strides still suffices.
  size_t total = 0;
  for (int pk : {1, pr.G}) {
    Problem q = pr;
    q.pack = pk;
    total = std::max(total, layout(variant, q, has_split || bwd ? split : 0).total);
  }
  return total;
}

static int check_scores_out(const char* fn, const void* scores, const int64_t* st) {
  if (scores == nullptr || st == nullptr) return fail(FAS_ERR_INVALID, fn, "scores is NULL");
  if (st[3] != 1) return fail(FAS_ERR_INVALID, fn, "scores innermost stride must be 1");
  if (reinterpret_cast<uintptr_t>(scores) & 1u)
    return fail(FAS_ERR_INVALID, fn, "scores is not 2-byte aligned");
  if (strides_out_of_range(st, 3))
    return fail(FAS_ERR_INVALID, fn, "scores strides must lie in [0, 2^46)");
  if ((int64_t)fas::kFwdRows * st[2] * 2 >= kMaxSliceBytes)
    return fail(FAS_ERR_UNSUPPORTED, fn, "score rows too long for 32-bit offsets");
  return FAS_OK;
}

// Scores alone through the scores-only kernel; mask selects the causal /
// key-range mask with masked entries written as 0.
static int run_scores(const char* fn, const fas_attn_args* a, const Problem& pr, void* scores,
               const int64_t* st, bool mask, void* stream) {
  fas::ScoresParams p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.scores = static_cast<uint16_t*>(scores);
  p.sq0 = a->q_stride[0]; p.sq1 = a->q_stride[1]; p.sq2 = a->q_stride[2];
  p.sk0 = a->k_stride[0]; p.sk1 = a->k_stride[1]; p.sk2 = a->k_stride[2];
  p.ss0 = st[0]; p.ss1 = st[1]; p.ss2 = st[2];
  p.q_bytes = slice_bytes(pr.M, p.sq2, pr.D);
  p.k_bytes = slice_bytes(pr.N, p.sk2, pr.D);
  p.B = pr.B; p.H = pr.H; p.G = pr.G; p.M = pr.M; p.N = pr.N;
  p.mask = mask && pr.causal ? 1 : 0;
  p.causal_off = pr.N - pr.M;
  p.nkb = (pr.N + fas::kScoresKeysPerBlock - 1) / fas::kScoresKeysPerBlock;
  // Row ranges when the key blocks give fewer than 512 workgroups (two per
  // CU), each at least 8 steps of 64 rows: a workgroup loads 32 KiB of K per
  // key group before its first step (B1 H8 S2048: 26.3 us with 4-step
  // ranges, 21.8 us with 8).
  {
    const int64_t steps = std::max<int64_t>(1, (pr.M + 63) / 64);
    const int64_t wgs = (int64_t)pr.B * pr.H * p.nkb;
    int64_t nrs = wgs >= 512 ? 1 : (512 + wgs - 1) / wgs;
    nrs = std::max<int64_t>(1, std::min(nrs, steps / 8));
    p.spr = (int)((steps + nrs - 1) / nrs);
    p.nrs = (int)((steps + p.spr - 1) / p.spr);
  }
  p.vec = aligned16(scores) && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 &&
                  pr.N % 8 == 0
              ? 1
              : 0;
  // Up to 512 query rows with 16-byte score stores: the resident-Q kernel,
  // one workgroup per CU, each walking two or more of its head's 512-key
  // blocks.
  // Under GQA a workgroup takes the largest power-of-two share of a KV
  // head's query heads whose rows fit (K loaded once for all of them), as
  // long as its q and score offsets stay 31-bit.
  if (p.vec && pr.M <= fas::kScoresResidentRows) {
    const int64_t nkb = (pr.N + fas::kScoresResidentKeys - 1) / fas::kScoresResidentKeys;
    int pshift = 0;
    auto fits = [&](int pk) {
      return pr.G % pk == 0 && (int64_t)pk * pr.M <= fas::kScoresResidentRows &&
             ((int64_t)(pk - 1) * p.sq1 + (int64_t)pr.M * p.sq2) * 2 < fas::kScoresResidentBytes &&
             ((int64_t)(pk - 1) * st[1] + (int64_t)(pr.M - 1) * st[2] + fas::kScoresResidentKeys) *
                     2 <
                 fas::kScoresResidentBytes;
    };
    while (fits(2 << pshift)) ++pshift;
    const int64_t groups = ((int64_t)pr.B * pr.H) >> pshift;
    const int64_t ngrp = std::min<int64_t>(nkb, (device_cu_count() + groups - 1) / groups);
    if (fits(1) && nkb >= 2 * ngrp) {
      p.ngrp = (int)ngrp;
      p.nkb = (int)nkb;
      p.pshift = pshift;
      if (pshift > 0)
        p.q_bytes = (uint32_t)(((int64_t)((1 << pshift) - 1) * p.sq1 + (int64_t)pr.M * p.sq2) * 2);
    }
  }
  p.sm_scale = pr.sm_scale;
  return hip_status(fn, fas::launch_scores(p, pr.dtype, pr.D, static_cast<hipStream_t>(stream)));
}

static int attention_with_scores_impl(const fas_attn_args* a, void* scores, const int64_t st[4],
                                   void* ws, size_t ws_bytes, void* stream) {
  static const char* fn = "fas_attention_with_scores";
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H * pr.M == 0) return FAS_OK;
  if ((rc = check_scores_out(fn, scores, st))) return rc;
  const Workspace w = layout(FAS_VARIANT_SCORES, pr, 0);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;
  if (w.has_split) {
    // Short query range: the fused writer would run one workgroup per row
    // block for every key tile; the key-split plain forward gives O and the
    // scores-only kernel writes the masked scores in parallel over keys.
    fas::FwdParams p = fwd_params(a, pr, false, fas::kFwdRows);
    rescale_dropout(p, a);
    apply_split(p, w, ws);
    if ((rc = run_fwd(fn, p, pr, fas::kFwdPlain, stream))) return rc;
    return run_scores(fn, a, pr, scores, st, true, stream);
  }
  int bm = fas::kFwdRows;
  // The score writer packs 2, 4 or 8 heads (its store layout keeps a lane's
  // head fixed) and addresses their score rows from the first head's, below
  // offset 2^31; otherwise each workgroup takes one head.
  Problem pw = pr;
  if (pw.pack > 1 &&
      ((pw.pack != 2 && pw.pack != 4 && pw.pack != 8) ||
       ((int64_t)(pw.pack - 1) * st[1] + (int64_t)(bm / pw.pack + 2) * st[2]) * 2 >= kMaxSliceBytes))
    pw.pack = 1;
  // One workgroup runs per CU.  When 256-row blocks would all run in one
  // round (the longest causal row block is then the critical path), unpacked
  // launches take 128-row blocks (4 waves): twice the workgroups, in two
  // rounds the mirror order balances (B1 H32 S1024: 45.7 -> 37.5 us; H16
  // S4096: 179 -> 145 us; H32 S2048: 94.3 -> 95.9 us).
  // (The dropout instances exist with 256-row blocks only.)
  const int vec_scores =
      aligned16(scores) && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 && pr.N % 8 == 0;
  const int64_t cus = device_cu_count();
  if (pw.pack == 1 && !(a->dropout_p > 0.f) &&
      (int64_t)pr.B * pr.H * ((pr.M + fas::kFwdRows - 1) / fas::kFwdRows) <= cus) {
    bm = fas::kFwdRows / 2;
    // When even the 128-row blocks all run in one round under a causal mask
    // with long rows, the writer takes 64-row blocks with each block's key
    // tiles split between its two wave pairs (16-byte score rows only): two
    // rounds of balanced pairs.  A step of it moves twice the K/V bytes per
    // score, so it pays only when the longest row block is long (measured:
    // B1 H8 S4096 0.118 -> 0.096 ms; B1 H32 S1024 0.0367 -> 0.0383 ms).
    if (vec_scores && pr.causal && pr.N >= 2048 &&
        (int64_t)pr.B * pr.H * ((pr.M + bm - 1) / bm) <= cus)
      bm = fas::kFwdRows / 4;
  }
  // 128-row blocks that all run in one round: the 8-wave key-split writer
  // (two waves per SIMD on each block's even and odd key tiles).
  const int key_split2 = bm == fas::kFwdRows / 2 && vec_scores &&
                         (int64_t)pr.B * pr.H * ((pr.M + bm - 1) / bm) <= cus;
  fas::FwdParams p = fwd_params(a, pw, false, bm);
  p.key_split2 = key_split2;
  rescale_dropout(p, a);
  p.scores = static_cast<uint16_t*>(scores);
  p.ss0 = st[0];
  p.ss1 = st[1];
  p.ss2 = st[2];
  p.vec_scores = vec_scores;
  // The writer runs one workgroup per CU; with no more workgroups than CUs
  // they all run at once and each writes its own zero triangle.
  p.zero_self = (int64_t)p.nrb * (pr.B * pr.H / pw.pack) <= cus ? 1 : 0;
  return run_fwd(fn, p, pr, fas::kFwdScores, stream);
}

int fas_attention_with_scores(const fas_attn_args* a, void* scores, const int64_t st[4], void* ws,
                              size_t ws_bytes, void* stream) {
  return attention_with_scores_impl(a, scores, st, ws, ws_bytes, stream);
}

int fas_attention_scores(const fas_attn_args* a, void* scores, const int64_t st[4],
                         void* stream) {
  static const char* fn = "fas_attention_scores";
  Problem pr;
  int rc;
  if ((rc = check_shape(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H * pr.M * pr.N == 0) return FAS_OK;
  if ((rc = check_tensor(fn, "q", a->q, a->q_stride, pr.M, pr.D))) return rc;
  if ((rc = check_tensor(fn, "k", a->k, a->k_stride, pr.N, pr.D))) return rc;
  if ((rc = check_scores_out(fn, scores, st))) return rc;
  return run_scores(fn, a, pr, scores, st, false, stream);
}

int fas_attention_with_row_sum(const fas_attn_args* a, float* row_sum, const int64_t st[3],
                               void* ws, size_t ws_bytes, void* stream) {
  static const char* fn = "fas_attention_with_row_sum";
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H * pr.M == 0) return FAS_OK;
  if ((rc = check_out3(fn, "row_sum", row_sum, st))) return rc;
  const Workspace w = layout(FAS_VARIANT_ROW_SUM, pr, 0);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;
  fas::FwdParams p = fwd_params(a, pr, false, fas::kFwdRows);
  apply_split(p, w, ws);
  p.aux = row_sum;
  p.sa0 = st[0];
  p.sa1 = st[1];
  p.sa2 = st[2];
  return run_fwd(fn, p, pr, fas::kFwdRowSum, stream);
}

int fas_attention_with_col_sum(const fas_attn_args* a, float* col_sum, const int64_t st[3],
                               void* ws, size_t ws_bytes, void* stream) {
  return run_raw("fas_attention_with_col_sum", FAS_VARIANT_COL_SUM, a, 0, col_sum, st, ws,
                 ws_bytes, stream);
}

int fas_attention_with_col_sum_sequential(const fas_attn_args* a, float* col_sum,
                                          const int64_t st[3], void* ws, size_t ws_bytes,
                                          void* stream) {
  return run_raw("fas_attention_with_col_sum_sequential", FAS_VARIANT_COL_SUM_SEQUENTIAL, a, 0,
                 col_sum, st, ws, ws_bytes, stream);
}

int fas_attention_with_softmax_col_sum(const fas_attn_args* a, float* col_sum, const int64_t st[3],
                                       void* ws, size_t ws_bytes, void* stream) {
  return run_softmax("fas_attention_with_softmax_col_sum", FAS_VARIANT_SOFTMAX_COL_SUM, a, 0,
                     col_sum, st, ws, ws_bytes, stream);
}

int fas_attention_with_softmax_col_sum_noalloc(const fas_attn_args* a, float* col_sum,
                                               const int64_t st[3], void* stream) {
  static const char* fn = "fas_attention_with_softmax_col_sum_noalloc";
  Problem pr;
  int rc;
  // Every argument check first: the scratch lookup below is a HIP call.
  if ((rc = check_args(fn, a, &pr))) return rc;
  if ((rc = check_out3(fn, "sum output", col_sum, st))) return rc;
  // The layout is bounded by the scratch: a key split that would not fit
  // takes fewer, longer splits (or none); what remains must fit.
  const Workspace w = layout(FAS_VARIANT_SOFTMAX_COL_SUM, pr, 0, kNoAllocScratchBytes);
  if (w.total > kNoAllocScratchBytes)
    return fail(FAS_ERR_WORKSPACE, fn,
                "needs %zu bytes of scratch, more than the %zu this entry point holds; call "
                "fas_attention_with_softmax_col_sum with a caller workspace instead",
                w.total, kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(fn, &ws))) return rc;
  return run_softmax(fn, FAS_VARIANT_SOFTMAX_COL_SUM, a, 0, col_sum, st, ws, kNoAllocScratchBytes,
                     stream, kNoAllocScratchBytes);
}

int fas_attention_cross_token_qk_sum(const fas_attn_args* a, int64_t split, float* cross,
                                     const int64_t st[3], void* ws, size_t ws_bytes, void* stream) {
  return run_raw("fas_attention_cross_token_qk_sum", FAS_VARIANT_CROSS_QK_SUM, a, split, cross, st,
                 ws, ws_bytes, stream);
}

int fas_attention_cross_token_softmax_sum(const fas_attn_args* a, int64_t split, float* cross,
                                          const int64_t st[3], void* ws, size_t ws_bytes,
                                          void* stream) {
  return run_softmax("fas_attention_cross_token_softmax_sum", FAS_VARIANT_CROSS_SOFTMAX_SUM, a,
                     split, cross, st, ws, ws_bytes, stream);
}

int fas_attention_cross_token_softmax_sum_buffered(const fas_attn_args* a, int64_t split,
                                                   float* cross, const int64_t st[3], void* ws,
                                                   size_t ws_bytes, void* stream) {
  return run_softmax("fas_attention_cross_token_softmax_sum_buffered",
                     FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED, a, split, cross, st, ws, ws_bytes,
                     stream);
}

int fas_attention_forward(const fas_attn_args* a, float* lse, const int64_t st[3], void* ws,
                          size_t ws_bytes, void* stream) {
  static const char* fn = "fas_attention_forward";
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H * pr.M == 0) return FAS_OK;
  if ((rc = check_out3(fn, "lse", lse, st))) return rc;
  const Workspace w = layout(FAS_VARIANT_ATTENTION_FORWARD, pr, 0);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;
  KeepLayout kl;
  if ((rc = check_keep(fn, a, pr, &kl))) return rc;
  fas::FwdParams p = fwd_params(a, pr, false, fas::kFwdRows);
  rescale_dropout(p, a);
  apply_split(p, w, ws);
  p.lse_ln = lse;
  p.sl0 = st[0];
  p.sl1 = st[1];
  p.sl2 = st[2];
  if (pr.keep) {
    p.drop_bits = at<uint32_t>(a->keep_bits, kl.keys);
    if (kl.has_rows) p.drop_rows = at<uint32_t>(a->keep_bits, kl.rows);
    p.rows32 = (int)(bwd_mpad(pr) / 32);
  }
  return run_fwd(fn, p, pr, pr.keep ? fas::kFwdPlainKeepBits : fas::kFwdPlain, stream);
}

int fas_total_attention(const fas_attn_args* a, const float* lse, const int64_t lst[3],
                        float* total, const int64_t tst[3], void* stream) {
  static const char* fn = "fas_total_attention";
  Problem pr;
  int rc;
  if ((rc = check_shape(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H * pr.N == 0) return FAS_OK;
  if ((rc = check_out3(fn, "total", total, tst))) return rc;
  if (pr.M == 0) return zero_out3(fn, total, tst, pr.B, pr.H, pr.N, stream);
  if (lse == nullptr || lst == nullptr) return fail(FAS_ERR_INVALID, fn, "lse is NULL");
  if (strides_out_of_range(lst, 3))
    return fail(FAS_ERR_INVALID, fn, "lse strides must lie in [0, 2^46)");
  if ((rc = check_tensor(fn, "q", a->q, a->q_stride, pr.M, pr.D))) return rc;
  if ((rc = check_tensor(fn, "k", a->k, a->k_stride, pr.N, pr.D))) return rc;
  fas::ColsmParams c{};
  c.q = static_cast<const uint16_t*>(a->q);
  c.k = static_cast<const uint16_t*>(a->k);
  c.lse_ln = lse;
  c.sl0 = lst[0]; c.sl1 = lst[1]; c.sl2 = lst[2];
  c.out = total;
  c.so0 = tst[0]; c.so1 = tst[1]; c.so2 = tst[2];
  c.sq0 = a->q_stride[0]; c.sq1 = a->q_stride[1]; c.sq2 = a->q_stride[2];
  c.sk0 = a->k_stride[0]; c.sk1 = a->k_stride[1]; c.sk2 = a->k_stride[2];
  c.q_bytes = slice_bytes(pr.M, c.sq2, pr.D);
  c.k_bytes = slice_bytes(pr.N, c.sk2, pr.D);
  c.qneg = pr.sm_scale < 0.f ? 0x80008000u : 0u;
  c.B = pr.B; c.H = pr.H; c.G = pr.G; c.M = pr.M; c.N = pr.N;
  c.row_lo = 0;
  c.ncols = pr.N;
  c.causal = pr.causal;
  c.causal_off = pr.N - pr.M;
  c.nkb = (pr.N + 255) / 256;
  c.qk_scale = qk_scale_of(pr.sm_scale);
  // One output row per query head, no head split (no forward pass here to
  // clear tickets).
  c.fold = 1;
  c.nsplit = 1;
  return hip_status(fn, fas::launch_colsm(c, pr.dtype, pr.D, false,
                                          static_cast<hipStream_t>(stream)));
}

int fas_attention_backward(const fas_attn_args* a, const void* dout, const int64_t gst[4],
                           const float* lse, const int64_t lst[3], void* dq,
                           const int64_t qst[4], void* dk, const int64_t kst[4], void* dv,
                           const int64_t vst[4], void* ws, size_t ws_bytes, void* stream) {
  static const char* fn = "fas_attention_backward";
  Problem pr;
  int rc;
  if ((rc = check_args(fn, a, &pr))) return rc;
  if ((int64_t)pr.B * pr.H == 0) return FAS_OK;
  if (pr.M > 0) {
    if (gst == nullptr || qst == nullptr || lst == nullptr || lse == nullptr)
      return fail(FAS_ERR_INVALID, fn, "dout, dq or lse is NULL");
    if (strides_out_of_range(lst, 3))
      return fail(FAS_ERR_INVALID, fn, "lse strides must lie in [0, 2^46)");
    if ((rc = check_tensor(fn, "dout", dout, gst, pr.M, pr.D))) return rc;
    if ((rc = check_tensor(fn, "dq", dq, qst, pr.M, pr.D))) return rc;
  }
  if (pr.N > 0) {
    if (kst == nullptr || vst == nullptr) return fail(FAS_ERR_INVALID, fn, "dk or dv is NULL");
    if ((rc = check_tensor(fn, "dk", dk, kst, pr.N, pr.D))) return rc;
    if ((rc = check_tensor(fn, "dv", dv, vst, pr.N, pr.D))) return rc;
  }
  const Workspace w = layout(FAS_VARIANT_ATTENTION_BACKWARD, pr, 0, ws_bytes);
  if ((rc = check_workspace(fn, w, ws, ws_bytes))) return rc;
  KeepLayout kl;
  if ((rc = check_keep(fn, a, pr, &kl))) return rc;
  if (pr.M > (1 << 26)) return fail(FAS_ERR_UNSUPPORTED, fn, "seqlen_q exceeds 2^26");

  fas::BwdParams p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<const uint16_t*>(a->out);
  p.dout = static_cast<const uint16_t*>(dout);
  p.lse = lse;
  p.nl = at<float>(ws, w.nl);
  p.delta = at<float>(ws, w.delta);
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.part = w.has_part ? at<float>(ws, w.part) : nullptr;
  p.sq0 = a->q_stride[0]; p.sq1 = a->q_stride[1]; p.sq2 = a->q_stride[2];
  p.sk0 = a->k_stride[0]; p.sk1 = a->k_stride[1]; p.sk2 = a->k_stride[2];
  p.sv0 = a->v_stride[0]; p.sv1 = a->v_stride[1]; p.sv2 = a->v_stride[2];
  p.so0 = a->out_stride[0]; p.so1 = a->out_stride[1]; p.so2 = a->out_stride[2];
  if (pr.M > 0) {
    p.sg0 = gst[0]; p.sg1 = gst[1]; p.sg2 = gst[2];
    p.sdq0 = qst[0]; p.sdq1 = qst[1]; p.sdq2 = qst[2];
    p.sl0 = lst[0]; p.sl1 = lst[1]; p.sl2 = lst[2];
  }
  if (pr.N > 0) {
    p.sdk0 = kst[0]; p.sdk1 = kst[1]; p.sdk2 = kst[2];
    p.sdv0 = vst[0]; p.sdv1 = vst[1]; p.sdv2 = vst[2];
  }
  p.q_bytes = slice_bytes(pr.M, p.sq2, pr.D);
  p.k_bytes = slice_bytes(pr.N, p.sk2, pr.D);
  p.v_bytes = slice_bytes(pr.N, p.sv2, pr.D);
  p.g_bytes = slice_bytes(pr.M, p.sg2, pr.D);
  p.qneg = pr.sm_scale < 0.f ? 0x80008000u : 0u;
  p.B = pr.B; p.H = pr.H; p.G = pr.G; p.Hk = pr.Hk; p.M = pr.M; p.N = pr.N;
  p.Mpad = (int)bwd_mpad(pr);
  p.causal = pr.causal;
  p.causal_off = pr.N - pr.M;
  p.nkb = (int)bwd_nkb(pr);
  p.nrb = p.Mpad / fas::kBwdBlock;
  p.nprep = (p.Mpad + (2048 / pr.D) - 1) / (2048 / pr.D);
  p.partial = bwd_partial(pr) ? 1 : 0;
  p.n32 = (pr.N + 31) / 32;
  if (w.has_bits) p.drop_bits = at<uint32_t>(ws, w.bits);
  if (w.has_ds) {
    p.ds = at<uint16_t>(ws, w.ds);
    p.ds_head = w.ds_head;
    p.ds_a = (int)bwd_ds_a(pr);
  }
  if (pr.keep) {
    // The forward's bits: dK/dV reads the key-major words, dQ the row blocks.
    p.keep_keys = at<uint32_t>(a->keep_bits, kl.keys);
    p.drop_bits = kl.has_rows ? at<uint32_t>(a->keep_bits, kl.rows) : nullptr;
  }
  p.sm_scale = std::fabs(pr.sm_scale);
  p.scale_signed = pr.sm_scale;
  p.qk_scale = qk_scale_of(pr.sm_scale);
  p.dropout = a->dropout_p > 0.f ? 1 : 0;
  p.drop = drop_params(a, pr);
  if (p.dropout) p.drop.scale = 1.f / (1.f - a->dropout_p);
  return hip_status(fn, fas::launch_bwd(p, pr.dtype, pr.D, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
