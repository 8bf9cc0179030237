// Exercises the host side of the C ABI (include/fas.h) on the CPU, built
// with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_host_sanitize.py from a host-only compile of the library's
// sources: no GPU, no device code.  Three parts:
//   1. fas_workspace_bytes over every variant and a sweep of shapes up to
//      the largest sizes the ABI accepts, which drives the 64-bit size and
//      offset arithmetic of the workspace layout, the key-split plan, the
//      backward's dS blocks and the keep-bit buffer;
//   2. every entry point with each kind of invalid request, which must be
//      rejected with its status and a message naming the entry point;
//   3. every entry point with valid small problems over host buffers of the
//      exact sizes: the request passes validation and parameter packing and
//      then fails at the launch (FAS_ERR_HIP, no device), so everything
//      before the launch runs under the sanitizers.
// Exit status 0 when every check holds; the sanitizers abort on their own.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "fas.h"

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond, ...)                                              \
  do {                                                                \
    ++g_checks;                                                       \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);       \
      std::fprintf(stderr, __VA_ARGS__);                              \
      std::fputc('\n', stderr);                                       \
      ++g_failures;                                                   \
    }                                                                 \
  } while (0)

constexpr size_t kBad = (size_t)-1;

// A 256-byte aligned host allocation of exactly `bytes` bytes (at least 1).
struct Buf {
  void* p = nullptr;
  explicit Buf(size_t bytes) {
    const size_t n = ((bytes ? bytes : 1) + 255) / 256 * 256;
    p = std::aligned_alloc(256, n);
  }
  ~Buf() { std::free(p); }
  Buf(const Buf&) = delete;
  Buf& operator=(const Buf&) = delete;
};

void contiguous(int64_t (&st)[4], int64_t H, int64_t L, int64_t D) {
  st[3] = 1;
  st[2] = D;
  st[1] = L * D;
  st[0] = H * L * D;
}

fas_attn_args shape_args(int64_t B, int64_t Hq, int64_t Hk, int64_t M, int64_t N, int64_t D,
                         int causal, float dropout_p = 0.f) {
  fas_attn_args a;
  std::memset(&a, 0, sizeof a);
  a.dtype = FAS_DTYPE_F16;
  a.causal = causal;
  a.sm_scale = 0.125f;
  a.batch = B;
  a.heads_q = Hq;
  a.heads_k = Hk;
  a.seqlen_q = M;
  a.seqlen_k = N;
  a.head_dim = D;
  contiguous(a.q_stride, Hq, M, D);
  contiguous(a.out_stride, Hq, M, D);
  contiguous(a.k_stride, Hk, N, D);
  contiguous(a.v_stride, Hk, N, D);
  a.dropout_p = dropout_p;
  a.dropout_seed = 0x1234567890abcdefull;
  a.dropout_offset = 96;
  return a;
}

// ------------------------------------------------------------------ part 1

void sweep_workspace_sizes() {
  const int64_t lens[] = {0, 1, 31, 32, 33, 255, 256, 257, 4096, 65536, 1 << 20, 1 << 28};
  const int64_t heads[][3] = {{1, 1, 1}, {1, 28, 4}, {3, 32, 8}, {1, 128, 128}, {256, 65536, 1},
                              {1, 1 << 24, 1 << 23}};
  const int64_t dims[] = {16, 128};
  for (int variant = FAS_VARIANT_SCORES; variant <= FAS_VARIANT_KEEP_BITS; ++variant)
    for (const auto& h : heads)
      for (int64_t M : lens)
        for (int64_t N : lens)
          for (int64_t D : dims)
            for (int causal = 0; causal < 2; ++causal)
              for (int drop = 0; drop < 2; ++drop) {
                fas_attn_args a = shape_args(h[0], h[1], h[2], M, N, D, causal, drop ? 0.1f : 0.f);
                const int64_t splits[] = {0, 1, N / 2, N};
                for (int64_t split : splits) {
                  const size_t w = fas_workspace_bytes(variant, &a, split);
                  if (w == kBad) {
                    CHECK(std::strlen(fas_last_error()) > 0,
                          "variant %d B%lld H%lld M%lld N%lld: (size_t)-1 without a message",
                          variant, (long long)h[0], (long long)h[1], (long long)M, (long long)N);
                    continue;
                  }
                  CHECK(w % 256 == 0, "variant %d: workspace %zu not a multiple of 256", variant, w);
                  // The softmax variants hold one fp32 normalizer per query row.
                  const bool softmax = variant == FAS_VARIANT_SOFTMAX_COL_SUM ||
                                       variant == FAS_VARIANT_CROSS_SOFTMAX_SUM ||
                                       variant == FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED;
                  if (softmax) {
                    const unsigned __int128 lse = (unsigned __int128)h[0] * h[1] * M * 4;
                    CHECK((unsigned __int128)w >= lse,
                          "variant %d B%lld H%lld M%lld N%lld: workspace %zu below the row "
                          "normalizers",
                          variant, (long long)h[0], (long long)h[1], (long long)M, (long long)N, w);
                  }
                }
              }
  // Requests the ABI rejects outright.
  fas_attn_args a = shape_args(1, 4, 4, 64, 64, 64, 1);
  CHECK(fas_workspace_bytes(-1, &a, 0) == kBad, "variant -1 accepted");
  CHECK(fas_workspace_bytes(FAS_VARIANT_KEEP_BITS + 1, &a, 0) == kBad, "variant 11 accepted");
  CHECK(fas_workspace_bytes(FAS_VARIANT_SCORES, nullptr, 0) == kBad, "NULL args accepted");
  a.head_dim = 48;
  CHECK(fas_workspace_bytes(FAS_VARIANT_SCORES, &a, 0) == kBad, "head_dim 48 accepted");
}

// ------------------------------------------------------------------ part 2/3

// Host tensors of one problem, exact sizes.
struct Problem {
  fas_attn_args a;
  int64_t B, Hq, Hk, M, N, D;
  Buf q, k, v, o, side, side2, dq, dk, dv, dout, lse;
  int64_t side_st[4], lse_st[3], dq_st[4], dk_st[4], dv_st[4], do_st[4];
  Problem(int64_t B_, int64_t Hq_, int64_t Hk_, int64_t M_, int64_t N_, int64_t D_, int causal)
      : B(B_), Hq(Hq_), Hk(Hk_), M(M_), N(N_), D(D_),
        q((size_t)(B_ * Hq_ * M_ * D_ * 2)),
        k((size_t)(B_ * Hk_ * N_ * D_ * 2)),
        v((size_t)(B_ * Hk_ * N_ * D_ * 2)),
        o((size_t)(B_ * Hq_ * M_ * D_ * 2)),
        side((size_t)(B_ * Hq_ * M_ * N_ * 2 + B_ * Hq_ * (M_ + N_) * 4)),
        side2((size_t)(B_ * Hq_ * N_ * 4)),
        dq((size_t)(B_ * Hq_ * M_ * D_ * 2)),
        dk((size_t)(B_ * Hk_ * N_ * D_ * 2)),
        dv((size_t)(B_ * Hk_ * N_ * D_ * 2)),
        dout((size_t)(B_ * Hq_ * M_ * D_ * 2)),
        lse((size_t)(B_ * Hq_ * M_ * 4)) {
    a = shape_args(B, Hq, Hk, M, N, D, causal);
    a.q = q.p;
    a.k = k.p;
    a.v = v.p;
    a.out = o.p;
    lse_st[0] = Hq * M;
    lse_st[1] = M;
    lse_st[2] = 1;
    contiguous(dq_st, Hq, M, D);
    contiguous(do_st, Hq, M, D);
    contiguous(dk_st, Hk, N, D);
    contiguous(dv_st, Hk, N, D);
  }
};

using Runner = int (*)(Problem&, void* ws, size_t ws_bytes, int64_t split);

int run_scores(Problem& p, void* ws, size_t n, int64_t) {
  int64_t st[4] = {p.Hq * p.M * p.N, p.M * p.N, p.N, 1};
  return fas_attention_with_scores(&p.a, p.side.p, st, ws, n, nullptr);
}
int run_scores_only(Problem& p, void*, size_t, int64_t) {
  int64_t st[4] = {p.Hq * p.M * p.N, p.M * p.N, p.N, 1};
  return fas_attention_scores(&p.a, p.side.p, st, nullptr);
}
int run_row(Problem& p, void* ws, size_t n, int64_t) {
  int64_t st[3] = {p.Hq * p.M, p.M, 1};
  return fas_attention_with_row_sum(&p.a, static_cast<float*>(p.side.p), st, ws, n, nullptr);
}
int64_t col_stride[3];
float* cols(Problem& p, int64_t ncols) {
  col_stride[0] = p.Hk * ncols;
  col_stride[1] = ncols;
  col_stride[2] = 1;
  return static_cast<float*>(p.side2.p);
}
int run_col(Problem& p, void* ws, size_t n, int64_t) {
  return fas_attention_with_col_sum(&p.a, cols(p, p.N), col_stride, ws, n, nullptr);
}
int run_col_seq(Problem& p, void* ws, size_t n, int64_t) {
  return fas_attention_with_col_sum_sequential(&p.a, cols(p, p.N), col_stride, ws, n, nullptr);
}
int run_colsm(Problem& p, void* ws, size_t n, int64_t) {
  return fas_attention_with_softmax_col_sum(&p.a, cols(p, p.N), col_stride, ws, n, nullptr);
}
int run_colsm_noalloc(Problem& p, void*, size_t, int64_t) {
  return fas_attention_with_softmax_col_sum_noalloc(&p.a, cols(p, p.N), col_stride, nullptr);
}
int run_xqk(Problem& p, void* ws, size_t n, int64_t split) {
  return fas_attention_cross_token_qk_sum(&p.a, split, cols(p, split), col_stride, ws, n, nullptr);
}
int run_xsm(Problem& p, void* ws, size_t n, int64_t split) {
  return fas_attention_cross_token_softmax_sum(&p.a, split, cols(p, split), col_stride, ws, n,
                                               nullptr);
}
int run_xbuf(Problem& p, void* ws, size_t n, int64_t split) {
  return fas_attention_cross_token_softmax_sum_buffered(&p.a, split, cols(p, split), col_stride,
                                                        ws, n, nullptr);
}
int run_fwd(Problem& p, void* ws, size_t n, int64_t) {
  return fas_attention_forward(&p.a, static_cast<float*>(p.lse.p), p.lse_st, ws, n, nullptr);
}
int run_total(Problem& p, void*, size_t, int64_t) {
  int64_t st[3] = {p.Hq * p.N, p.N, 1};
  return fas_total_attention(&p.a, static_cast<const float*>(p.lse.p), p.lse_st,
                             static_cast<float*>(p.side2.p), st, nullptr);
}
int run_bwd(Problem& p, void* ws, size_t n, int64_t) {
  return fas_attention_backward(&p.a, p.dout.p, p.do_st, static_cast<const float*>(p.lse.p),
                                p.lse_st, p.dq.p, p.dq_st, p.dk.p, p.dk_st, p.dv.p, p.dv_st, ws, n,
                                nullptr);
}

struct EntryPoint {
  const char* name;
  Runner run;
  int variant;  // workspace variant, -1: none
  bool split;   // takes a split index
  bool qk_only; // reads only q and k (v and out are not checked)
};

const EntryPoint kEntryPoints[] = {
    {"fas_attention_with_scores", run_scores, FAS_VARIANT_SCORES, false},
    {"fas_attention_scores", run_scores_only, -1, false, true},
    {"fas_attention_with_row_sum", run_row, FAS_VARIANT_ROW_SUM, false},
    {"fas_attention_with_col_sum", run_col, FAS_VARIANT_COL_SUM, false},
    {"fas_attention_with_col_sum_sequential", run_col_seq, FAS_VARIANT_COL_SUM_SEQUENTIAL, false},
    {"fas_attention_with_softmax_col_sum", run_colsm, FAS_VARIANT_SOFTMAX_COL_SUM, false},
    {"fas_attention_with_softmax_col_sum_noalloc", run_colsm_noalloc, -1, false},
    {"fas_attention_cross_token_qk_sum", run_xqk, FAS_VARIANT_CROSS_QK_SUM, true},
    {"fas_attention_cross_token_softmax_sum", run_xsm, FAS_VARIANT_CROSS_SOFTMAX_SUM, true},
    {"fas_attention_cross_token_softmax_sum_buffered", run_xbuf,
     FAS_VARIANT_CROSS_SOFTMAX_SUM_BUFFERED, true},
    {"fas_attention_forward", run_fwd, FAS_VARIANT_ATTENTION_FORWARD, false},
    {"fas_total_attention", run_total, -1, false, true},
    {"fas_attention_backward", run_bwd, FAS_VARIANT_ATTENTION_BACKWARD, false},
};

bool names(const EntryPoint& e) {
  return std::string(fas_last_error()).find(e.name) != std::string::npos;
}

// Calls e on p with its full workspace (none when the size query itself
// rejects the request: the entry point must then reject it too); returns
// the status.
int call_with_workspace(const EntryPoint& e, Problem& p, int64_t split) {
  size_t n = 0;
  if (e.variant >= 0) {
    n = fas_workspace_bytes(e.variant, &p.a, split);
    if (n == kBad) n = 0;
  }
  Buf ws(n);
  return e.run(p, n ? ws.p : nullptr, n, split);
}

void invalid_requests() {
  for (const EntryPoint& e : kEntryPoints) {
    const int64_t split = e.split ? 40 : 0;
    auto expect = [&](const char* what, int rc, int want) {
      CHECK(rc == want, "%s, %s: status %d, expected %d (%s)", e.name, what, rc, want,
            fas_last_error());
      CHECK(rc == FAS_OK || names(e), "%s, %s: message \"%s\" does not name it", e.name, what,
            fas_last_error());
    };
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.dtype = 7;
      expect("dtype 7", call_with_workspace(e, p, split), FAS_ERR_UNSUPPORTED);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.causal = 2;
      expect("causal 2", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 3, 96, 80, 64, 1);
      expect("heads 4 / 3", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.sm_scale = std::numeric_limits<float>::quiet_NaN();
      expect("NaN sm_scale", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.dropout_p = 1.f;
      expect("dropout_p 1", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.seqlen_q = -1;
      expect("negative M", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.seqlen_k = (int64_t)1 << 40;
      expect("N = 2^40", call_with_workspace(e, p, split), FAS_ERR_UNSUPPORTED);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.q = nullptr;
      expect("NULL q", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.q_stride[3] = 2;
      expect("q stride[3] 2", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.k = static_cast<const char*>(p.a.k) + 2;
      expect("k misaligned", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    if (!e.qk_only) {
      // Row strides from the top of the int64 range: the span check must
      // not overflow.
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.v_stride[2] = INT64_MAX - 7;
      p.a.v_stride[1] = INT64_MAX - 7;
      p.a.v_stride[0] = INT64_MAX - 7;
      expect("v stride near 2^63", call_with_workspace(e, p, split), FAS_ERR_UNSUPPORTED);
    }
    if (!e.qk_only) {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.out_stride[2] = 32;
      expect("out rows overlap", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    {
      // k's row stride at the top of the int64 range (k is read by every
      // entry point).
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.k_stride[2] = INT64_MAX - 7;
      expect("k row stride near 2^63", call_with_workspace(e, p, split), FAS_ERR_UNSUPPORTED);
    }
    {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      p.a.q_stride[1] = -64 * 96;
      expect("negative q head stride", call_with_workspace(e, p, split), FAS_ERR_INVALID);
    }
    if (e.split) {
      Problem p(1, 4, 2, 96, 80, 64, 1);
      expect("split 0", call_with_workspace(e, p, 0), FAS_ERR_INVALID);
      Problem p2(1, 4, 2, 96, 80, 64, 1);
      expect("split N + 1", call_with_workspace(e, p2, 81), FAS_ERR_INVALID);
    }
    if (e.variant >= 0) {
      Problem p(1, 4, 2, 96, 1024, 64, 1);
      const size_t n = fas_workspace_bytes(e.variant, &p.a, split);
      if (n != kBad && n > 0) {
        Buf ws(n + 256);
        // The backward takes any size from the one without stored dS up.
        const size_t need = e.variant == FAS_VARIANT_ATTENTION_BACKWARD
                                ? fas_workspace_bytes(e.variant, &p.a, 1)
                                : n;
        expect("workspace one byte short", e.run(p, ws.p, need - 1, split), FAS_ERR_WORKSPACE);
        expect("no workspace", e.run(p, nullptr, n, split), FAS_ERR_WORKSPACE);
        expect("misaligned workspace", e.run(p, static_cast<char*>(ws.p) + 16, n, split),
               FAS_ERR_INVALID);
      }
    }
  }
  // NULL args.
  int64_t st4[4] = {0, 0, 0, 1};
  CHECK(fas_attention_with_scores(nullptr, nullptr, st4, nullptr, 0, nullptr) == FAS_ERR_INVALID,
        "NULL args accepted");
}

void valid_requests_fail_at_launch() {
  struct Shape {
    int64_t B, Hq, Hk, M, N, D;
    int causal;
  };
  const Shape shapes[] = {
      {1, 4, 4, 256, 256, 64, 1}, {2, 4, 2, 200, 300, 128, 1}, {1, 8, 1, 130, 100, 32, 1},
      {1, 2, 2, 77, 333, 16, 0},  {1, 4, 2, 32, 4096, 128, 1}, {1, 2, 2, 1, 64, 128, 1},
      {1, 2, 2, 64, 1, 64, 0},    {1, 7, 1, 0, 64, 64, 1},     {1, 2, 2, 64, 0, 64, 1},
  };
  for (const Shape& s : shapes)
    for (const EntryPoint& e : kEntryPoints)
      for (int drop = 0; drop < 2; ++drop) {
        Problem p(s.B, s.Hq, s.Hk, s.M, s.N, s.D, s.causal);
        if (drop) p.a.dropout_p = 0.2f;
        const int64_t split = e.split ? (s.N > 1 ? s.N / 2 : 1) : 0;
        if (e.split && s.N == 0) continue;
        const int rc = call_with_workspace(e, p, split);
        CHECK(rc == FAS_OK || rc == FAS_ERR_HIP,
              "%s B%lld H%lld/%lld M%lld N%lld D%lld causal %d dropout %d: status %d (%s)", e.name,
              (long long)s.B, (long long)s.Hq, (long long)s.Hk, (long long)s.M, (long long)s.N,
              (long long)s.D, s.causal, drop, rc, fas_last_error());
      }
}

}  // namespace

int main() {
  CHECK(fas_abi_version() == FAS_ABI_VERSION, "ABI version %d", fas_abi_version());
  sweep_workspace_sizes();
  invalid_requests();
  valid_requests_fail_at_launch();
  std::printf("host driver: %d checks, %d failures\n", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
