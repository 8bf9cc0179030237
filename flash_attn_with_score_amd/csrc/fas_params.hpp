// Kernel-side parameter blocks shared by the host dispatcher (fas_api.cpp)
// and the gfx950 kernels (fas_fwd.hpp, fas_sums.hpp).  Plain data only.
#pragma once
#include <stdint.h>

namespace fas {

// Side product of the forward kernel (fas_fwd.hpp).
enum FwdMode : int {
  kFwdPlain = 0,   // output (+ optional base-2 LSE)
  kFwdScores = 1,  // + (B,H,M,N) scaled scores, masked -> 0
  kFwdRowSum = 2,  // + (B,H,M) row sums of scaled scores
  kFwdRegion = 3,  // + fp32 raw scores of rows >= split, keys < split
  kFwdPlainKeepBits = 4  // kFwdPlain with dropout, storing the keep decisions (drop_bits)
};

// Dropout of the attention weights with the reference's random stream:
// element (b, h, i, j) is kept iff Triton's tl.rand(seed, offset + ((b*H + h)
// *M + i)*N + j, n_rounds=6) > p (attention_with_scores.py:70-75, 173-176).
// The index is taken mod 2^32 (the reference's int32 arithmetic) and the
// counter's high word is used only for offsets >= 2^31 (a 64-bit offset).
//
// tl.rand is Philox4x32-6 on counter (x0, w1, 0, 0): x0 = (offset + index)
// mod 2^32, w1 = 0 for an int32 offset, else the offset's high word plus the
// carry of that sum.  Round 0 multiplies word 2 = 0, so it leaves (w1 ^ k0,
// 0, hi(A x0) ^ k1, lo(A x0)); round 1's word-0 product A (w1 ^ k0) then
// takes one of two wave-uniform values, which the host supplies.
constexpr uint32_t kPhiloxMulA = 0xD2511F53u;   // word 0 multiplier
constexpr uint32_t kPhiloxMulB = 0xCD9E8D57u;   // word 2 multiplier
constexpr uint32_t kPhiloxWeylA = 0x9E3779B9u;  // key word 0 increment
constexpr uint32_t kPhiloxWeylB = 0xBB67AE85u;  // key word 1 increment
struct DropParams {
  uint32_t off_lo;     // offset mod 2^32: x0 = off_lo + index
  uint32_t carry_lim;  // w1 is w1[1] iff x0 < carry_lim (the sum carried), else w1[0]
  uint32_t k0, k1;     // Philox key: the seed's low and high words
  // Round 1's word-0 product A (w1 ^ k0) for w1 without the carry, and the
  // exclusive or of each half with its value for w1 with the carry:
  uint32_t r1_hi, r1_hi_carry;  // hi(A (w1 ^ k0)) ^ (k1 + kPhiloxWeylB)
  uint32_t r1_lo, r1_lo_carry;  // lo(A (w1 ^ k0))
  // Keep iff (word 0 - keep_lo) mod 2^32 < keep_span: Triton's uniform of
  // word x exceeds p exactly on an interval of x mod 2^32 (host-made).
  uint32_t keep_lo, keep_span;
  int n;               // N of the element index
  float scale;         // O multiplier: 1/(1-p) where the reference rescales, else 1
};

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse2;       // optional (B*H, M) contiguous: m*qk_scale + log2(l), +inf for empty rows
  float* lse_ln;     // optional (B,H,M) strided: m*sm_scale + ln(l), -inf for empty rows
  uint16_t* scores;  // kFwdScores
  float* aux;        // kFwdRowSum: (B,H,M) strided
  // kFwdRegion: the region (rows >= split, keys < split) as fp16 base-2
  // exponents y = (s - t) * qk_scale relative to t, the row's maximum over
  // the region keys of its 64-key tile: region (B*H, M - split, split)
  // contiguous, region_m (ceil(split / 64), region_rows) the t * qk_scale,
  // tile-major so a wave's rows of one tile are adjacent.
  uint16_t* region;
  float* region_m;
  int64_t region_rows;  // B*H*(M - split)
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t sv0, sv1, sv2;
  int64_t so0, so1, so2;
  int64_t ss0, ss1, ss2;
  int64_t sa0, sa1, sa2;
  int64_t sl0, sl1, sl2;  // lse_ln strides
  uint32_t q_bytes, k_bytes, v_bytes, o_bytes;  // buffer extents from (b, first packed head)
  uint32_t qneg;     // 0x80008000 to negate q (negative sm_scale), else 0
  int B, H, G, M, N, split;
  int causal;
  int causal_off;    // key j admissible for query i iff causal_off + i >= j
  // GQA packing: a workgroup serves `pack` consecutive query heads of one
  // KV head (pack divides G; 1 = one head per workgroup).  Its rows are
  // virtual rows v = pos * pack + j (position pos of head h0 + j), so every
  // K/V tile it stages in LDS is used by all packed heads.
  int pack;
  int pack_shift;    // log2(pack) when pack is 1, 2, 4 or 8 (the score writer's packings)
  int nrb;           // virtual row blocks per group of `pack` heads
  int bm;            // rows per workgroup (32 per wave; the score writer takes 128 or 256)
  int vec_scores;    // scores rows 16-byte aligned and N % 8 == 0
  int zero_self;     // score writer: 1 = a workgroup writes its own row block's zeros
                     // (all workgroups run at once), 0 = its mirror row block's
  int vec_region;    // split % 8 == 0
  int key_split2;    // score writer with 128-row blocks: 1 = the 8-wave key-split
                     // instance (wave pairs take the even and odd key tiles)
  int dropout;       // 1: the dropout instances (modes other than kFwdRegion)
  DropParams drop;   // scale also applies in the key-split combine (1 without dropout)
  // kFwdPlainKeepBits: the keep decisions as bits, word
  // ((b*H + h) * ceil(M/32) + i/32) * N + j holding rows 32*(i/32) .. +31
  // of key j (bit i % 32); and, when drop_rows is set (attention's forward),
  // again in the backward's row blocks, word
  // (((b*H + h) * rows32 + i/32) * ceil(N/32) + j/32) * 32 + i % 32 (bit j % 32).
  uint32_t* drop_bits;
  uint32_t* drop_rows;
  int rows32;        // the backward's padded rows / 32
  // Split over keys (kFwdPlain, kFwdRowSum): nsplit workgroups per row block,
  // each taking tps key tiles and writing fp32 partials at row pitch Mpad
  // (= nrb * rows per workgroup); a combine pass merges them.
  int nsplit;        // 1 = no split
  int tps;
  int Mpad;          // >= M: row pitch of the partials (positions, not virtual rows)
  float* part_o;     // (B*H, nsplit, Mpad, D) unnormalised O
  float* part_m;     // (B*H, nsplit, Mpad) base-2 exponent offset, -inf if none
  float* part_l;     // (B*H, nsplit, Mpad) sum of the weights
  float* part_r;     // (B*H, nsplit, Mpad) raw row sums (kFwdRowSum)
  float sm_scale;    // |sm_scale|
  float qk_scale;    // |sm_scale| * log2(e)
  // Words workgroup 0 sets to zero before anything else: the tickets of the
  // column pass that follows on the same stream (ColsmParams.ticket).
  uint32_t* zero_words;
  int n_zero_words;
};

}  // namespace fas

namespace fas {

// Key-outer column sums of the softmax weights (fas_sums.hpp).
struct ColsmParams {
  const uint16_t* q;
  const uint16_t* k;
  const float* lse2;     // (B*H, M) base-2 LSE from the forward pass
  const float* lse_ln;   // or, when set, the natural-log normalizer (B,H,M) strided
  int64_t sl0, sl1, sl2;
  const uint16_t* region;  // buffered source: fp16 exponents (FwdParams::region)
  const float* region_m;   // and their per-64-key-tile, per-row offsets
  int64_t region_rows;
  float* out;            // (B, H / fold, ncols) strided output
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t so0, so1, so2;
  uint32_t q_bytes, k_bytes;
  uint32_t qneg;
  int B, H, G, M, N;
  // Head folding: output column group og = b * (H / fold) + ho sums the
  // query heads ho*fold .. ho*fold + fold - 1 (fold = G: the column sums per
  // KV head; fold = 1: per query head, total_attention).  The fold's heads
  // are dealt to nsplit workgroups per key block (pair), split s taking
  // heads s, s + nsplit, ...; with nsplit > 1 each writes its column sums to
  // part[(og * nsplit + s) * ncols + key] and bumps ticket[og * nunits +
  // unit] (unit = the key block or pair), and the workgroup that brings the
  // ticket to nsplit adds the nsplit partials in split order into out.
  // The tickets start at 0: the forward pass of the same call clears them
  // (FwdParams.zero_words).
  int fold, nsplit;
  float* part;
  uint32_t* ticket;
  int row_lo;            // first query row that contributes (0, or split)
  int ncols;             // keys summed: N, or split
  int split;             // region row offset / pitch (buffered)
  int causal, causal_off;
  int nkb;               // key blocks
  float qk_scale;        // |sm_scale| * log2(e)
  int dropout;           // 1: weights pass through the dropout mask (Philox), 2: through
                         // the forward's keep bits (drop_bits, FwdParams layout)
  DropParams drop;
  const uint32_t* drop_bits;
};

// Raw-score column sums by linearity: sum_i (q_i . k_j) = (sum_i q_i) . k_j.
struct RawParams {
  const uint16_t* q;
  const uint16_t* k;
  float* bsum;           // (B*Hk, nblk + 1, D) fp32 per-block sums of q (slot nblk unused)
  float* out;            // (B, Hk, ncols) strided
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t so0, so1, so2;
  int B, H, G, Hk, M, N, D;
  int row_lo;            // rows [row_lo, M) contribute
  int nblk;              // 64-row blocks of [row_lo, M)
  int ncols;
  int causal, causal_off;
  int nextra;            // causal: key blocks below causal_off (all rows admissible)
  int kgroups;           // full sums: 64-key groups per workgroup (set by the launcher)
  float sm_scale;        // signed
};

// Backward pass of attention() (fas_bwd.hpp).
struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;      // natural-log normalizer L (B,H,M) strided, -inf for empty rows
  float* nl;             // workspace (B*H, Mpad): -L*log2(e), -inf for rows that see no key
  float* delta;          // workspace (B*H, Mpad): -sum_d O*dO (0 past M)
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* part;           // workspace (B*H, N, 2D) fp32 per-query-head dK | dV (partial mode)
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t sv0, sv1, sv2;
  int64_t so0, so1, so2;
  int64_t sg0, sg1, sg2;   // dout
  int64_t sdq0, sdq1, sdq2;
  int64_t sdk0, sdk1, sdk2;
  int64_t sdv0, sdv1, sdv2;
  int64_t sl0, sl1, sl2;
  uint32_t q_bytes, k_bytes, v_bytes, g_bytes;
  uint32_t qneg;          // sign flip of the operand that carries sm_scale's sign
  int B, H, G, Hk, M, N, Mpad;
  int causal, causal_off;
  int nkb;               // 128-key blocks (dK/dV kernel)
  int nrb;               // 128-row blocks (dQ kernel)
  int nprep;             // row groups per (b, head) of the prep kernel
  int partial;           // dK/dV kernel: one query head per workgroup, fp32 partials
  float sm_scale;        // |sm_scale|
  float scale_signed;    // sm_scale with its sign: dQ = s sum_j dS_ij k_j, dK = s sum_i dS_ij q_i
  float qk_scale;        // |sm_scale| * log2(e)
  int dropout;           // 1: the dropout instances (flash.py:653-659, 705-731, 843-890)
  DropParams drop;       // scale = 1/(1-p)
  // Optional with dropout: the dK/dV kernel stores its keep decisions for
  // the dQ kernel, word (((b*H + h) * Mpad/32 + i/32) * n32 + j/32) * 32 +
  // i % 32 holding keys 32*(j/32) .. +31 of row i (bit j % 32): the 32 rows
  // of a block are consecutive words; null: dQ evaluates Philox.
  uint32_t* drop_bits;
  int n32;               // ceil(N / 32)
  // The forward's key-major keep words (FwdParams.drop_bits layout), when
  // the caller kept them: the dK/dV kernel reads them instead of evaluating
  // Philox and does not write drop_bits (which then holds the forward's
  // row blocks).
  const uint32_t* keep_keys;
  // Optional: dS = P (dP - delta) in the input type, stored by the dK/dV
  // kernel and read by bwd_dq_ds_kernel (dQ = s dS K, no recomputation).
  // Per (b, h): ds_head blocks of 32 rows x 32 keys, 2 KiB each, only the
  // blocks a causal mask leaves visible (ds_block_start); null: bwd_dq_kernel
  // recomputes S and dP.
  uint16_t* ds;
  int64_t ds_head;       // blocks per (b, h); ds_head * 2048 < 2^31
  int ds_a;              // visible 32-key blocks of 32-row block r: clamp(r + ds_a, 0, n32)
};

// First dS block of 32-row block r in its head's compact layout: the sum over
// r' < r of clamp(r' + a, 0, n), the visible 32-key blocks of each earlier
// row block (a = n for no mask).  Closed form: rows with r' + a <= 0 add
// nothing, rows with r' + a >= n add n, the rows between an arithmetic run.
__host__ __device__ inline int64_t ds_block_start(int64_t r, int64_t a, int64_t n) {
  const int64_t lo = a < 0 ? -a : 0;
  const int64_t hi = n - a > lo ? n - a : lo;
  const int64_t r1 = r < lo ? lo : (r > hi ? hi : r);
  const int64_t up = r > hi ? r - hi : 0;
  return (r1 - lo) * (lo + r1 - 1 + 2 * a) / 2 + n * up;
}
// The same in 32-bit arithmetic, for heads whose blocks number below 2^20
// (every term and partial sum then stays below 2^21).
__host__ __device__ inline int ds_block_start32(int r, int a, int n) {
  const int lo = a < 0 ? -a : 0;
  const int hi = n - a > lo ? n - a : lo;
  const int r1 = r < lo ? lo : (r > hi ? hi : r);
  const int up = r > hi ? r - hi : 0;
  return (r1 - lo) * (lo + r1 - 1 + 2 * a) / 2 + n * up;
}

}  // namespace fas

namespace fas {

// Scores alone (fas_scores.hpp): (q . k) * sm_scale in the input dtype.
struct ScoresParams {
  const uint16_t* q;
  const uint16_t* k;
  uint16_t* scores;
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t ss0, ss1, ss2;
  uint32_t q_bytes, k_bytes;
  int B, H, G, M, N;
  int mask;           // 1: causal / key-range mask, masked entries written as 0
  int causal_off;     // key j admissible for query i iff causal_off + i >= j
  int nkb;            // 256-key blocks (512-key blocks for the resident-Q kernel)
  int nrs;            // row ranges per key block
  int spr;            // 64-row steps per row range
  int ngrp;           // > 0: resident-Q kernel with ngrp workgroups per head group
  // Resident-Q kernel: a group is 2^pshift consecutive query heads of one KV
  // head (pshift > 0 only under GQA, 2^pshift * M <= 512), its virtual rows
  // v = m * 2^pshift + j holding position m of head h0 + j.
  int pshift;
  int vec;            // base and row strides 16-byte aligned, N % 8 == 0: 16-byte stores
  float sm_scale;     // signed
};

}  // namespace fas
