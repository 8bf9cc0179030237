// gfx950 flash-attention forward with fused side products.
//
// One template covers the forward pass of every entry point of the
// reference's Triton family (FA2 forward state attention_with_scores.py:82-198
// and its copies in the other kernels); what differs is the side product
// written from the score tile while it is still in registers:
//
//   kFwdPlain   output (and optionally the base-2 log-sum-exp per row)
//   kFwdScores  + the (B,H,M,N) matrix (q.k)*sm_scale, masked -> 0
//               (attention_with_scores.py:141-162), including the never
//               computed causal upper triangle, written as zeros
//   kFwdRowSum  + per-row sum of masked scaled scores
//               (attention_with_row_sum.py:146-156)
//   kFwdRegion  + the scores of the region rows >= split, keys < split, the
//               first pass of the buffered cross-token softmax sum
//               (attention_cross_token_softmax_sum.py:539-552), as fp16
//               base-2 exponents relative to a per-row, per-tile maximum
//               (masked -> -inf)
//   kFwdPlainKeepBits
//               kFwdPlain with dropout, + the keep decisions as bits for the
//               softmax column pass (which then need not evaluate Philox)
//
// Design (MI355X-first):
//  * Workgroup = NW wave64s, 32 query rows per wave, BM = 32*NW rows; key
//    tiles of 64.  K and V tiles are staged row-major in LDS (XOR-swizzled
//    16-byte chunks), double-buffered: tile t+1 is fetched with LDS DMA
//    (out-of-range keys read as 0) while tile t is consumed.
//  * Scores are computed transposed, S^T = K Q^T (A = K rows from LDS,
//    B = Q held in VGPRs), so lane l owns query row l%32 and 32 of the 64
//    keys: row max / row sum of the online softmax are in-lane reductions
//    plus one exchange with lane l^32.
//  * O^T += V^T P^T: P^T is already in the B-operand layout in the lane that
//    computed it; V^T comes from the row-major V tile through
//    ds_read_b64_tr_b16.  The per-row rescale is a per-lane scalar.
//  * Lazy rescaling: the running maximum used as exponent offset is only
//    raised when a tile's maximum exceeds it by more than 2^8 in the base-2
//    exponent, so most tiles skip the O/l rescale.  The result is the same
//    softmax (every term is divided by the same l at the end).
//  * Masks are applied only on tiles that cross the causal diagonal or the
//    key-length edge; all other tiles take an unmasked path.
//  * Score writer (kFwdScores, 8 waves, or 4 with 128-row blocks when 256-row
//    blocks would leave CUs idle): the first half of the waves ("loaders")
//    fetch K/V and never store inside the loop, so their wait for the DMA is
//    never a wait for stores; the second half ("storers") issue every global
//    score store.
//    A CU can only drain stores at its share of HBM write bandwidth, and a
//    wave that issues a store into a full queue stalls, so each storer
//    spreads a fixed number of stores per key tile between its MFMAs
//    (the partner's and its own staged tile of the previous key tile during
//    S = K Q^T, zero slots during O += P V) instead of issuing them in
//    bursts.
//    All score stores are non-temporal: the 1 GiB stream then does not evict
//    the K/V tiles the other workgroups of the head still read from L2
//    (measured 355 -> 316 us at B1 H32 S4096 D128).
//    Each workgroup writes the zeros of its *mirror* row block nrb-1-rb, so
//    long-running workgroups carry the zeros of short ones and the write
//    stream stays even over the kernel's life -- unless every workgroup runs
//    at once (p.zero_self), where each writes its own.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

#include <type_traits>

namespace fas {

// Maps a workgroup id to (row block, group), a group being one batch entry's
// `pack` query heads of one KV head.  Workgroups are dealt to the 8 XCDs
// round-robin by id, and each XCD has its own L2, so the mapping keeps a
// group's row blocks on as few XCDs as it can:
//  * ngroups a multiple of 8: each XCD gets a contiguous set of groups;
//  * ngroups 1, 2 or 4 (and nrb a multiple of 8/ngroups): each group gets
//    8/ngroups XCDs, which take its row blocks in turn;
//  * otherwise groups are dealt round-robin.
// Within an XCD, row blocks run in descending length for causal masks.
__device__ __forceinline__ void map_block(int bid, int nrb, int ngroups, bool causal, int& rb,
                                          int& grp) {
  const int x = bid & 7, s = bid >> 3;
  if ((ngroups & 7) == 0) {
    const int per = ngroups >> 3;
    grp = x * per + s % per;
    rb = s / per;
  } else if ((8 % ngroups) == 0 && nrb % (8 / ngroups) == 0) {
    const int k = 8 / ngroups;
    grp = x / k;
    rb = s * k + x % k;
  } else {
    grp = bid % ngroups;
    rb = bid / ngroups;
  }
  if (causal) rb = nrb - 1 - rb;
}

// Byte offset that every buffer access treats as out of range (dropped).
constexpr uint32_t kOffNone = 0x80000000u;

// Score-row addressing for the score writer's stores.  A store instruction
// covers 8 consecutive virtual rows V..V+7 (V a multiple of 8), lane l
// writing row V + l/8.  The score writer packs 1, 2, 4 or 8 heads (shift =
// log2 pack), so the lane's head (l/8) % pack is the same in every such
// group and its position is V/pack + (l/8 >> shift): one per-lane offset
// (lane_off, which also holds the lane's 16-byte chunk) plus a uniform
// (V/pack - pos0) * row_bytes, from a buffer based at position pos0 of the
// group's first head.  Rows past M: with one head they fall outside the
// buffer's extent; with several they would land in the next head's rows,
// so the lane's position (lpos) is checked against a uniform limit.
struct RowGeom {
  int shift = 0, M = 0, pos0 = 0;
  uint32_t row_bytes = 0, head_bytes = 0;
  __device__ __forceinline__ uint32_t lane_off(int lane) const {
    const int lrow = lane >> 3;
    return (uint32_t)(lrow & ((1 << shift) - 1)) * head_bytes + (uint32_t)(lrow >> shift) * row_bytes +
           (uint32_t)(16 * (lane & 7));
  }
  // Uniform part of the offset of the 8-row group starting at virtual row V.
  __device__ __forceinline__ uint32_t group_off(int V) const {
    return (uint32_t)((V >> shift) - pos0) * row_bytes;
  }
};

// Zero writer for the never-computed causal part of two 32-row rectangles of
// a row block: virtual rows [ra, ra + 32) x keys [za, N) and [rb, rb + 32) x
// keys [zb, N) (row numbers absolute, za and zb multiples of 64).  Each
// store covers 8 rows x 64 keys: eight full 128-byte row segments, lane l
// writing row l / 8, 16-byte chunk l % 8.  The writer walks eight runs --
// the 8-row groups of a, then those of b -- each left to right in batches of
// eight 64-key blocks, so the HBM sees long runs along each row: measured on
// the MI355X, writing a 1 GiB score matrix this way runs at 6.2 TB/s
// against 3.9 TB/s when every store moves to other rows.
// Inside the key loop only full batches are written: eight blocks that lie
// wholly below key N.  Store i of a batch takes the lane's row offset as
// voffset (kOffNone for rows past M), the batch's key offset as the
// wave-uniform scalar offset and 128*i as the immediate, so a batch costs
// one vector select and scalar bookkeeping.  The remaining blocks of each
// run (fewer than eight, the last one possibly cut by N) are written by
// tail() after the loop.
template <bool PACK>
struct ZeroRuns {
  int run = 8;          // current run, 0-3 in a, 4-7 in b, 8 = no full batch left
  int nb = 0;           // full batches left in the current run
  uint32_t koff = 0;    // byte offset of the batch's first key
  uint32_t roff = 0;    // uniform offset of the current run's 8-row group
  int lim = 0;          // PACK: positions of the current run's group below M
  int ra = 0, rb = 0, za = 0, zb = 0, ca = 0, cb = 0, N = 0;
  uint32_t lane_off = 0;  // the lane's row in the group and its chunk
  int lpos = 0;           // PACK: the lane's position within the group
  RowGeom geo;

  // 64-key blocks per row of a rectangle starting at key z whose first row
  // lies inside the matrix, and how many full batches they hold.
  __device__ __forceinline__ static int blocks(int N, int z, bool rows_valid) {
    return (rows_valid && N > z) ? (N - z + 63) >> 6 : 0;
  }
  __device__ __forceinline__ static int full_batches(int N, int c) {
    return c > 0 ? (c - ((N & 63) != 0 ? 1 : 0)) >> 3 : 0;
  }
  __device__ __forceinline__ void init(int ra_, int za_, int rb_, int zb_, int N_, int lane,
                                       const RowGeom& g) {
    ra = ra_; rb = rb_; za = za_; zb = zb_; N = N_; geo = g;
    lane_off = g.lane_off(lane);
    lpos = (lane >> 3) >> g.shift;
    ca = blocks(N, za, (ra >> g.shift) < g.M);
    cb = blocks(N, zb, (rb >> g.shift) < g.M);
    start(full_batches(N, ca) > 0 ? 0 : (full_batches(N, cb) > 0 ? 4 : 8));
  }
  __device__ __forceinline__ int run_first(int r) const { return (r < 4 ? ra : rb) + 8 * (r & 3); }
  __device__ __forceinline__ void start(int r) {
    run = r;
    const bool in_a = r < 4;
    nb = r < 8 ? full_batches(N, in_a ? ca : cb) : 0;
    koff = (uint32_t)(in_a ? za : zb) * 2u;
    roff = geo.group_off(run_first(r & 7));
    lim = geo.M - (run_first(r & 7) >> geo.shift);
  }
  __device__ __forceinline__ bool pending() const { return run < 8; }
  // voffset of store 0 of the current batch (kOffNone once no full batch is
  // left, or for a row past M); store i adds 128*i.
  __device__ __forceinline__ uint32_t vbase() const {
    return run < 8 && (!PACK || lpos < lim) ? roff + lane_off : kOffNone;
  }
  __device__ __forceinline__ void advance() {
    koff += 1024u;
    if (--nb == 0 && run < 8)
      start(run == 3 && full_batches(N, cb) == 0 ? 8 : run + 1);
  }
  // Blocks of every run past its full batches, masked at key N.
  template <class Store>
  __device__ __forceinline__ void tail(int lane_key, Store&& store) const {
    for (int r = 0; r < 8; ++r) {
      const bool in_a = r < 4;
      const int c = in_a ? ca : cb, z = in_a ? za : zb;
      const uint32_t ro = geo.group_off(run_first(r));
      const bool row_ok = !PACK || lpos < geo.M - (run_first(r) >> geo.shift);
      for (int kb = 8 * full_batches(N, c); kb < c; ++kb) {
        const int k = z + 64 * kb;
        store(lane_key < N - k && row_ok ? ro + lane_off : kOffNone, (uint32_t)k * 2u);
      }
    }
  }
};

// Scheduling hint for a storer's MFMA phase: alternate M MFMAs and one
// global store, so each store finds room in the CU's store queue and the
// wave never stalls on a burst.
template <int N, int M = 2>
__device__ __forceinline__ void interleave_mfma_stores() {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, M, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);  // VMEM write
  }
}

// Schedule of one S^T = K Q^T tile (2 MFMAs and 2 operand fetches per
// k-step): fetches run PD k-steps ahead of their MFMAs; NST global stores
// of the same region go one per k-step.
template <int KS, int NST>
__device__ __forceinline__ void sched_score_tile() {
  constexpr int PD = KS < 2 ? KS : 2;
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * PD, 0);  // DS read
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
    if (i + PD < KS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    if (i < NST) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);  // VMEM write
  }
  if (NST > KS) __builtin_amdgcn_sched_group_barrier(0x040, NST > KS ? NST - KS : 1, 0);
}

// LDS of the region mode's row-major staging (kFwdRegion only: other
// instances never instantiate these, so their LDS holds none of it).
template <int NW>
__device__ __forceinline__ u32x4* region_stage() {
  __shared__ __attribute__((aligned(16))) u32x4 a[NW * 256];
  return a;
}
template <int BM>
__device__ __forceinline__ int64_t* region_rows() {
  __shared__ int64_t a[BM];
  return a;
}

// PACK: GQA packing (p.pack query heads per workgroup, per-lane heads and
// positions); without it the workgroup's rows are one head's and every
// per-lane head offset folds away at compile time.
// Two waves per SIMD, except for the 4-wave score writer, whose LDS (one
// workgroup per CU) allows one.
// KS2 (unpacked score writer): row blocks of 32 * NW / 2 rows whose key
// range is split between the wave pairs: loader wave i takes the even key
// tiles and storer wave NW/2 + i the odd ones of the same 32 rows, so a step
// stages two key tiles; at the end each storer hands its partial O, offset
// and weight sum to its loader through LDS.  For problems whose 128-row
// blocks all run in one round, where the longest causal row block alone set
// the kernel time:
//  * 4 waves, 64-row blocks: two rounds whose longest-first pairs (rb,
//    15 - rb) all take the same number of steps (one wave per SIMD);
//  * 8 waves, 128-row blocks: one round at two waves per SIMD, half the steps
//    of the 4-wave 128-row writer per row block.  Its K/V stages fill 128 KiB
//    of LDS, so the loaders' score tiles are single-buffered: a second
//    barrier in each step (after the tiles are staged) hands them to the
//    storers, which store both tiles of the step during O += P V.
template <class E, int D, int MODE, int NW, bool DROP, bool PACK, bool KS2 = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 1 : 2, 2)))
void fwd_kernel(const FwdParams p) {
  static_assert(MODE != kFwdScores || NW == 8 || NW == 4, "the score writer uses 4 or 8 waves");
  static_assert(!KS2 || (MODE == kFwdScores && !DROP && !PACK),
                "the key-split writer is the unpacked score writer");
  constexpr int NH = NW / 2;  // score writer: loader waves [0, NH), storer waves [NH, NW)
  const int pack = PACK ? p.pack : 1;
  constexpr int KS = D / 16;               // MFMA k-steps over the head dim
  constexpr int DB = (D + 31) / 32;        // 32-dim blocks of O^T
  constexpr int BM = KS2 ? 32 * NH : 32 * NW;
  constexpr int NTS = KS2 ? 2 : 1;         // key tiles per step (per LDS stage)
  constexpr int BN = 64;
  constexpr int TILE = BN * D;             // elements per K or V tile
  constexpr int BLOCKS = TILE / 512;       // 1 KiB DMA blocks per tile
  constexpr int RPB = 512 / D;             // tile rows per DMA block
  constexpr int CPR = D / 8;               // 16-byte chunks per row
  constexpr bool kSplit = MODE == kFwdScores;
  constexpr int NL = kSplit ? NH : NW;     // waves issuing tile loads
  constexpr int QPW = (BLOCKS + NL - 1) / NL;
  // Score tiles leave through LDS (4 KiB per 32-row wave tile), so that
  // every global store instruction writes 8 full 128-byte row segments:
  // 2 stages x NH loader tiles, then one tile per storer (kMid: one stage of
  // loader tiles, handed over within the step).
  constexpr bool kMid = KS2 && NW == 8;
  constexpr int TSZ = 256;  // 16-byte units per wave tile
  constexpr int SG = kSplit ? (kMid ? 2 : 3) * NH * TSZ : 1;
  constexpr int kLoaderStg = kMid ? 1 : 2;  // stages of loader tiles
  constexpr int kOwnStg = kLoaderStg * NH;  // first storer tile
  // Zero-store slots per key tile and storer (issued during O += P V).
  constexpr int kZero = 8;  // zero stores per key tile: one ZeroRuns batch

  // K/V stages; after the key loop (KS2) the storers' partial O, offsets and
  // weight sums pass through the same LDS, which is sized for the larger.
  union KvLds {
    uint16_t t[2][NTS][2][TILE];
    float merge[KS2 ? NH * (DB * 16 + 2) * 64 : 1];
  };
  __shared__ __attribute__((aligned(16))) KvLds kv_lds;
  auto& kv = kv_lds.t;
  __shared__ __attribute__((aligned(16))) u32x4 stg[SG];
  // Region tiles (kFwdRegion) leave through LDS too: a wave's 32 x 64 fp16
  // tile (4 KiB, 16-byte chunks XOR-swizzled by row) is read back row-major,
  // so each store writes eight whole 128-byte row pieces; rofs holds each
  // virtual row's row index in the region (-1 outside it).
  constexpr bool kRegion = MODE == kFwdRegion;
  u32x4* rstg = nullptr;
  int64_t* rofs = nullptr;
  if constexpr (kRegion) {
    rstg = region_stage<NW>();
    rofs = region_rows<BM>();
  }

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const bool loader = !kSplit || wave < NH;
  // The wave's 32-row slice of the row block, and (KS2) its key-tile parity.
  const int slice = KS2 ? (wave & (NH - 1)) : wave;
  const int kpar = KS2 && !loader ? 1 : 0;
  if (blockIdx.x == 0 && p.zero_words != nullptr)
    for (int i = tid; i < p.n_zero_words; i += NW * 64) p.zero_words[i] = 0u;

  // Split over keys: the plain and row-sum modes may give a row block to
  // nsplit workgroups, each over its own share of the key tiles.
  constexpr bool kCanSplit = MODE == kFwdPlain || MODE == kFwdPlainKeepBits || MODE == kFwdRowSum;
  int rb, grp, split = 0;
  {
    int bid = blockIdx.x;
    if constexpr (kCanSplit) {
      split = bid % p.nsplit;
      bid /= p.nsplit;
    }
    map_block(bid, p.nrb, p.B * p.H / pack, p.causal != 0, rb, grp);
  }
  // The group's heads h0 .. h0 + pack - 1 share KV head hk.  Virtual row
  // v = pos * pack + j is position pos of head h0 + j; a lane owns one
  // virtual row, so its position and head are per-lane values.
  const int gpb = p.H / pack;  // groups per batch entry
  const int b = grp / gpb, h0 = (grp - b * gpb) * pack, hk = h0 / p.G;
  const int row0 = rb * BM;
  const int wrow0 = row0 + 32 * slice;
  const int vrow = wrow0 + c;
  const int qpos = vrow / pack;
  const int qh = h0 + (vrow - qpos * pack);
  const int bh = b * p.H + qh;
  const bool row_ok = qpos < p.M;
  // First and last position of a run of virtual rows [r, r + n).
  auto pos_lo = [&](int r) { return r / pack; };
  auto pos_hi = [&](int r, int n) { return min(p.M - 1, (r + n - 1) / pack); };

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h0 * p.sq1, p.q_bytes);
  const i32x4 wk = make_rsrc_words(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const i32x4 wv = make_rsrc_words(p.v + b * p.sv0 + hk * p.sv1, p.v_bytes);
  const uint32_t kv_base = lds_addr(&kv[0][0][0][0]);
  // Byte offsets of the lane's q and out rows (kOffNone past M: q reads
  // zeros, out stores are dropped).
  const uint32_t qoff = row_ok ? (uint32_t)(((int64_t)(qh - h0) * p.sq1 + (int64_t)qpos * p.sq2) * 2)
                               : kOffNone;
  const uint32_t ooff = row_ok ? (uint32_t)(((int64_t)(qh - h0) * p.so1 + (int64_t)qpos * p.so2) * 2)
                               : kOffNone;

  // Key range of a wave starting at virtual row r: tiles [0, wt(r)) are
  // computed (up to its last position's diagonal), tiles [0, tfull) need no
  // mask.
  auto wtiles_of = [&](int r) {
    if (pos_lo(r) >= p.M) return 0;  // every row of the wave lies past M
    const int whi = p.causal ? min(p.N, max(0, p.causal_off + pos_hi(r, 32) + 1)) : p.N;
    return (whi + BN - 1) / BN;
  };
  const int hi = p.causal ? min(p.N, max(0, p.causal_off + pos_hi(row0, BM) + 1)) : p.N;
  const int ntiles = (hi + BN - 1) / BN;
  // This workgroup's key tiles [t_begin, t_end): all of them, or one split's
  // share (possibly none).
  // Loop steps [t_begin, t_end): one key tile each, or (KS2) two.
  int t_begin = 0, t_end = KS2 ? (ntiles + 1) / 2 : ntiles;
  if constexpr (kCanSplit) {
    if (p.nsplit > 1) {
      t_begin = min(ntiles, split * p.tps);
      t_end = min(ntiles, t_begin + p.tps);
    }
  }
  const int wtiles = wtiles_of(wrow0);
  int tfull = p.N / BN;
  if (p.causal) tfull = min(tfull, max(0, p.causal_off + pos_lo(wrow0) + 1) / BN);

  // Q (B operand of S^T = K Q^T): lane holds Q[qpos][16ks + 8g, +8) of
  // head qh.
  u32x4 qreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qreg[ks] = buf_load16(rq, qoff + (uint32_t)((16 * ks + 8 * g) * 2)) ^ p.qneg;

  // Step t -> LDS stage: its key tiles (t, or KS2: 2t and 2t + 1 in slots
  // 0 and 1); block q of K (and of V) is rows [q*RPB, +RPB); lane l fills
  // physical chunk l % CPR of row q*RPB + l / CPR.
  // The global offset of a lane's 16 bytes, (key * stride + 8 ch) * 2, is a
  // per-lane part (its row within the block and its chunk; the swizzle of
  // row q*RPB + l/CPR repeats with period PQ in q) plus the uniform
  // (tile * BN + q * RPB) * stride * 2, and the LDS destination is the
  // stage base plus a constant.  Each part passes through an opaque copy per
  // step: hoisted out of the loop, the 2*QPW*NTS offsets and destinations
  // per stage were kept in registers the loop lacks (spilled).
  constexpr int PQ = D == 128 ? 4 : (D == 64 ? 2 : 1);
  const uint32_t sk2 = (uint32_t)p.sk2, sv2 = (uint32_t)p.sv2;
  auto issue_tile = [&](int t, int stage) __attribute__((always_inline)) {
    if (!loader) return;
    uint32_t kvb = kv_base;
    asm("" : "+s"(kvb) : "s"(t));
#pragma unroll
    for (int slot = 0; slot < NTS; ++slot) {
      const int tile = NTS * t + slot;
      if (KS2 && tile >= ntiles) break;
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        const int q = wave + i * NL;
        if (BLOCKS % NL == 0 || q < BLOCKS) {
          const int rl = lane / CPR;
          const int ch = (lane % CPR) ^ swz<D>((q % PQ) * RPB + rl);
          uint32_t lk = (uint32_t)(rl * sk2 + ch * 8) * 2u;
          uint32_t lv = (uint32_t)(rl * sv2 + ch * 8) * 2u;
          asm("" : "+v"(lk), "+v"(lv) : "s"(t));
          uint32_t kr = (uint32_t)(tile * BN + q * RPB);
          asm("" : "+s"(kr));
          const uint32_t lb =
              kvb + (uint32_t)(((stage * NTS + slot) * 2 * TILE + q * 512) * 2);
          dma16(wk, lk + kr * sk2 * 2u, __builtin_amdgcn_readfirstlane(lb));
          dma16(wv, lv + kr * sv2 * 2u, __builtin_amdgcn_readfirstlane(lb + TILE * 2));
        }
      }
    }
  };
  // ---- score writer state (kFwdScores) ----
  // Storers exist only for 16-byte aligned score rows; otherwise every wave
  // writes its own scores element-wise.
  const bool vec = MODE == kFwdScores && p.vec_scores != 0;
  const bool storer = vec && !loader;
  const int pwave = wave - NH;  // the loader wave a storer serves
  const int pwtiles = kSplit ? wtiles_of(row0 + 32 * pwave) : 0;
  // Lane (row l/8, chunk l%8) of an 8-row x 128-byte store.
  int lane_key = 8 * (lane & 7);
  __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scores, 0);
  __amdgpu_buffer_rsrc_t rz = rs;
  ZeroRuns<PACK> zr;
  // Score rows (RowGeom): the storer's stores address rows 8i + l/8 of a
  // 32-row wave tile through the lane's fixed offset plus a uniform part.
  const int sshift = PACK ? p.pack_shift : 0;
  RowGeom gs;
  uint32_t lane_off = 0;
  const int lpos = (lane >> 3) >> sshift;
  if constexpr (MODE == kFwdScores) {
    // rs covers the group's heads from the block's first position, rz the
    // same from the mirror block's first position.  The extents pass
    // through readfirstlane: they may be computed on the vector ALU, and a
    // descriptor in VGPRs costs a loop around every store.
    const uint32_t hspan = (uint32_t)((pack - 1) * p.ss1 * 2);
    const int pos0 = min(p.M, pos_lo(row0));
    const int pos1 = min(p.M, pos_lo(row0 + BM - 1) + 1);
    rs = make_rsrc(p.scores + b * p.ss0 + h0 * p.ss1 + (int64_t)pos0 * p.ss2,
                   __builtin_amdgcn_readfirstlane(hspan + (uint32_t)((pos1 - pos0) * p.ss2 * 2)));
    gs = RowGeom{sshift, p.M, pos0, (uint32_t)(p.ss2 * 2), (uint32_t)(p.ss1 * 2)};
    lane_off = gs.lane_off(lane);
    // Zeros of the mirror row block, or of its own when every workgroup
    // runs at once (then the longest row blocks would also carry the largest
    // triangles).
    const int mrow0 = (p.zero_self ? rb : p.nrb - 1 - rb) * BM;
    const int mpos0 = min(p.M, pos_lo(mrow0));
    const int mpos1 = min(p.M, pos_lo(mrow0 + BM - 1) + 1);
    rz = make_rsrc(p.scores + b * p.ss0 + h0 * p.ss1 + (int64_t)mpos0 * p.ss2,
                   __builtin_amdgcn_readfirstlane(hspan + (uint32_t)((mpos1 - mpos0) * p.ss2 * 2)));
    if (storer) {
      RowGeom gz = gs;
      gz.pos0 = mpos0;
      const int wa = wtiles_of(mrow0 + 32 * wave), wb = wtiles_of(mrow0 + 32 * pwave);
      if constexpr (KS2)  // the storer's slice of the mirror block (no second rectangle)
        zr.init(mrow0 + 32 * pwave, wb * BN, 1 << 29, p.N, p.N, lane, gz);
      else
        zr.init(mrow0 + 32 * wave, wa * BN, mrow0 + 32 * pwave, wb * BN, p.N, lane, gz);
    }
  }
  // Staged score tile: row r (32 rows), 16-byte chunk ch (8 per row) at
  // unit r*8 + (ch ^ ((r >> 1) & 7)): conflict-free both for the MFMA-layout
  // writes (16 rows, one chunk) and the row-major reads (2 rows, 8 chunks).
  auto stage_tile = [&](int base, const f32x16 (&sv)[2], bool masked)
                        __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x16& x = sv[j >> 1];
      const int r0 = 8 * (j & 1);
      float v[8];
      if (masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = x[r0 + e] == neg_inf() ? 0.f : x[r0 + e] * p.sm_scale;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = x[r0 + e] * p.sm_scale;
      }
      stg[base + c * 8 + ((2 * j + g) ^ ((c >> 1) & 7))] =
          u32x4{E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]),
                E::pack(v[6], v[7])};
    }
  };
  // Rows 8i + l/8, chunk l%8 of a staged tile, and their global offsets
  // (rows rbase.. of the row block, keys k0..; kOffNone when !valid or past
  // key N - 1).
  auto read_staged = [&](int base, u32x4 (&w)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + (lane >> 3), ch = lane & 7;
      w[i] = stg[base + r * 8 + (ch ^ ((r >> 1) & 7))];
    }
  };
  // Rows 8i + l/8 of the wave tile starting at virtual row T, keys k0..
  auto staged_offsets = [&](int T, int k0, bool valid, uint32_t (&o)[4])
                            __attribute__((always_inline)) {
    const bool ok = valid && k0 + lane_key < p.N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int V = T + 8 * i;
      const bool row_ok = !PACK || lpos < p.M - (V >> sshift);
      o[i] = ok && row_ok ? gs.group_off(V) + (uint32_t)(k0 * 2) + lane_off : kOffNone;
    }
  };
  // One batch of kZero = 8 zero stores.
  auto zero_batch = [&]() __attribute__((always_inline)) {
    const uint32_t vb = zr.vbase();
#pragma unroll
    for (int i = 0; i < kZero; ++i)
      buf_store16_nt(u32x4{0u, 0u, 0u, 0u}, rz, vb + 128u * (uint32_t)i, zr.koff);
    zr.advance();
  };
  // Score tiles of step t of the partner (staged by wave pwave in step t)
  // and of the storer itself (staged in step t, single buffer): key tile t
  // of both, or (KS2, same rows) tiles 2t and 2t + 1.
  auto staged_pair = [&](int t, u32x4 (&w)[8], uint32_t (&o)[8]) __attribute__((always_inline)) {
    u32x4 wp[4], wo[4];
    uint32_t op[4], oo[4];
    const int tp = NTS * t, to = NTS * t + (NTS - 1);
    read_staged(((kMid ? 0 : (t & 1)) * NH + pwave) * TSZ, wp);
    read_staged((kOwnStg + pwave) * TSZ, wo);
    staged_offsets(row0 + 32 * pwave, tp * BN, t >= 0 && tp < pwtiles, op);
    staged_offsets(row0 + 32 * slice, to * BN, t >= 0 && to < wtiles, oo);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = wp[i];
      o[i] = op[i];
      w[4 + i] = wo[i];
      o[4 + i] = oo[i];
    }
  };

  float m_ref = neg_inf(), l_i = 0.f, rsum = 0.f;
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};

  // S^T tile: register r of s[kb] holds key k0 + 32*kb + acc_row(r, g).
  // Every K operand fetch is written before the MFMAs; the caller pins the
  // schedule (sched_score_tile) so each fetch runs PD k-steps ahead of the
  // MFMAs that consume it and no MFMA waits on a fresh LDS read.
  // XA (tile index tw): the fetch addresses are formed in the call as
  // kaddr ^ (ks << 5) from an opaque per-tile copy of the lane's byte offset
  // kaddr of k-step 0 (row perm_row(c), logical chunk g: chunk 2ks + g is
  // physical 2ks ^ (g ^ swz(row)), and row * 2D has no bit below 2D), instead
  // of KS loop-invariant addresses held in registers through the key loop.
  const uint32_t kaddr = (uint32_t)(2 * tile_off<D>(perm_row(c), g));
  auto score_tile = [&](const uint16_t* kt, f32x16 (&s)[2], int tw, auto xa)
                        __attribute__((always_inline)) {
    u32x4 a0[KS], a1[KS];
    if constexpr (decltype(xa)::value) {
      uint32_t ka = kaddr;
      asm("" : "+v"(ka) : "s"(tw));
      const char* kb = reinterpret_cast<const char*>(kt);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint32_t off = ka ^ (uint32_t)(ks << 5);
        a0[ks] = *reinterpret_cast<const u32x4*>(kb + off);
        a1[ks] = *reinterpret_cast<const u32x4*>(kb + off + 64 * D);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        a0[ks] = lds_row_chunk<D>(kt, perm_row(c), ks, g);
        a1[ks] = lds_row_chunk<D>(kt, 32 + perm_row(c), ks, g);
      }
    }
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s[0] = E::mma(a0[ks], qreg[ks], s[0]);
      s[1] = E::mma(a1[ks], qreg[ks], s[1]);
    }
  };
  // P = exp2(s*qk_scale - offset), packed as the B operands of
  // O^T += V^T P^T.  Returns the lane's sum of its 32 weights of the tile.
  // For fp16 the sum is taken from the packed values two at a time (v_dot2
  // against (1, 1)): the same rounded weights the product uses, at half the
  // adds; bf16 weights are too coarse for that and are summed in fp32.
  auto make_p = [&](const f32x16 (&s)[2], u32x4 (&pb)[4]) __attribute__((always_inline)) {
    const float nb = (m_ref == neg_inf() ? 0.f : m_ref) * p.qk_scale;
    float lt = 0.f;
#pragma unroll
    for (int cs = 0; cs < 4; ++cs) {
      const f32x16& sv = s[cs >> 1];
      const int r0 = 8 * (cs & 1);
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = exp2f_fast(fmaf(sv[r0 + e], p.qk_scale, -nb));
      pb[cs] = u32x4{E::pack(pv[0], pv[1]), E::pack(pv[2], pv[3]), E::pack(pv[4], pv[5]),
                     E::pack(pv[6], pv[7])};
      if constexpr (E::kPackedRowSum) {
#pragma unroll
        for (int w = 0; w < 4; ++w) lt = E::sum2(pb[cs][w], lt);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) lt += pv[e];
      }
    }
    return lt;
  };
  // Dropout (DROP instances): zero the packed weights of dropped elements
  // after the row sum has taken them (attention_with_scores.py:169-176).
  // Weight e of pb[cs] is key k0 + 16cs + 8g + e of this lane's row.
  const uint32_t drow = ((uint32_t)bh * (uint32_t)p.M + (uint32_t)qpos) * (uint32_t)p.drop.n;
  // Keep bits for the softmax column pass (kFwdPlainKeepBits): the wave's
  // 32 rows of one key form one word.  A ballot of a keep decision gives
  // two: lanes 0-31 (g = 0) hold rows 0-31 of key k, lanes 32-63 the same
  // rows of key k + 8.  Lane L collects the word of key k0 + L and stores it
  // (keys past N are not stored: a row-word's keys are its pitch).
  constexpr bool kBits = MODE == kFwdPlainKeepBits;
  static_assert(!kBits || DROP, "keep bits exist only with dropout");
  __amdgpu_buffer_rsrc_t rbits = make_rsrc(p.drop_bits, 0), rrows = rbits;
  uint32_t wbase = 0;
  if constexpr (kBits) {
    const int r32 = (p.M + 31) >> 5;
    rbits = make_rsrc(p.drop_bits + (int64_t)(b * p.H + h0) * r32 * p.N,
                      __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)r32 * p.N * 4)));
    wbase = (uint32_t)(wrow0 >> 5) * (uint32_t)p.N;
    if (p.drop_rows != nullptr) {
      const int64_t head = (int64_t)p.rows32 * ((p.N + 31) >> 5) * 32;
      rrows = make_rsrc(p.drop_rows + (int64_t)(b * p.H + h0) * head,
                        __builtin_amdgcn_readfirstlane((uint32_t)(head * 4)));
    }
  }
  auto drop_p = [&](u32x4 (&pb)[4], int k0) __attribute__((always_inline)) {
    // The keep decisions first (32 independent Philox evaluations the
    // compiler interleaves), then the lane writes in a pass of their own:
    // instructions are not moved across inline assembly.
    bool keep[32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int cs = i >> 2, w = i & 3;
      const uint32_t i0 = drow + (uint32_t)(k0 + 16 * cs + 8 * g + 2 * w);
      keep[2 * i] = dropout_keep(p.drop, i0);
      keep[2 * i + 1] = dropout_keep(p.drop, i0 + 1);
      pb[cs][w] &= (keep[2 * i] ? 0xFFFFu : 0u) | (keep[2 * i + 1] ? 0xFFFF0000u : 0u);
    }
    uint32_t word = 0;
    if constexpr (kBits) {
      // Keep pairs i and i + 1 (keys 16 cs + 2 w + {0, 1}, + 8 in the high
      // halves) per group of four ballots.
      static_for<8>([&](auto step) __attribute__((always_inline)) {
        constexpr int i = 2 * decltype(step)::value;
        constexpr int L = 16 * (i >> 2) + 2 * (i & 3);
        const uint64_t bk[4] = {__builtin_amdgcn_ballot_w64(keep[2 * i]),
                                __builtin_amdgcn_ballot_w64(keep[2 * i + 1]),
                                __builtin_amdgcn_ballot_w64(keep[2 * i + 2]),
                                __builtin_amdgcn_ballot_w64(keep[2 * i + 3])};
        write_lanes8<L, L + 8, L + 1, L + 9, L + 2, L + 10, L + 3, L + 11>(word, bk);
      });
    }
    if (kBits && wrow0 < p.M)
      __builtin_amdgcn_raw_buffer_store_b32(
          word, rbits, k0 + lane < p.N ? (wbase + (uint32_t)(k0 + lane)) * 4u : kOffNone, 0, 0);
    if (kBits && p.drop_rows != nullptr) {
      // The backward's row blocks: this row's keys k0 .. k0+31 and
      // k0+32 .. k0+63 as two words.  Keep pair i holds keys
      // 16 (i/4) + 8 g + 2 (i%4) + {0, 1}; each half-wave holds half of
      // every word, the other half comes from lane l ^ 32.
      uint32_t part[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int bit = 16 * ((i >> 2) & 1) + 8 * g + 2 * (i & 3);
        part[i >> 3] |= (keep[2 * i] ? 1u << bit : 0u) | (keep[2 * i + 1] ? 2u << bit : 0u);
      }
      float lo0, hi0, lo1, hi1;
      lane_halves(__builtin_bit_cast(float, part[0]), lo0, hi0);
      lane_halves(__builtin_bit_cast(float, part[1]), lo1, hi1);
      const uint32_t full =
          g == 0 ? __builtin_bit_cast(uint32_t, lo0) | __builtin_bit_cast(uint32_t, hi0)
                 : __builtin_bit_cast(uint32_t, lo1) | __builtin_bit_cast(uint32_t, hi1);
      const int kw = (k0 >> 5) + g, n32 = (p.N + 31) >> 5;
      __builtin_amdgcn_raw_buffer_store_b32(
          full, rrows,
          kw < n32 && wrow0 < p.M ? (uint32_t)((((wrow0 >> 5) * n32 + kw) << 5) + c) * 4u
                                  : kOffNone,
          0, 0);
    }
  };
  // Online softmax, base 2, on raw scores.  Offset update: the tile maximum
  // (combined over the two half-waves of a row) raises a row's offset m_ref
  // when it exceeds it by more than 2^8 in the base-2 exponent, rescaling
  // that row's O and l.
  auto update_offset_of = [&](const f32x16 (&s)[2]) __attribute__((always_inline)) {
    float mx = neg_inf();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = xor32_max(mx);
    const bool grow = mx > m_ref && (m_ref == neg_inf() || (mx - m_ref) * p.qk_scale > 8.f);
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? mx : m_ref;
      const float alpha = m_ref == neg_inf() ? 0.f : exp2f_fast((m_ref - m_new) * p.qk_scale);
      l_i *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
      m_ref = m_new;
    }
  };
  // Causal / key-range mask of a tile starting at key k0: masked -> -inf.
  auto apply_mask = [&](f32x16 (&s)[2], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * kb + acc_row(r, g);
        const bool ok = key < p.N && (!p.causal || p.causal_off + qpos >= key);
        if (!ok) s[kb][r] = neg_inf();
      }
  };
  auto pv_mma = [&](const u32x4 (&pb)[4], const uint16_t* vt) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int cs = 0; cs < 4; ++cs)
        oacc[db] = E::mma(lds_vt_operand<D>(vt, db, cs, lane), pb[cs], oacc[db]);
  };

  if constexpr (kRegion) {
    if (tid < BM) {
      const int v = row0 + tid, pos = v / pack;
      const int head = h0 + (v - pos * pack);
      rofs[tid] = pos >= p.split && pos < p.M
                      ? (int64_t)(b * p.H + head) * (p.M - p.split) + (pos - p.split)
                      : -1;
    }
  }
  if (t_begin < t_end) issue_tile(t_begin, 0);
  if (loader) vm_wait_all();
  lds_barrier();
  // Whether some row of this wave lies in the region (wave-uniform).
  const bool wave_region = kRegion && pos_hi(wrow0, 32) >= p.split && pos_lo(wrow0) < p.M;

  // The key-tile loop, instantiated once per wave role so that neither copy
  // merges with the other inside the loop.
  // NZ (storer copy for a workgroup with no zeros to write, e.g. every
  // non-causal one): the step's score stores go between the O += P V MFMAs,
  // where the zero batches would be, and the S MFMAs run without stores.
  auto main_loop = [&](auto role, auto nz_tag) __attribute__((always_inline)) {
    constexpr bool ST = decltype(role)::value;
    constexpr bool NZ = ST && decltype(nz_tag)::value;

    // One key tile; the LDS stage is a compile-time constant, so the
    // per-lane operand addresses are loop-invariant and the stage offset
    // folds into the LDS instructions' immediate offsets. Only the copy
    // with MK set carries the causal / key-range mask, so tiles below the
    // diagonal run no compare-and-select code at all.
    auto step = [&](int it, auto stage_tag, auto mask_tag) __attribute__((always_inline)) {
      constexpr int stage = decltype(stage_tag)::value;
      constexpr bool MK = decltype(mask_tag)::value;
      // KS2: the storers (the ST copy; KS2 launches always have storers)
      // take the odd tiles.  A compile-time slot keeps the LDS operand
      // addresses of the two roles apart; with the slot a runtime value
      // every address carried it and the storer's loop spilled.
      constexpr int kp = KS2 && ST ? 1 : 0;
      const int tw = NTS * it + kp;  // this wave's key tile
      const bool masked = MK && tw >= tfull;
      if (it + 1 < t_end) issue_tile(it + 1, stage ^ 1);
      const uint16_t* kt = kv[stage][kp][0];
      const uint16_t* vt = kv[stage][kp][1];
      const int k0 = tw * BN;

      if constexpr (kMid) {
        // As below (the storer reads back the tiles of the step before and
        // stores them between its S MFMAs), but a barrier after S lets every
        // storer finish that read-back before any wave stages this step's
        // tile into the single buffer.
        const bool act = tw < wtiles;
        f32x16 s[2];
        u32x4 w[8];
        uint32_t o[8];
        if constexpr (ST) {
          staged_pair(it - 1, w, o);
          if (act) {
            __builtin_amdgcn_sched_barrier(0);
            score_tile(kt, s, tw, std::true_type{});
            if constexpr (!NZ) {
#pragma unroll
              for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
              sched_score_tile<KS, 8>();
            } else {
              sched_score_tile<KS, 0>();
            }
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
          }
        } else if (act) {
          score_tile(kt, s, tw, std::true_type{});
          sched_score_tile<KS, 0>();
        }
        lds_barrier();
        if (act) {
          if (masked) apply_mask(s, k0);
          stage_tile((loader ? wave : kOwnStg + pwave) * TSZ, s, masked);
          update_offset_of(s);
          u32x4 pb[4];
          l_i += make_p(s, pb);
          if constexpr (ST && !NZ) {
            // Keep the stored tiles' registers until the weights are formed.
#pragma unroll
            for (int i = 0; i < 8; ++i) asm volatile("" ::"v"(w[i]));
          }
          pv_mma(pb, vt);
          if constexpr (ST) {
            if constexpr (NZ) {
#pragma unroll
              for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
            } else {
              zero_batch();
            }
            interleave_mfma_stores<kZero>();
          }
        } else if constexpr (ST) {
          zero_batch();
        }
      } else if (tw < wtiles) {
        f32x16 s[2];
        u32x4 w[8];
        uint32_t o[8];
        if constexpr (ST) {
          // S = K Q^T with the partner's and its own tile it-1 stored in between.
          staged_pair(it - 1, w, o);
          __builtin_amdgcn_sched_barrier(0);
          score_tile(kt, s, tw, std::integral_constant<bool, kSplit>{});
          if constexpr (!NZ) {
#pragma unroll
            for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
            sched_score_tile<KS, 8>();
          } else {
            sched_score_tile<KS, 0>();
          }
        } else {
          score_tile(kt, s, tw, std::integral_constant<bool, kSplit>{});
          sched_score_tile<KS, 0>();
        }
        if (masked) apply_mask(s, k0);

        if constexpr (MODE == kFwdScores) {
          if (vec) {
            if (loader) {
              stage_tile((stage * NH + wave) * TSZ, s, masked);
            } else {
              // The storer reads this tile back row-major in the next key
              // tile (staged_pair), from other lanes of the same wave.  A
              // wave's LDS accesses execute in issue order, so only the
              // compiler must keep the order: the wave barrier keeps this
              // iteration's read-back before these writes, and the step's
              // closing lds_barrier (an asm with a memory clobber) keeps the
              // writes before the next iteration's read-back.
              __builtin_amdgcn_wave_barrier();
              stage_tile((NW + pwave) * TSZ, s, masked);
            }
          } else if (row_ok) {
            uint16_t* sr = p.scores + b * p.ss0 + qh * p.ss1 + (int64_t)qpos * p.ss2;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int key = k0 + 32 * kb + acc_row(r, g);
                const float x = s[kb][r];
                if (key < p.N) sr[key] = E::cvt(x == neg_inf() ? 0.f : x * p.sm_scale);
              }
          }
        }
        if constexpr (MODE == kFwdRowSum) {
          // Masked scores (-inf) count as 0; only the masked loop copy can
          // hold any, so the others add the tile straight (a pairwise tree:
          // one add per score instead of compare, select and add).
          float t[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x0 = s[0][r], x1 = s[1][r];
            if (masked) {
              x0 = x0 == neg_inf() ? 0.f : x0;
              x1 = x1 == neg_inf() ? 0.f : x1;
            }
            t[r] = x0 + x1;
          }
#pragma unroll
          for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
            for (int r = 0; r < w; ++r) t[r] += t[r + w];
          rsum += t[0];
        }
        if constexpr (MODE == kFwdRegion) {
          if (wave_region && k0 < p.split) {
            // t: the row's maximum over the tile's region keys (keys past
            // split masked out of it); the region keeps y = (s - t) * qk_scale
            // in fp16 (<= 0, near 0 for the weights that matter) and t *
            // qk_scale per row and tile (0 when every region key is masked,
            // whose y are then -inf).
            float mx = neg_inf();
            if (k0 + BN <= p.split) {
#pragma unroll
              for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
            } else {
#pragma unroll
              for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                  if (k0 + 32 * kb + acc_row(r, g) < p.split) mx = fmaxf(mx, s[kb][r]);
            }
            mx = xor32_max(mx);
            const float mt = mx == neg_inf() ? 0.f : mx * p.qk_scale;
            const int tile = k0 / BN;
            if (g == 0) {
              const int64_t r = rofs[32 * wave + c];
              if (r >= 0) p.region_m[tile * p.region_rows + r] = mt;
            }
            if (p.vec_region) {
              // Staged like a score tile (row c, 16-byte chunk 4 kb + 2 hf + g
              // at unit c * 8 + (chunk ^ ((c >> 1) & 7))) and read back
              // row-major: each store writes eight whole 128-byte row pieces.
              u32x4* tile_u = &rstg[wave * 256];
              __builtin_amdgcn_wave_barrier();
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const f32x16& x = s[j >> 1];
                const int r0 = 8 * (j & 1);
                float y[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = fmaf(x[r0 + e], p.qk_scale, -mt);
                tile_u[c * 8 + ((2 * j + g) ^ ((c >> 1) & 7))] =
                    u32x4{F16::pack(y[0], y[1]), F16::pack(y[2], y[3]), F16::pack(y[4], y[5]),
                          F16::pack(y[6], y[7])};
              }
              __builtin_amdgcn_wave_barrier();
              // Lane l takes chunk l % 8 (keys k0 + 8 (l % 8) .. + 7) of rows
              // 8 i + l / 8; chunks past split are not stored (split % 8 == 0).
              const int ch = lane & 7, key = k0 + 8 * ch;
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int R = 8 * i + (lane >> 3);
                const u32x4 val = tile_u[R * 8 + (ch ^ ((R >> 1) & 7))];
                const int64_t r = rofs[32 * wave + R];
                if (r >= 0 && key < p.split)
                  __builtin_nontemporal_store(
                      val, reinterpret_cast<u32x4*>(p.region + r * p.split + key));
              }
            } else if (qpos >= p.split && row_ok) {
              uint16_t* brow =
                  p.region + ((int64_t)bh * (p.M - p.split) + (qpos - p.split)) * p.split;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const f32x16& sv = s[j >> 1];
                const int r0 = 8 * (j & 1);
                const int key0 = k0 + 16 * j + 8 * g;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  if (key0 + e < p.split) brow[key0 + e] = F16::cvt(fmaf(sv[r0 + e], p.qk_scale, -mt));
              }
            }
          }
        }

        auto update_offset = [&]() __attribute__((always_inline)) { update_offset_of(s); };
        u32x4 pb[4];
        float lt;
        if constexpr (MODE == kFwdScores) {
          // The score writer updates the offset first: its weights and
          // O += P V then share one block and overlap, which measured
          // faster there (229.7 vs 236.9 us at the metric shape).
          update_offset();
          lt = make_p(s, pb);
        } else {
          // Elsewhere the weights are formed with the current offset first.
          // Only if some lane's tile weights sum past 2^14 (so a weight
          // exceeds 2^9: its row maximum rose by more than the 2^8 the
          // offset may lag) or a row has no offset yet does the wave update
          // the offset and form the weights again; every weight stays below
          // 2^14, inside the fp16 range of the product.  This skips the
          // maximum on nearly every tile (plain forward 144.9 -> 140.3 us).
          lt = make_p(s, pb);
          const bool redo = !(lt <= 16384.f) || m_ref == neg_inf();
          if (__builtin_amdgcn_ballot_w64(redo) != 0) {
            update_offset();
            lt = make_p(s, pb);
          }
        }
        l_i += lt;
        if constexpr (ST) {
          // Keep the stored tiles' registers until the weights are formed.
#pragma unroll
          for (int i = 0; i < 8; ++i) asm volatile("" ::"v"(w[i]));
        }
        if constexpr (DROP) drop_p(pb, k0);
        if constexpr (ST) {
          // O += P V with zero slots (NZ: the score stores) in between.
          pv_mma(pb, vt);
          if constexpr (NZ) {
#pragma unroll
            for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
          } else {
            zero_batch();
          }
          interleave_mfma_stores<kZero>();
        } else {
          pv_mma(pb, vt);
        }
      } else if constexpr (ST) {
        u32x4 w[8];
        uint32_t o[8];
        staged_pair(it - 1, w, o);
#pragma unroll
        for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
        zero_batch();
      }
      if (loader) vm_wait_all();
      lds_barrier();
    };
    // Tile it uses LDS stage (it - t_begin) & 1. Pairs of full tiles first,
    // then the rest (diagonal and key-edge tiles, and an odd full tile)
    // masked; every wave runs t_end - t_begin steps in all, one workgroup
    // barrier each.
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // (KS2: step it is full for this wave if its tile 2 it + kpar is.)
    const int full_steps = KS2 ? max(0, tfull - kpar + 1) / 2 : tfull;
    const int full_end = max(t_begin, min(full_steps, t_end));
    int it = t_begin;
    for (; it + 1 < full_end; it += 2) {
      step(it, S0{}, std::false_type{});
      step(it + 1, S1{}, std::false_type{});
    }
    for (; it < t_end; it += 2) {
      step(it, S0{}, std::true_type{});
      if (it + 1 < t_end) step(it + 1, S1{}, std::true_type{});
    }
  };
  if constexpr (kSplit) {
    if (storer) {
      // (Packed GQA writers keep one storer copy: their registers have no
      // room for a second.)
      if constexpr (PACK) {
        main_loop(std::true_type{}, std::false_type{});
      } else {
        if (zr.pending())
          main_loop(std::true_type{}, std::false_type{});
        else
          main_loop(std::true_type{}, std::true_type{});
      }
    } else {
      main_loop(std::false_type{}, std::false_type{});
    }
  } else {
    main_loop(std::false_type{}, std::false_type{});
  }
  // Lane-derived values used after the key loop are formed again from an
  // opaque copy of the lane id instead of being carried through the loop
  // (where the score writer has no register left for them).
  int lane_e = lane;
  asm volatile("" : "+v"(lane_e));
  if constexpr (MODE == kFwdScores) {
    if (storer) {
      lane_key = 8 * (lane_e & 7);
      lane_off = gs.lane_off(lane_e);
      zr.lane_off = lane_off;
      u32x4 w[8];
      uint32_t o[8];
      staged_pair(t_end - 1, w, o);
#pragma unroll
      for (int i = 0; i < 8; ++i) buf_store16_nt(w[i], rs, o[i]);
      while (zr.pending()) zero_batch();
      zr.tail(lane_key, [&](uint32_t vo, uint32_t so) {
        buf_store16_nt(u32x4{0u, 0u, 0u, 0u}, rz, vo, so);
      });
    }
    if (!vec) {  // element-wise zero triangle for unaligned rows
      const int z0 = min(p.N, wtiles * BN);
      for (int rr = 0; rr < 32; ++rr) {
        const int v = wrow0 + rr, pos = v / pack;
        if (pos >= p.M) break;
        uint16_t* sr = p.scores + b * p.ss0 + (h0 + v - pos * pack) * p.ss1 + (int64_t)pos * p.ss2;
        for (int key = z0 + lane; key < p.N; key += 64) sr[key] = 0;
      }
    }
  }

  if constexpr (KS2) {
    // The storer's partial O, offset and weight sum meet its loader's in LDS
    // (the K/V tiles' space, free after the loop); lane l of both holds the
    // same row and head dims.
    float* mb = kv_lds.merge + slice * (DB * 16 + 2) * 64;
    lds_barrier();
    if (!loader) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) mb[(db * 16 + r) * 64 + lane] = oacc[db][r];
      mb[DB * 16 * 64 + lane] = m_ref;
      mb[(DB * 16 + 1) * 64 + lane] = l_i;
    }
    lds_barrier();
    if (!loader) return;
    const float mo = mb[DB * 16 * 64 + lane], lo = mb[(DB * 16 + 1) * 64 + lane];
    const float mn = fmaxf(m_ref, mo);
    const float a0 = m_ref == neg_inf() ? 0.f : exp2f_fast((m_ref - mn) * p.qk_scale);
    const float a1 = mo == neg_inf() ? 0.f : exp2f_fast((mo - mn) * p.qk_scale);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        oacc[db][r] = oacc[db][r] * a0 + mb[(db * 16 + r) * 64 + lane] * a1;
    l_i = l_i * a0 + lo * a1;
    m_ref = mn;
  }
  // Epilogue: O = acc / l, base-2 LSE, row sums.
  const float l_tot = xor32_add(l_i);
  if constexpr (kCanSplit) {
    if (p.nsplit > 1) {
      // One split's share: unnormalised O, offset and weight sum (and the
      // raw row sum) in fp32 for fwd_combine_kernel.
      const float r_tot = MODE == kFwdRowSum ? xor32_add(rsum) : 0.f;
      if (row_ok) {
        const int64_t prow = ((int64_t)bh * p.nsplit + split) * p.Mpad + qpos;
        float* po = p.part_o + prow * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int d0 = 32 * db + 16 * hf + 8 * g;
            if (d0 < D) {
              const f32x16& o = oacc[db];
              const int r0 = 8 * hf;
              *reinterpret_cast<f32x4*>(po + d0) = f32x4{o[r0], o[r0 + 1], o[r0 + 2], o[r0 + 3]};
              *reinterpret_cast<f32x4*>(po + d0 + 4) =
                  f32x4{o[r0 + 4], o[r0 + 5], o[r0 + 6], o[r0 + 7]};
            }
          }
        if (g == 0) {
          p.part_m[prow] = m_ref == neg_inf() ? neg_inf() : m_ref * p.qk_scale;
          p.part_l[prow] = l_tot;
          if constexpr (MODE == kFwdRowSum) p.part_r[prow] = r_tot;
        }
      }
      return;
    }
  }
  const int g_e = lane_e >> 5;
  float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if constexpr (DROP) inv *= p.drop.scale;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.o + b * p.so0 + h0 * p.so1, p.o_bytes);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int d0 = 32 * db + 16 * hf + 8 * g_e;
      if (d0 < D) {
        const f32x16& o = oacc[db];
        const int r0 = 8 * hf;
        const u32x4 w = {E::pack(o[r0 + 0] * inv, o[r0 + 1] * inv),
                         E::pack(o[r0 + 2] * inv, o[r0 + 3] * inv),
                         E::pack(o[r0 + 4] * inv, o[r0 + 5] * inv),
                         E::pack(o[r0 + 6] * inv, o[r0 + 7] * inv)};
        buf_store16(w, ro, ooff == kOffNone ? kOffNone : ooff + (uint32_t)(d0 * 2));
      }
    }
  if (g == 0 && row_ok) {
    const float lse2 = m_ref * p.qk_scale + log2f_fast(l_tot);
    if (p.lse2 != nullptr) p.lse2[(int64_t)bh * p.M + qpos] = l_tot > 0.f ? lse2 : pos_inf();
    // attention()'s log normalizer m * sm_scale + ln(l) (flash.py:477-483).
    if constexpr (MODE == kFwdPlain || MODE == kFwdPlainKeepBits)
      if (p.lse_ln != nullptr)
        p.lse_ln[b * p.sl0 + qh * p.sl1 + (int64_t)qpos * p.sl2] =
            l_tot > 0.f ? lse2 * 0.69314718055994531f : neg_inf();
  }
  if constexpr (MODE == kFwdRowSum) {
    const float r = xor32_add(rsum);
    if (g == 0 && row_ok) p.aux[b * p.sa0 + qh * p.sa1 + (int64_t)qpos * p.sa2] = r * p.sm_scale;
  }
}

// Merges the key splits of fwd_kernel: per row, offset M = max over splits,
// weights 2^(m_s - M), l = sum w_s l_s, O = sum w_s O_s / l, base-2 LSE
// M + log2 l (+inf for rows that saw no key), and the summed row sums.
// D/8 threads per row, 8 head dims each.
template <class E, int D, int MODE>
__global__ __launch_bounds__(256) void fwd_combine_kernel(const FwdParams p) {
  constexpr int CPR = D / 8;
  constexpr int RPB = 256 / CPR;
  const int nblk = (p.M + RPB - 1) / RPB;
  const int bh = blockIdx.x / nblk;
  const int row = (blockIdx.x % nblk) * RPB + (int)threadIdx.x / CPR;
  const int ch = (int)threadIdx.x % CPR;
  if (row >= p.M) return;
  const int b = bh / p.H, h = bh % p.H;
  const int64_t base = (int64_t)bh * p.nsplit * p.Mpad + row;
  float mx = neg_inf();
  // Unrolled so the independent loads of several splits are in flight at once.
#pragma unroll 8
  for (int sp = 0; sp < p.nsplit; ++sp) mx = fmaxf(mx, p.part_m[base + (int64_t)sp * p.Mpad]);
  float l = 0.f, r = 0.f, acc[8] = {};
  // Every split wrote its partials (an empty one: O 0, l 0, offset -inf), so
  // each split's loads are unconditional and eight splits' are in flight at
  // once; a split with offset -inf gets weight 0 by a select (a branch on
  // the loaded offset held each split's O loads back: 14.7 us for 33.5 MB of
  // partials at B1 H32 M256 N16384).
#pragma unroll 8
  for (int sp = 0; sp < p.nsplit; ++sp) {
    const int64_t pr = base + (int64_t)sp * p.Mpad;
    if constexpr (MODE == kFwdRowSum) r += p.part_r[pr];
    const float ms = p.part_m[pr];
    const float w = ms == neg_inf() ? 0.f : exp2f_fast(ms - mx);
    l = fmaf(w, p.part_l[pr], l);
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(p.part_o + pr * D + 8 * ch);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(p.part_o + pr * D + 8 * ch + 4);
    acc[0] = fmaf(w, x0.x, acc[0]); acc[1] = fmaf(w, x0.y, acc[1]);
    acc[2] = fmaf(w, x0.z, acc[2]); acc[3] = fmaf(w, x0.w, acc[3]);
    acc[4] = fmaf(w, x1.x, acc[4]); acc[5] = fmaf(w, x1.y, acc[5]);
    acc[6] = fmaf(w, x1.z, acc[6]); acc[7] = fmaf(w, x1.w, acc[7]);
  }
  const float inv = l > 0.f ? p.drop.scale / l : 0.f;
  *reinterpret_cast<u32x4*>(p.o + b * p.so0 + h * p.so1 + (int64_t)row * p.so2 + 8 * ch) =
      u32x4{E::pack(acc[0] * inv, acc[1] * inv), E::pack(acc[2] * inv, acc[3] * inv),
            E::pack(acc[4] * inv, acc[5] * inv), E::pack(acc[6] * inv, acc[7] * inv)};
  if (ch == 0) {
    const float lse2 = mx + log2f_fast(l);
    if (p.lse2 != nullptr) p.lse2[(int64_t)bh * p.M + row] = l > 0.f ? lse2 : pos_inf();
    if constexpr (MODE == kFwdPlain || MODE == kFwdPlainKeepBits)
      if (p.lse_ln != nullptr)
        p.lse_ln[b * p.sl0 + h * p.sl1 + (int64_t)row * p.sl2] =
            l > 0.f ? lse2 * 0.69314718055994531f : neg_inf();
    if constexpr (MODE == kFwdRowSum)
      p.aux[b * p.sa0 + h * p.sa1 + (int64_t)row * p.sa2] = r * p.sm_scale;
  }
}

template <class E, int D, int MODE, int NW, bool DROP, bool PACK, bool KS2 = false>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  constexpr bool kCanSplit = MODE == kFwdPlain || MODE == kFwdPlainKeepBits || MODE == kFwdRowSum;
  const int64_t nsplit = kCanSplit ? p.nsplit : 1;
  const dim3 grid((unsigned)((int64_t)p.nrb * (p.B * p.H / p.pack) * nsplit)), block(NW * 64);
  hipLaunchKernelGGL((fwd_kernel<E, D, MODE, NW, DROP, PACK, KS2>), grid, block, 0, stream, p);
  if constexpr (kCanSplit) {
    if (p.nsplit > 1 && p.M > 0) {
      const int64_t nblk = (p.M + 2048 / D - 1) / (2048 / D);
      constexpr int CM = MODE == kFwdPlainKeepBits ? kFwdPlain : MODE;
      hipLaunchKernelGGL((fwd_combine_kernel<E, D, CM>),
                         dim3((unsigned)(nblk * p.B * p.H)), dim3(256), 0, stream, p);
    }
  }
  return hipGetLastError();
}

template <int MODE, int NW, bool DROP = false, bool PACK = false, bool KS2 = false>
hipError_t launch_fwd_mode(const FwdParams& p, int dtype, int d, hipStream_t s) {
  if (dtype == 0) {
    switch (d) {
      case 16: return launch_fwd_t<F16, 16, MODE, NW, DROP, PACK, KS2>(p, s);
      case 32: return launch_fwd_t<F16, 32, MODE, NW, DROP, PACK, KS2>(p, s);
      case 64: return launch_fwd_t<F16, 64, MODE, NW, DROP, PACK, KS2>(p, s);
      case 128: return launch_fwd_t<F16, 128, MODE, NW, DROP, PACK, KS2>(p, s);
    }
  } else {
    switch (d) {
      case 16: return launch_fwd_t<BF16, 16, MODE, NW, DROP, PACK, KS2>(p, s);
      case 32: return launch_fwd_t<BF16, 32, MODE, NW, DROP, PACK, KS2>(p, s);
      case 64: return launch_fwd_t<BF16, 64, MODE, NW, DROP, PACK, KS2>(p, s);
      case 128: return launch_fwd_t<BF16, 128, MODE, NW, DROP, PACK, KS2>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
