// gfx950 kernel for the attention scores alone: scores[b, h, i, j] =
// (q_i . k_j) * sm_scale in the input dtype.
//
// Serves compute_attention_scores (attention_scores.py:154-223, no mask) and
// the score output of attention_with_scores for short query ranges, where
// the fused score writer would run one workgroup per head (masked entries
// written as 0, attention_with_scores.py:141-148).  The work is a write
// stream, so the kernel is shaped by what the HBM takes best (store-only
// probes on the MI355X, 1 GiB of 8 KiB rows): every store instruction writes
// whole 128-byte row runs (partial rows run at a sixth of the rate), and few
// rows are written at once over the chip, each in long runs (256 rows per
// workgroup advancing 128 bytes at a time: 3.5 TB/s; 32 rows per workgroup
// written by four concurrent streams: 5.9 TB/s).
//
// A workgroup owns 256 keys of one head and walks all query rows in steps
// of 64.  Its 8 waves are 4 key groups (64 keys, held in VGPRs for the
// workgroup's life as the A operands of S^T = K Q^T) x 2 row groups (32 rows
// of the step).  Each step's 64 Q rows pass through LDS (double-buffered,
// loaded through registers, so the compiler's wait counts cover them beside
// the score stores); every wave turns its 32 x 64 score tile into 16-bit
// values in a private LDS stage that it reads back row-major: four
// non-temporal stores of 8 rows x 128 bytes.  The key blocks of a head run
// side by side on one XCD (its L2 holds the head's Q once), advance through
// the rows at the same pace, and so write each score row as several
// concurrent 512-byte runs while only a few thousand rows are open over the
// chip.  Q is read once per key block, K once.
//
// Short query ranges (M <= 512) give such a workgroup only a few steps
// after its K load, so there scores_qres_kernel keeps the head's Q rows
// resident in LDS instead and walks several key blocks of the head, the next
// block's K loaded into a second register set while the current one's steps
// run.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

namespace fas {

// Byte offset past every buffer extent: the store is dropped.
constexpr uint32_t kOffNoneScores = 0x80000000u;
// Extent of a head group's score buffer in the resident-Q kernel: the host
// keeps every valid store offset below it.
constexpr uint32_t kScoresGroupBytes = 0x7ffffff0u;

constexpr int kScoresWaves = 8;
constexpr int kScoresRows = 64;    // query rows per step (2 row groups x 32)
constexpr int kScoresKeys = 256;   // keys per workgroup (4 key groups x 64)
constexpr int kScoresResRows = 512;  // most query rows resident in scores_qres_kernel

// The wave's 64 keys [k0, k0 + 64) as A operands of S^T = K Q^T (keys past
// N read as zeros): a0 holds keys k0 + perm_row(c), a1 those 32 above.
template <int D>
__device__ __forceinline__ void scores_load_keys(u32x4 (&a0)[D / 16], u32x4 (&a1)[D / 16],
                                                 __amdgpu_buffer_rsrc_t rk, int k0, int64_t sk2,
                                                 int c, int g) {
  const uint32_t o0 = (uint32_t)(((k0 + perm_row(c)) * sk2 + 8 * g) * 2);
  const uint32_t o1 = (uint32_t)(((k0 + 32 + perm_row(c)) * sk2 + 8 * g) * 2);
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    a0[ks] = buf_load16(rk, o0 + 32 * ks);
    a1[ks] = buf_load16(rk, o1 + 32 * ks);
  }
}

// One wave's 32 x 64 score tile: query rows wrow0 + c (their Q rows at row
// qrow + c of the LDS tile qt) against keys [k0, k0 + 64) held in a0 / a1,
// scaled by sm_scale, masked, converted and stored through the wave's LDS
// stage st.  VEC_ONLY: the caller runs only with p.vec set (no per-element
// store path).
// GROUP (the resident-Q kernel): rows are the virtual rows of a head group
// (2^p.pshift heads from shead on) and every lane's store carries its own
// validity, past M or N at kOffNoneScores.
template <class E, int D, bool MASK, bool VEC_ONLY = false, bool GROUP = false>
__device__ __forceinline__ void scores_tile(const ScoresParams& p, const uint16_t* qt, int qrow,
                                            const u32x4 (&a0)[D / 16], const u32x4 (&a1)[D / 16],
                                            u32x4* st, uint16_t* shead, int wrow0, int k0,
                                            int lane) {
  constexpr int KS = D / 16;
  const int c = lane & 31, g = lane >> 5;
  // S^T tile: register r of s[j] holds key k0 + 32j + 16(r/8) + 8g + r%8
  // of query row wrow0 + c.  Every tile runs its MFMAs: keys past N hold
  // zero K rows, and masked entries are zeroed below (a branch around the
  // MFMAs would cost 32 register moves per tile to merge the zeros).
  f32x16 s[2];
  {
    u32x4 qb[KS];
    // Rows 64 apart share a swizzle, so steps differ only in qt (an
    // immediate offset) and one lane offset serves every step.
    const uint32_t qoff = row_chunk_offset<D>(qrow + c, g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] = lds_row_chunk(qt, qoff, ks);
    s[0] = E::mma(a0[0], qb[0], f32x16{});
    s[1] = E::mma(a1[0], qb[0], f32x16{});
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) {
      s[0] = E::mma(a0[ks], qb[ks], s[0]);
      s[1] = E::mma(a1[ks], qb[ks], s[1]);
    }
  }
  const bool key_ok = k0 + 8 * (lane & 7) < p.N;  // the lane's store unit lies below N
  // The lane's query row (its position within the head for a group).
  const int row = GROUP ? (wrow0 + c) >> p.pshift : wrow0 + c;
  if (VEC_ONLY || p.vec) {
    // Stage row c, 16-byte unit u = 4j + 2hf + g at c*8 + (u ^ ((c/2) & 7)):
    // conflict-free for these writes (one unit of 32 rows) and for the
    // row-major reads below (8 units of 8 rows).  The stage is private to
    // the wave and LDS accesses of a wave execute in order, so wave
    // barriers (compiler ordering points) suffice around the hand-over.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int u = 4 * j + 2 * hf + g;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] = s[j][8 * hf + e] * p.sm_scale;
          if (MASK && p.causal_off + row < k0 + 8 * u + e) v[e] = 0.f;
        }
        st[c * 8 + (u ^ ((c >> 1) & 7))] =
            u32x4{E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]),
                  E::pack(v[6], v[7])};
      }
    __builtin_amdgcn_wave_barrier();
    // Lane l stores unit l % 8 of rows l / 8 + 8i: whole 128-byte runs.
    const int u = lane & 7;
    if constexpr (GROUP) {
      // Row v = wrow0 + r is position (wrow0 >> pshift) + (r >> pshift) of
      // head h0 + (r & (2^pshift - 1)) (wrow0 is a multiple of 32), so the
      // lane offsets from the step's first position are the same in every
      // step; the host bounds every valid offset below kScoresGroupBytes.
      const int m0 = wrow0 >> p.pshift;
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(shead + (int64_t)m0 * p.ss2 + k0, kScoresGroupBytes);
      const int jm = (1 << p.pshift) - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (lane >> 3) + 8 * i, mr = r >> p.pshift;
        const u32x4 val = st[r * 8 + (u ^ ((r >> 1) & 7))];
        buf_store16_nt(val, rs,
                       key_ok && m0 + mr < p.M
                           ? (uint32_t)(((r & jm) * p.ss1 + mr * p.ss2 + 8 * u) * 2)
                           : kOffNoneScores);
      }
    } else {
      // The buffer ends at the wave's last key below N in its last row below
      // M (row stride >= N), so stores to rows past M drop out.
      const int nrows = min(32, p.M - wrow0), nkeys = min(64, p.N - k0);
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(shead + (int64_t)wrow0 * p.ss2 + k0,
                    __builtin_amdgcn_readfirstlane(
                        nrows > 0 && nkeys > 0
                            ? (uint32_t)(((int64_t)(nrows - 1) * p.ss2 + nkeys) * 2)
                            : 0u));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (lane >> 3) + 8 * i;
        const u32x4 val = st[r * 8 + (u ^ ((r >> 1) & 7))];
        buf_store16_nt(val, rs, key_ok ? (uint32_t)((r * p.ss2 + 8 * u) * 2) : kOffNoneScores);
      }
    }
  } else if (!VEC_ONLY && row < p.M) {
    uint16_t* sr = shead + (int64_t)row * p.ss2;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = k0 + 32 * j + 16 * hf + 8 * g + e;
          float v = s[j][8 * hf + e] * p.sm_scale;
          if (MASK && p.causal_off + row < key) v = 0.f;
          if (key < p.N) sr[key] = E::cvt(v);
        }
  }
}

// MASK: the causal / key-range mask of attention_with_scores (entries with
// key > causal_off + row written as 0); a template flag, so the unmasked
// instance (compute_attention_scores) carries no per-score compare.  VEC:
// p.vec is set (every step issues the same four stores per lane, so the
// wait for the next step's Q leaves the step's stores in flight).
template <class E, int D, bool MASK, bool VEC>
__global__ __launch_bounds__(64 * kScoresWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void scores_kernel(const ScoresParams p) {
  constexpr int KS = D / 16;
  constexpr int CPR = D / 8;                                   // 16-byte chunks per row
  constexpr int QCH = kScoresRows * CPR;                       // chunks of a step's Q rows
  constexpr int CPT = (QCH + 64 * kScoresWaves - 1) / (64 * kScoresWaves);
  __shared__ __attribute__((aligned(16))) uint16_t qtile[2][kScoresRows * D];
  __shared__ __attribute__((aligned(16))) u32x4 stg[kScoresWaves][256];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int kg = wave & 3, rg = wave >> 2;
  // A head has nkb key blocks x nrs row ranges (row ranges only when the key
  // blocks alone leave the chip short of workgroups).  Workgroups go to the
  // 8 XCDs round-robin by id.  With B*H a multiple of 8 each XCD takes a
  // contiguous set of heads, so a head's workgroups run together on one XCD.
  int kb, rs, bh;
  {
    const int bid = blockIdx.x, heads = p.B * p.H, per_head = p.nkb * p.nrs;
    int w;
    if ((heads & 7) == 0) {
      const int per = heads >> 3, x = bid & 7, sidx = bid >> 3;
      bh = x * per + sidx / per_head;
      w = sidx % per_head;
    } else {
      bh = bid / per_head;
      w = bid % per_head;
    }
    rs = w / p.nkb;
    kb = w % p.nkb;
  }
  const int b = bh / p.H, h = bh % p.H, hk = h / p.G;
  const int k0 = kScoresKeys * kb + 64 * kg;  // the wave's first key
  // This workgroup's steps of 64 rows: [t_begin, t_end).
  const int nsteps = (p.M + kScoresRows - 1) / kScoresRows;
  const int t_begin = min(nsteps, rs * p.spr), t_end = min(nsteps, t_begin + p.spr);
  // An empty row range leaves now: on every path into the step loop the
  // wait for the first step's Q then covers the K loads too, and the
  // compiler waits for nothing before a step's MFMAs (a path with K still
  // pending made it wait for every outstanding load and store there).
  if (t_begin >= t_end) return;

  // The wave's 64 keys as A operands.
  u32x4 a0[KS], a1[KS];
  scores_load_keys<D>(a0, a1, make_rsrc(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes), k0, p.sk2, c, g);
  // Q rows of step t: chunk tid + 512 i is (row, 16-byte chunk ch); rows
  // past M read as zeros.
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
  u32x4 qst[CPT];
  auto load_q = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + 64 * kScoresWaves * i;
      if (QCH % (64 * kScoresWaves) == 0 || id < QCH) {
        const int row = t * kScoresRows + id / CPR, ch = id % CPR;
        qst[i] = buf_load16(rq, (uint32_t)((row * p.sq2 + ch * 8) * 2));
      }
    }
  };
  auto write_q = [&](int stage) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + 64 * kScoresWaves * i;
      if (QCH % (64 * kScoresWaves) == 0 || id < QCH)
        *reinterpret_cast<u32x4*>(&qtile[stage][tile_off<D>(id / CPR, id % CPR)]) = qst[i];
    }
  };

  uint16_t* const shead = p.scores + b * p.ss0 + h * p.ss1;
  load_q(t_begin);
  write_q(0);
  lds_barrier();
  u32x4* const st = stg[wave];
  for (int t = t_begin; t < t_end; ++t) {
    const int stage = (t - t_begin) & 1;
    if (t + 1 < t_end) load_q(t + 1);
    const int row0 = t * kScoresRows;      // the step's first row
    const int wrow0 = row0 + 32 * rg;      // the wave's first row
    scores_tile<E, D, MASK, VEC>(p, qtile[stage], 32 * rg, a0, a1, st, shead, wrow0, k0, lane);
    if (t + 1 < t_end) write_q(stage ^ 1);
    lds_barrier();
  }
}


// Short query ranges (M <= kScoresResRows): the head's query rows stay in
// LDS and the workgroup walks key blocks w, w + ngrp, w + 2 ngrp, ... of its
// head.  Each block's K is loaded into the other register set while the
// block before it runs, so the K loads overlap that block's score stores;
// between blocks no Q is loaded and no barrier is taken.  The workgroups of
// a head that run at once write neighbouring key blocks of the same rows.
// Under GQA a workgroup serves 2^pshift query heads of one KV head (their
// rows interleaved, 2^pshift * M <= 512), so their K is loaded once.
// ROWS (32, 64, 128, 256 or 512, the fewest that cover 2^pshift * M) rows
// are resident.
// The 8 waves are 8 key groups of 64 keys (512-key blocks) that run the
// block's rows in steps of 32: every wave loads its keys once, where row
// groups of one key group would each load them (M = 32 with two row groups
// of 256-key blocks: 97 against 52 us at B1 H32 N32768), and each step
// writes 1 KiB runs of 32 rows.  With up to 160 KiB of LDS (D = 128, 512
// rows) and up to 256 VGPRs one workgroup (8 waves, two per SIMD) runs per
// CU.  Whole 16-byte score stores only (p.vec).
template <class E, int D, bool MASK, int ROWS>
__global__ __launch_bounds__(64 * kScoresWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void scores_qres_kernel(const ScoresParams p) {
  static_assert(ROWS == 32 || ROWS == 64 || ROWS == 128 || ROWS == 256 || ROWS == 512,
                "resident rows");
  constexpr int KS = D / 16;
  constexpr int KPB = 64 * kScoresWaves;                // keys per block
  constexpr int NST = ROWS / 32;                        // steps of 32 rows per block
  constexpr int CPR = D / 8;                            // 16-byte chunks per row
  constexpr int QCH = ROWS * CPR;                       // chunks of the resident rows
  constexpr int CPT = (QCH + 64 * kScoresWaves - 1) / (64 * kScoresWaves);  // per thread
  __shared__ __attribute__((aligned(16))) uint16_t qtile[ROWS * D];
  __shared__ __attribute__((aligned(16))) u32x4 stg[kScoresWaves][256];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int kg = wave;  // the wave's key group
  // A head group has ngrp workgroups; XCD assignment as in scores_kernel,
  // over the B * H / 2^pshift groups.
  int w, bg;
  {
    const int bid = blockIdx.x, groups = (p.B * p.H) >> p.pshift;
    if ((groups & 7) == 0) {
      const int per = groups >> 3, x = bid & 7, sidx = bid >> 3;
      bg = x * per + sidx / p.ngrp;
      w = sidx % p.ngrp;
    } else {
      bg = bid / p.ngrp;
      w = bid % p.ngrp;
    }
  }
  const int hg = p.H >> p.pshift;  // groups per batch entry
  const int b = bg / hg, h = (bg % hg) << p.pshift, hk = h / p.G;  // h: the group's first head
  uint16_t* const shead = p.scores + b * p.ss0 + h * p.ss1;
  u32x4* const st = stg[wave];
  const uint16_t* const kbase = p.k + b * p.sk0 + hk * p.sk1;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, p.k_bytes);
  // The same base with no bytes: the loads past the head's last key block
  // still issue but read zeros without a memory access, so every path
  // into a block's MFMAs has the same loads outstanding and the compiler
  // waits only for the block's own K there.
  const __amdgpu_buffer_rsrc_t rk_none = make_rsrc(kbase, 0u);
  u32x4 a0[KS], a1[KS], b0[KS], b1[KS];
  scores_load_keys<D>(a0, a1, rk, KPB * w + 64 * kg, p.sk2, c, g);
  {
    // Virtual rows [0, ROWS): chunk tid + 512 i is (row v, 16-byte chunk
    // ch), v holding position v >> pshift of head h + (v & (2^pshift - 1));
    // positions past M read as zeros.
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
    const int jm = (1 << p.pshift) - 1;
    u32x4 qst[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + 64 * kScoresWaves * i, row = id / CPR, ch = id % CPR;
      const int m = row >> p.pshift;
      if (QCH % (64 * kScoresWaves) == 0 || id < QCH)
        qst[i] = buf_load16(rq, m < p.M ? (uint32_t)(((row & jm) * p.sq1 + m * p.sq2 + ch * 8) * 2)
                                        : kOffNoneScores);
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + 64 * kScoresWaves * i, row = id / CPR, ch = id % CPR;
      if (QCH % (64 * kScoresWaves) == 0 || id < QCH)
        *reinterpret_cast<u32x4*>(&qtile[tile_off<D>(row, ch)]) = qst[i];
    }
  }
  // vmcnt(0): the first block's K has arrived (the compiler may issue its
  // loads after Q's), so no load from before the loop is outstanding when
  // the block loop starts.
  __builtin_amdgcn_s_waitcnt(0x0f70);
  lds_barrier();

  // All NST steps run (rows past M hold zero Q rows and their stores drop
  // out): with a fixed number of stores per block, the compiler's wait for
  // a block's K covers only stores of blocks before the one that loaded it.
  auto block = [&](const u32x4(&x0)[KS], const u32x4(&x1)[KS], int kb)
                   __attribute__((always_inline)) {
    const int k0 = KPB * kb + 64 * kg;  // the wave's first key
    // Up to 8 steps unrolled (512 rows: a loop of two, which keeps the
    // 256-VGPR budget).
#pragma unroll 8
    for (int t = 0; t < NST; ++t)
      scores_tile<E, D, MASK, true, true>(p, qtile + 32 * D * t, 0, x0, x1, st, shead, 32 * t, k0,
                                          lane);
  };
  auto load = [&](u32x4(&x0)[KS], u32x4(&x1)[KS], int kb) __attribute__((always_inline)) {
    scores_load_keys<D>(x0, x1, kb < p.nkb ? rk : rk_none, KPB * kb + 64 * kg, p.sk2, c, g);
  };
  // One block ahead: the next block's K moves into a0/a1 after the steps.
  // (Two blocks ahead in three register sets taking turns needs ~255 VGPRs
  // at D = 128, and the compiler then reuses K registers for Q operands
  // and waits for the newest loads at the top of each block.)
  for (int kb = w; kb < p.nkb; kb += p.ngrp) {
    load(b0, b1, kb + p.ngrp);
    block(a0, a1, kb);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      a0[ks] = b0[ks];
      a1[ks] = b1[ks];
    }
  }
}

}  // namespace fas
