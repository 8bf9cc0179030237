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
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

namespace fas {

// Byte offset past every buffer extent: the store is dropped.
constexpr uint32_t kOffNoneScores = 0x80000000u;

constexpr int kScoresWaves = 8;
constexpr int kScoresRows = 64;    // query rows per step (2 row groups x 32)
constexpr int kScoresKeys = 256;   // keys per workgroup (4 key groups x 64)

// MASK: the causal / key-range mask of attention_with_scores (entries with
// key > causal_off + row written as 0); a template flag, so the unmasked
// instance (compute_attention_scores) carries no per-score compare.
template <class E, int D, bool MASK>
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

  // The wave's 64 keys as A operands (keys past N read as zeros).
  u32x4 a0[KS], a1[KS];
  {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      a0[ks] = buf_load16(rk, (uint32_t)(((k0 + perm_row(c)) * p.sk2 + 16 * ks + 8 * g) * 2));
      a1[ks] = buf_load16(rk, (uint32_t)(((k0 + 32 + perm_row(c)) * p.sk2 + 16 * ks + 8 * g) * 2));
    }
  }
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
  const bool key_ok = k0 + 8 * (lane & 7) < p.N;  // the lane's store unit lies below N
  if (t_begin < t_end) {
    load_q(t_begin);
    write_q(0);
  }
  lds_barrier();
  u32x4* const st = stg[wave];
  for (int t = t_begin; t < t_end; ++t) {
    const int stage = (t - t_begin) & 1;
    if (t + 1 < t_end) load_q(t + 1);
    const int row0 = t * kScoresRows;      // the step's first row
    const int wrow0 = row0 + 32 * rg;      // the wave's first row
    // S^T tile: register r of s[j] holds key k0 + 32j + 16(r/8) + 8g + r%8
    // of query row wrow0 + c.  Every tile runs its MFMAs: keys past N hold
    // zero K rows, and masked entries are zeroed below (a branch around the
    // MFMAs would cost 32 register moves per tile to merge the zeros).
    f32x16 s[2];
    {
      const uint16_t* qt = qtile[stage];
      u32x4 qb[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qb[ks] = lds_row_chunk<D>(qt, 32 * rg + c, ks, g);
      s[0] = E::mma(a0[0], qb[0], f32x16{});
      s[1] = E::mma(a1[0], qb[0], f32x16{});
#pragma unroll
      for (int ks = 1; ks < KS; ++ks) {
        s[0] = E::mma(a0[ks], qb[ks], s[0]);
        s[1] = E::mma(a1[ks], qb[ks], s[1]);
      }
    }
    const int row = wrow0 + c;  // the lane's query row
    if (p.vec) {
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
      // The buffer ends at the wave's last key below N in its last row below
      // M (row stride >= N), so stores to rows past M drop out.
      const int nrows = min(32, p.M - wrow0), nkeys = min(64, p.N - k0);
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(shead + (int64_t)wrow0 * p.ss2 + k0,
                    __builtin_amdgcn_readfirstlane(
                        nrows > 0 && nkeys > 0
                            ? (uint32_t)(((int64_t)(nrows - 1) * p.ss2 + nkeys) * 2)
                            : 0u));
      const int u = lane & 7;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (lane >> 3) + 8 * i;
        const u32x4 val = st[r * 8 + (u ^ ((r >> 1) & 7))];
        buf_store16_nt(val, rs, key_ok ? (uint32_t)((r * p.ss2 + 8 * u) * 2) : kOffNoneScores);
      }
    } else if (row < p.M) {
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
    if (t + 1 < t_end) write_q(stage ^ 1);
    lds_barrier();
  }
}

}  // namespace fas
