// gfx950 kernel for the attention scores alone: scores[b, h, i, j] =
// (q_i . k_j) * sm_scale in the input dtype.
//
// Serves compute_attention_scores (attention_scores.py:154-223, no mask) and
// the score output of attention_with_scores for short query ranges, where
// the fused score writer would run one workgroup per head (masked entries
// written as 0, attention_with_scores.py:141-148).  The work is a write
// stream, so the stores are shaped for HBM: every score leaves in a whole
// 128-byte run of one row.
//
// A workgroup of four waves takes 256 query rows and 128 keys.  The keys' K
// rows are copied once into a swizzled LDS tile.  Each wave holds 64 query
// rows of Q (two 32-row B operands of S^T = K Q^T) and runs over the tile in
// 64-key chunks: two 32-key A operands from LDS, four MFMA blocks.  Lane
// (c, g) then owns rows c and 32 + c and keys 16*hf + 8g + [0, 8) of each
// block; the wave packs its 64 x 64 chunk into a private LDS stage (16-byte
// units XOR-swizzled by row) and reads it back row-major, eight lanes per
// 128-byte row run, for non-temporal 16-byte stores.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

namespace fas {

constexpr int kScoresWaves = 4;
constexpr int kScoresRows = 64 * kScoresWaves;  // query rows per workgroup
constexpr int kScoresKeys = 128;                // keys per workgroup, staged in LDS

template <class E, int D>
__global__ __launch_bounds__(64 * kScoresWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void scores_kernel(const ScoresParams p) {
  constexpr int KS = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t ktile[kScoresKeys * D];
  __shared__ __attribute__((aligned(16))) uint16_t stage_all[kScoresWaves][64 * 64];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int kblk = blockIdx.x % p.nkb;
  const int rest = blockIdx.x / p.nkb;
  const int rb = rest % p.nrb, bh = rest / p.nrb;
  const int b = bh / p.H, h = bh % p.H, hk = h / p.G;
  const int key_base = kScoresKeys * kblk;
  const int row0 = kScoresRows * rb + 64 * wave;  // the wave's first row
  uint16_t* stage = stage_all[wave];
  // Key j is kept for row i iff j <= causal_off + i.  A workgroup whose keys
  // all lie above its last row's diagonal only writes zeros.
  const bool live = !p.mask || key_base <= p.causal_off + kScoresRows * (rb + 1) - 1;
  if (live)
    dma_tile<D, kScoresKeys, kScoresWaves>(
        make_rsrc_words(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes), p.sk2, key_base,
        lds_addr(ktile), wave, lane);
  u32x4 qreg[2][KS];
  if (row0 < p.M) {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qreg[hh][ks] =
            buf_load16(rq, (uint32_t)(((row0 + 32 * hh + c) * p.sq2 + 16 * ks + 8 * g) * 2));
  }
  if (live) {
    vm_wait_all();
    __builtin_amdgcn_s_barrier();
  }
  if (row0 >= p.M) return;

  uint16_t* sbase = p.scores + b * p.ss0 + h * p.ss1;
  for (int ch = 0; ch < kScoresKeys / 64; ++ch) {
    const int kc = key_base + 64 * ch;
    if (kc >= p.N) break;
    f32x16 s[2][2];  // [row half][32-key block]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key0 = kc + 32 * kb;
      s[0][kb] = f32x16{};
      s[1][kb] = f32x16{};
      // Blocks above the wave's diagonal skip the MFMAs (all entries masked).
      if (live && key0 < p.N && (!p.mask || key0 <= p.causal_off + row0 + 63)) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const u32x4 a = lds_row_chunk<D>(ktile, 64 * ch + 32 * kb + perm_row(c), ks, g);
          s[0][kb] = E::mma(a, qreg[0][ks], s[0][kb]);
          s[1][kb] = E::mma(a, qreg[1][ks], s[1][kb]);
        }
      }
    }
    // Register r of block kb holds key kc + 32kb + 16*(r/8) + 8g + r%8.
    if (p.vec) {
      // The wave's private stage is written in the MFMA layout and read back
      // row-major by other lanes of the same wave.  A wave's LDS accesses
      // execute in issue order, so a wave barrier (no instruction, an
      // ordering point for the compiler) on each side of the hand-over is
      // all the synchronisation this needs: before the read-back, and before
      // the next chunk overwrites the stage.
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int r = 32 * hh + c, row = row0 + r;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int u = 4 * kb + 2 * hf + g;  // 16-byte unit of the 64-key row run
            const int k8 = kc + 8 * u;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              v[e] = s[hh][kb][8 * hf + e] * p.sm_scale;
              if (p.mask && p.causal_off + row < k8 + e) v[e] = 0.f;
            }
            *reinterpret_cast<u32x4*>(stage + r * 64 + ((u ^ (r & 7)) << 3)) =
                u32x4{E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]),
                      E::pack(v[6], v[7])};
          }
      }
      __builtin_amdgcn_wave_barrier();
      // Row-major read-back: lane l takes unit l % 8 of rows l / 8 + 8i.
      const int u = lane & 7;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = (lane >> 3) + 8 * i, row = row0 + r;
        const u32x4 val = *reinterpret_cast<const u32x4*>(stage + r * 64 + ((u ^ (r & 7)) << 3));
        if (row < p.M && kc + 8 * u < p.N)
          __builtin_nontemporal_store(
              val, reinterpret_cast<u32x4*>(sbase + (int64_t)row * p.ss2 + kc + 8 * u));
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = row0 + 32 * hh + c;
        if (row >= p.M) continue;
        uint16_t* srow = sbase + (int64_t)row * p.ss2;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int k8 = kc + 32 * kb + 16 * hf + 8 * g;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              float v = s[hh][kb][8 * hf + e] * p.sm_scale;
              if (p.mask && p.causal_off + row < k8 + e) v = 0.f;
              if (k8 + e < p.N) srow[k8 + e] = E::cvt(v);
            }
          }
      }
    }
  }
}

}  // namespace fas
