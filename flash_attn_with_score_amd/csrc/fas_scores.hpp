// gfx950 kernel for the attention scores alone: scores[b, h, i, j] =
// (q_i . k_j) * sm_scale in the input dtype.
//
// Serves compute_attention_scores (attention_scores.py:154-223, no mask) and
// the score output of attention_with_scores for short query ranges, where
// the fused score writer would run one workgroup per head (masked entries
// written as 0, attention_with_scores.py:141-148).  The work is a write
// stream: a workgroup of four waves takes 32 query rows and 512 keys, each
// wave 128 keys in four 32-key blocks.  A wave holds its rows' Q as the B
// operand of S^T = K Q^T (K rows are read straight from global memory as A
// operands, the block's 32 x D slice contiguous), so lane (c, g) owns query
// row c and keys 16*hf + 8g + [0, 8) of each block: two 16-byte stores per
// block, 32-byte runs per row that L2 merges into full lines.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

namespace fas {

template <class E, int D>
__global__ __launch_bounds__(256) void scores_kernel(const ScoresParams p) {
  constexpr int KS = D / 16;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int nkb = p.nkb;
  const int kblk = blockIdx.x % nkb;
  const int rest = blockIdx.x / nkb;
  const int rb = rest % p.nrb, bh = rest / p.nrb;
  const int b = bh / p.H, h = bh % p.H, hk = h / p.G;
  const int row = 32 * rb + c;

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  u32x4 qreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qreg[ks] = buf_load16(rq, (uint32_t)((row * p.sq2 + 16 * ks + 8 * g) * 2));

  uint16_t* srow = p.scores + b * p.ss0 + h * p.ss1 + (int64_t)row * p.ss2;
  const bool row_ok = row < p.M;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int key0 = 512 * kblk + 128 * wave + 32 * kb;
    if (key0 >= p.N) break;
    // A operand: K row key0 + perm_row(c), head dims [16ks + 8g, +8).
    u32x4 a[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      a[ks] = buf_load16(rk, (uint32_t)(((key0 + perm_row(c)) * p.sk2 + 16 * ks + 8 * g) * 2));
    f32x16 s = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s = E::mma(a[ks], qreg[ks], s);
    if (!row_ok) continue;
    // Register r holds key key0 + acc_row(r, g) = key0 + 16*(r/8) + 8g + r%8.
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int k8 = key0 + 16 * hf + 8 * g;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = s[8 * hf + e] * p.sm_scale;
        if (p.mask && p.causal_off + row < k8 + e) v[e] = 0.f;
      }
      if (p.vec && k8 + 8 <= p.N) {
        *reinterpret_cast<u32x4*>(srow + k8) =
            u32x4{E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]),
                  E::pack(v[6], v[7])};
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k8 + e < p.N) srow[k8 + e] = E::cvt(v[e]);
      }
    }
  }
}

}  // namespace fas
