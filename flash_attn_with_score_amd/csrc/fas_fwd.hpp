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
//   kFwdRegion  + raw fp32 scores of the region rows >= split, keys < split
//               (masked -> -inf), the first pass of the buffered cross-token
//               softmax sum (attention_cross_token_softmax_sum.py:539-552)
//
// Design (MI355X-first):
//  * Workgroup = NW wave64s, 32 query rows per wave, BM = 32*NW rows; key
//    tiles of 64.  K and V tiles are staged row-major in LDS (XOR-swizzled
//    16-byte chunks), double-buffered: tile t+1 is fetched with buffer loads
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
//  * The score-writing variant streams the causal zero triangle out in
//    chunks interleaved with the compute loop, so each wave keeps the
//    write queue busy while its MFMA work runs; each workgroup writes the
//    zeros of its mirror row block, which evens the write stream over time.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

namespace fas {

// Maps a workgroup id to (row block, batch*head).  Workgroups are dealt to
// the 8 XCDs round-robin by id; when B*H is a multiple of 8, each XCD gets a
// contiguous set of heads (one KV group stays in one L2) and, within it,
// row blocks in descending length for causal masks.
__device__ __forceinline__ void map_block(int bid, int nrb, int BH, bool causal, int& rb,
                                          int& bh) {
  if ((BH & 7) == 0) {
    const int x = bid & 7, s = bid >> 3, per = BH >> 3;
    bh = x * per + s % per;
    rb = s / per;
  } else {
    bh = bid % BH;
    rb = bid / BH;
  }
  if (causal) rb = nrb - 1 - rb;
}

// Zero writer for the never-computed causal part of 32 score rows: keys
// [z0, N) of rows [rbase, rbase + 32) of a row block.  Lane l covers chunks
// l, l+64, ... of a row (16 bytes each), so each store instruction writes
// 1 KiB contiguous; the row offset is wave-uniform (SGPR) and the lane's
// column offset loop-invariant, so a store costs no vector arithmetic;
// lanes past the row's last chunk use an offset beyond the buffer (dropped).
// `rows_per_call` rows are written per call.
struct ZeroFill {
  int next = 32, nrows = 0, rows_per_call = 0, nfull = 0, rbase = 0;
  uint32_t vbase = 0, vlast = 0;
  bool has_last = false;

  __device__ __forceinline__ void init(int N, int wtiles, int rbase_, int rows_valid, int lane,
                                       int ntiles) {
    rbase = rbase_;
    const int z0 = wtiles * 64;
    const int cpr = (N - z0) / 8;  // chunks per row (N % 8 == 0 on this path)
    next = 32;
    // Only rows below M are written: the row offset travels in soffset, so
    // the descriptor's range check is not relied on for rows.
    nrows = min(32, rows_valid);
    if (cpr > 0 && rows_valid > 0) {
      next = 0;
      rows_per_call = (32 + max(ntiles, 1) - 1) / max(ntiles, 1);
      nfull = cpr / 64;
      const int rem = cpr % 64;
      has_last = rem != 0;
      vbase = (uint32_t)((z0 + 8 * lane) * 2);
      // Lanes past the row's last chunk aim beyond the buffer: dropped.
      vlast = lane < rem ? vbase + (uint32_t)(nfull * 1024) : 0x80000000u;
    }
  }
  __device__ __forceinline__ void run(int rows, __amdgpu_buffer_rsrc_t rz, int64_t ss2) {
    const int end = min(nrows, next + rows);
    for (int r = next; r < end; ++r) {
      const uint32_t soff = (uint32_t)((rbase + r) * ss2 * 2);
      for (int j = 0; j < nfull; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rz, vbase + 1024u * j, soff,
                                               kAuxNT);
      if (has_last)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rz, vlast, soff, kAuxNT);
    }
    next = max(next, end);
  }
};

template <class E, int D, int MODE, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_kernel(const FwdParams p) {
  constexpr int KS = D / 16;               // MFMA k-steps over the head dim
  constexpr int DB = (D + 31) / 32;        // 32-dim blocks of O^T
  constexpr int BM = 32 * NW;
  constexpr int BN = 64;
  constexpr int TILE = BN * D;             // elements per K or V tile
  constexpr int BLOCKS = TILE / 512;       // 1 KiB DMA blocks per tile
  constexpr int RPB = 512 / D;             // tile rows per DMA block
  constexpr int CPR = D / 8;               // 16-byte chunks per row
  // Score writer with 8 waves: waves 0-3 fetch K/V and stage their score
  // tiles in LDS; waves 4-7 never load inside the loop and issue every
  // global score store (their own and their partner's) plus the zero
  // triangle, so no wave ever waits for a store to finish.
  constexpr bool kSplit = MODE == kFwdScores && NW == 8;
  constexpr int NL = kSplit ? 4 : NW;      // waves issuing tile loads
  constexpr int QPW = (BLOCKS + NL - 1) / NL;
  // Score tiles leave through LDS (4 KiB per 32-row wave tile), so that
  // every global store instruction writes 8 full 128-byte row segments.
  // Split mode: 2 stages x 4 loader tiles, then one tile per storer.
  constexpr int TSZ = 256;  // 16-byte units per wave tile
  constexpr int SG = MODE != kFwdScores ? 1 : (kSplit ? (8 + 4) * TSZ : NW * TSZ);

  __shared__ __attribute__((aligned(16))) uint16_t kv[2][2][TILE];
  __shared__ __attribute__((aligned(16))) u32x4 stg[SG];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const bool loader = !kSplit || wave < 4;

  int rb, bh;
  map_block(blockIdx.x, p.nrb, p.B * p.H, p.causal != 0, rb, bh);
  const int h = bh % p.H, b = bh / p.H, hk = h / p.G;
  const int row0 = rb * BM;
  const int wrow0 = row0 + 32 * wave;
  const int qrow = wrow0 + c;

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
  const i32x4 wk = make_rsrc_words(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const i32x4 wv = make_rsrc_words(p.v + b * p.sv0 + hk * p.sv1, p.v_bytes);
  const uint32_t kv_base = lds_addr(&kv[0][0][0]);

  // Key range of a wave starting at row r: tiles [0, wt(r)) are computed,
  // tiles [0, tf(r)) need no mask.
  auto wtiles_of = [&](int r) {
    const int whi = p.causal ? min(p.N, max(0, p.causal_off + r + 32)) : p.N;
    return (whi + BN - 1) / BN;
  };
  const int hi = p.causal ? min(p.N, max(0, p.causal_off + row0 + BM)) : p.N;
  const int ntiles = (hi + BN - 1) / BN;
  const int wtiles = wtiles_of(wrow0);
  int tfull = p.N / BN;
  if (p.causal) tfull = min(tfull, max(0, p.causal_off + wrow0 + 1) / BN);

  // Q (B operand of S^T = K Q^T): lane holds Q[qrow][16ks + 8g, +8).
  u32x4 qreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qreg[ks] = buf_load16(rq, (uint32_t)((qrow * p.sq2 + 16 * ks + 8 * g) * 2)) ^ p.qneg;

  // Tile t -> LDS stage: block q of K (and of V) is rows [q*RPB, +RPB);
  // lane l fills physical chunk l % CPR of row q*RPB + l / CPR.
  auto issue_tile = [&](int t, int stage) {
    if (!loader) return;
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int q = wave + i * NL;
      if (BLOCKS % NL == 0 || q < BLOCKS) {
        const int row = q * RPB + lane / CPR;
        const int ch = (lane % CPR) ^ swz<D>(row);
        const int key = t * BN + row;
        const uint32_t lb = kv_base + (uint32_t)((stage * 2 * TILE + q * 512) * 2);
        dma16(wk, (uint32_t)((key * p.sk2 + ch * 8) * 2), __builtin_amdgcn_readfirstlane(lb));
        dma16(wv, (uint32_t)((key * p.sv2 + ch * 8) * 2),
              __builtin_amdgcn_readfirstlane(lb + TILE * 2));
      }
    }
  };

  // Score-matrix writer (kFwdScores).  Rows past M fall outside the buffer.
  __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scores, 0);
  // Zero triangle: a workgroup writes the never-computed part of its
  // *mirror* row block nrb-1-rb (same head).  Row blocks with much compute
  // have little zero area and vice versa, so every workgroup streams a
  // similar share of zeros spread over its own iterations, and the HBM write
  // stream stays even instead of arriving with the short blocks at the end.
  __amdgpu_buffer_rsrc_t rz = rs;
  ZeroFill zf_own, zf_partner;
  const int pwave = wave - 4;  // split mode: the loader wave a storer serves
  const int prow0 = row0 + 32 * pwave;
  const int pwtiles = kSplit ? wtiles_of(prow0) : 0;
  if constexpr (MODE == kFwdScores) {
    const int64_t base = b * p.ss0 + h * p.ss1 + (int64_t)row0 * p.ss2;
    const int rows = max(0, min(BM, p.M - row0));
    rs = make_rsrc(p.scores + base, (uint32_t)(rows * p.ss2 * 2));
    const int mrow0 = (p.nrb - 1 - rb) * BM;
    const int mrows = max(0, min(BM, p.M - mrow0));
    rz = make_rsrc(p.scores + b * p.ss0 + h * p.ss1 + (int64_t)mrow0 * p.ss2,
                   (uint32_t)(mrows * p.ss2 * 2));
    if (p.vec_scores && (!kSplit || !loader)) {
      const int r_own = mrow0 + 32 * wave, r_par = mrow0 + 32 * pwave;
      zf_own.init(p.N, wtiles_of(r_own), 32 * wave, p.M - r_own, lane, ntiles);
      if (kSplit) zf_partner.init(p.N, wtiles_of(r_par), 32 * pwave, p.M - r_par, lane, ntiles);
    }
  }
  auto zero_fill = [&]() {
    if constexpr (MODE == kFwdScores) {
      zf_own.run(zf_own.rows_per_call, rz, p.ss2);
      if constexpr (kSplit) zf_partner.run(zf_partner.rows_per_call, rz, p.ss2);
    }
  };
  // Staged score tile: row r (32 rows), 16-byte chunk ch (8 per row) at
  // unit r*8 + (ch ^ ((r >> 1) & 7)): conflict-free both for the MFMA-layout
  // writes (16 rows, one chunk) and the row-major reads (2 rows, 8 chunks).
  auto stage_tile = [&](int base, const f32x16 (&sv)[2], bool masked) {
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
  auto store_tile = [&](int base, int rbase, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + (lane >> 3), ch = lane & 7;
      const u32x4 w = stg[base + r * 8 + (ch ^ ((r >> 1) & 7))];
      const int key0 = k0 + 8 * ch;
      if (key0 < p.N) buf_store16(w, rs, (uint32_t)(((rbase + r) * p.ss2 + key0) * 2));
    }
  };
  // Storer side of split mode: the partner's staged score tile t.
  auto flush_partner = [&](int t) {
    if constexpr (kSplit) {
      if (!loader && p.vec_scores && t >= 0 && t < pwtiles)
        store_tile(((t & 1) * 4 + pwave) * TSZ, 32 * pwave, t * BN);
    }
  };

  float m_ref = neg_inf(), l_i = 0.f, rsum = 0.f;
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};

  if (ntiles > 0) issue_tile(0, 0);
  if (loader) vm_wait_all();
  lds_barrier();

  for (int it = 0; it < ntiles; ++it) {
    const int stage = it & 1;
    if (it + 1 < ntiles) issue_tile(it + 1, stage ^ 1);
    flush_partner(it - 1);
    const uint16_t* kt = kv[stage][0];
    const uint16_t* vt = kv[stage][1];
    const int k0 = it * BN;

    if (it < wtiles) {
      f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 a0 = lds_row_chunk<D>(kt, perm_row(c), ks, g);
        const u32x4 a1 = lds_row_chunk<D>(kt, 32 + perm_row(c), ks, g);
        s[0] = E::mma(a0, qreg[ks], s[0]);
        s[1] = E::mma(a1, qreg[ks], s[1]);
      }
      // Register r of s[kb] holds key k0 + 32*kb + acc_row(r, g).
      if (it >= tfull) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * kb + acc_row(r, g);
            const bool ok = key < p.N && (!p.causal || p.causal_off + qrow >= key);
            if (!ok) s[kb][r] = neg_inf();
          }
      }

      if constexpr (MODE == kFwdScores) {
        if (p.vec_scores) {
          if (kSplit && loader) {
            stage_tile((stage * 4 + wave) * TSZ, s, it >= tfull);
          } else {
            // A wave reads back its own LDS writes in order: no barrier.
            const int base = kSplit ? (8 + pwave) * TSZ : wave * TSZ;
            stage_tile(base, s, it >= tfull);
            store_tile(base, 32 * wave, k0);
          }
        } else if (qrow < p.M) {
          uint16_t* srow = p.scores + b * p.ss0 + h * p.ss1 + (int64_t)qrow * p.ss2;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = k0 + 32 * kb + acc_row(r, g);
              const float x = s[kb][r];
              if (key < p.N) srow[key] = E::cvt(x == neg_inf() ? 0.f : x * p.sm_scale);
            }
        }
      }
      zero_fill();
      if constexpr (MODE == kFwdRowSum) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) rsum += s[kb][r] == neg_inf() ? 0.f : s[kb][r];
      }
      if constexpr (MODE == kFwdRegion) {
        if (qrow >= p.split && qrow < p.M && k0 < p.split) {
          float* brow = p.region + ((int64_t)bh * (p.M - p.split) + (qrow - p.split)) * p.split;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x16& sv = s[j >> 1];
            const int r0 = 8 * (j & 1);
            const int key0 = k0 + 16 * j + 8 * g;
            if (p.vec_region && key0 + 8 <= p.split) {
              *reinterpret_cast<f32x4*>(brow + key0) =
                  f32x4{sv[r0 + 0], sv[r0 + 1], sv[r0 + 2], sv[r0 + 3]};
              *reinterpret_cast<f32x4*>(brow + key0 + 4) =
                  f32x4{sv[r0 + 4], sv[r0 + 5], sv[r0 + 6], sv[r0 + 7]};
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (key0 + e < p.split) brow[key0 + e] = sv[r0 + e];
            }
          }
        }
      }

      // Online softmax, base 2, on raw scores.
      float mx = neg_inf();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const bool grow = mx > m_ref && (m_ref == neg_inf() || (mx - m_ref) * p.qk_scale > 8.f);
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float m_new = grow ? mx : m_ref;
        const float alpha = m_ref == neg_inf() ? 0.f : exp2f_fast((m_ref - m_new) * p.qk_scale);
        l_i *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
        m_ref = m_new;
      }
      const float nb = (m_ref == neg_inf() ? 0.f : m_ref) * p.qk_scale;
      u32x4 pb[4];
#pragma unroll
      for (int cs = 0; cs < 4; ++cs) {
        const f32x16& sv = s[cs >> 1];
        const int r0 = 8 * (cs & 1);
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = exp2f_fast(fmaf(sv[r0 + e], p.qk_scale, -nb));
          l_i += pv[e];
        }
        pb[cs] = u32x4{E::pack(pv[0], pv[1]), E::pack(pv[2], pv[3]), E::pack(pv[4], pv[5]),
                       E::pack(pv[6], pv[7])};
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int cs = 0; cs < 4; ++cs)
          oacc[db] = E::mma(lds_vt_operand<D>(vt, db, cs, lane), pb[cs], oacc[db]);
    } else {
      zero_fill();
    }
    if (loader) vm_wait_all();
    lds_barrier();
  }
  flush_partner(ntiles - 1);
  if constexpr (MODE == kFwdScores) {
    zf_own.run(32, rz, p.ss2);
    if constexpr (kSplit) zf_partner.run(32, rz, p.ss2);
    if (!p.vec_scores) {  // element-wise zero triangle for unaligned rows
      const int z0 = min(p.N, wtiles * BN);
      for (int rr = 0; rr < 32; ++rr) {
        const int row = wrow0 + rr;
        if (row >= p.M) break;
        uint16_t* srow = p.scores + b * p.ss0 + h * p.ss1 + (int64_t)row * p.ss2;
        for (int key = z0 + lane; key < p.N; key += 64) srow[key] = 0;
      }
    }
  }

  // Epilogue: O = acc / l, base-2 LSE, row sums.
  const float l_tot = l_i + __shfl_xor(l_i, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.o + b * p.so0 + h * p.so1, p.o_bytes);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int d0 = 32 * db + 16 * hf + 8 * g;
      if (d0 < D) {
        const f32x16& o = oacc[db];
        const int r0 = 8 * hf;
        const u32x4 w = {E::pack(o[r0 + 0] * inv, o[r0 + 1] * inv),
                         E::pack(o[r0 + 2] * inv, o[r0 + 3] * inv),
                         E::pack(o[r0 + 4] * inv, o[r0 + 5] * inv),
                         E::pack(o[r0 + 6] * inv, o[r0 + 7] * inv)};
        buf_store16(w, ro, (uint32_t)((qrow * p.so2 + d0) * 2));
      }
    }
  if (g == 0 && qrow < p.M) {
    if (p.lse2 != nullptr)
      p.lse2[(int64_t)bh * p.M + qrow] =
          l_tot > 0.f ? m_ref * p.qk_scale + log2f_fast(l_tot) : pos_inf();
  }
  if constexpr (MODE == kFwdRowSum) {
    const float r = rsum + __shfl_xor(rsum, 32);
    if (g == 0 && qrow < p.M) p.aux[b * p.sa0 + h * p.sa1 + (int64_t)qrow * p.sa2] = r * p.sm_scale;
  }
}

template <class E, int D, int MODE, int NW>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)p.nrb * p.B * p.H)), block(NW * 64);
  hipLaunchKernelGGL((fwd_kernel<E, D, MODE, NW>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int MODE, int NW>
hipError_t launch_fwd_mode(const FwdParams& p, int dtype, int d, hipStream_t s) {
  if (dtype == 0) {
    switch (d) {
      case 16: return launch_fwd_t<F16, 16, MODE, NW>(p, s);
      case 32: return launch_fwd_t<F16, 32, MODE, NW>(p, s);
      case 64: return launch_fwd_t<F16, 64, MODE, NW>(p, s);
      case 128: return launch_fwd_t<F16, 128, MODE, NW>(p, s);
    }
  } else {
    switch (d) {
      case 16: return launch_fwd_t<BF16, 16, MODE, NW>(p, s);
      case 32: return launch_fwd_t<BF16, 32, MODE, NW>(p, s);
      case 64: return launch_fwd_t<BF16, 64, MODE, NW>(p, s);
      case 128: return launch_fwd_t<BF16, 128, MODE, NW>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
