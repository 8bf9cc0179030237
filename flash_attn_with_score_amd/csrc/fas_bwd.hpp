// gfx950 backward pass of attention() (flash.py:172-261): dQ, dK and dV from
// dO, the forward output O and its natural-log normalizer L.
//
//   bwd_prep_kernel   per query row: -delta = -sum_d O dO (flash.py:532-578) and
//                     nl = -L log2(e), the base-2 exponent offset of the row's
//                     softmax weights (-inf for rows that see no key and for
//                     the padding rows past M), both into the workspace.
//   bwd_dkdv_kernel   key-block outer (flash.py:581-755).  A wave owns 32 keys
//                     and holds their K and V rows in VGPRs as B operands;
//                     64-row tiles of Q and dO arrive in LDS by DMA.  Per
//                     32-row block:
//                       S = Q K^T,  P = exp2(S qk_scale + nl),
//                       dP - delta = dO V^T (the accumulator starts at -delta),
//                       dS = P (dP - delta),
//                       dV^T += dO^T P,  dK^T += Q^T dS.
//                     Keys sit on lanes, so P and dS leave the accumulator
//                     directly as B operands; dO^T and Q^T are read from the
//                     row-major tiles with the transposing LDS load.  GQA: a
//                     workgroup walks every query head of its KV group, so dK
//                     and dV are summed over the group in fp32 (the reference
//                     sums per-head fp16 results, flash.py:258-259).  When
//                     that leaves too few workgroups for the chip, each
//                     workgroup takes one query head and writes fp32 partials
//                     that bwd_dkdv_reduce_kernel adds in head order.
//   bwd_dq_kernel     query-block outer (flash.py:758-918), the forward pass's
//                     data flow: a wave owns 32 rows, holds their Q and dO as B
//                     operands, and streams 64-key tiles of K and V:
//                       S^T = K Q^T,  P^T,  dP^T - delta = V dO^T,  dS^T,
//                       dQ^T += K^T dS^T.
// Masked pairs (causal, keys >= N) get P = 0 and so dS = 0; the products are
// fp16/bf16 MFMAs with fp32 accumulation, with P and dS rounded to the input
// type before their products as in the reference (flash.py:687, 721, 904).
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

#include <type_traits>

namespace fas {

constexpr float kLog2e = 1.44269504088896341f;
// Byte offset past every buffer extent: the access is dropped (store) or
// reads 0 (load).
constexpr uint32_t kOffNoneBwd = 0x80000000u;

// Packs accumulator registers 8cs..8cs+7 (contraction indices 8g..8g+7 of
// k-step cs) as an MFMA B operand.
template <class E>
__device__ __forceinline__ u32x4 pack_b(const f32x16& x, int cs) {
  const int r = 8 * cs;
  return u32x4{E::pack(x[r + 0], x[r + 1]), E::pack(x[r + 2], x[r + 3]),
               E::pack(x[r + 4], x[r + 5]), E::pack(x[r + 6], x[r + 7])};
}

// Eight consecutive fp32 values of LDS row array a starting at index i0 into
// registers [8hf, 8hf + 8) of x.
__device__ __forceinline__ void load8(f32x16& x, const float* a, int i0, int hf) {
  const f32x4 u = *reinterpret_cast<const f32x4*>(a + i0);
  const f32x4 w = *reinterpret_cast<const f32x4*>(a + i0 + 4);
  x[8 * hf + 0] = u.x; x[8 * hf + 1] = u.y; x[8 * hf + 2] = u.z; x[8 * hf + 3] = u.w;
  x[8 * hf + 4] = w.x; x[8 * hf + 5] = w.y; x[8 * hf + 6] = w.z; x[8 * hf + 7] = w.w;
}

// ---------------------------------------------------------------- prep

template <class E, int D>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const BwdParams p) {
  constexpr int CPR = D / 8;      // lanes per row
  constexpr int RPB = 256 / CPR;  // rows per workgroup
  const int bh = blockIdx.x / p.nprep, b = bh / p.H, h = bh % p.H;
  const int row = (blockIdx.x % p.nprep) * RPB + (int)threadIdx.x / CPR;
  const int ch = (int)threadIdx.x % CPR;
  if (row >= p.Mpad) return;  // whole row groups: the shuffles below stay in range
  float acc = 0.f;
  if (row < p.M) {
    const u32x4 o = *reinterpret_cast<const u32x4*>(p.o + b * p.so0 + h * p.so1 +
                                                    (int64_t)row * p.so2 + 8 * ch);
    const u32x4 d = *reinterpret_cast<const u32x4*>(p.dout + b * p.sg0 + h * p.sg1 +
                                                    (int64_t)row * p.sg2 + 8 * ch);
    float x[8], y[8];
    unpack8<E>(o, x);
    unpack8<E>(d, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(x[e], y[e], acc);
  }
#pragma unroll
  for (int w = 1; w < CPR; w <<= 1) acc += __shfl_xor(acc, w);
  if (ch == 0) {
    float nl = neg_inf();
    if (row < p.M) {
      const float L = p.lse[b * p.sl0 + h * p.sl1 + (int64_t)row * p.sl2];
      if (L != neg_inf()) nl = -L * kLog2e;
    }
    p.nl[(int64_t)bh * p.Mpad + row] = nl;
    p.delta[(int64_t)bh * p.Mpad + row] = -acc;
  }
}

// ---------------------------------------------------------------- dK, dV

// DROP: the forward's dropout mask Z (keep = 1) and r = 1/(1-p) enter as
// dV = r sum_i (Z P)_ij dO_i and dS = P (r Z dP - delta) (flash.py:705-731);
// the dP accumulator then starts at 0 and delta is added afterwards.  DROP 1
// evaluates Z (Philox) and, with drop_bits, stores it for the dQ kernel;
// DROP 2 reads the forward's keep words (keep_keys) and has no Philox code.
template <class E, int D, int DROP>
__global__ __launch_bounds__(256) void bwd_dkdv_kernel(const BwdParams p) {
  constexpr int KS = D / 16;               // k-steps over the head dim
  constexpr int DB = D >= 32 ? D / 32 : 1;  // 32-dim blocks of dK^T / dV^T
  constexpr int NW = 4;
  constexpr int BK = 32 * NW;              // keys per workgroup
  constexpr int TQ = 64;                   // query rows per tile
  constexpr int TILE = TQ * D;

  __shared__ __attribute__((aligned(16))) uint16_t qlds[2][TILE];
  __shared__ __attribute__((aligned(16))) uint16_t glds[2][TILE];  // dO
  __shared__ __attribute__((aligned(16))) float nlds[2][TQ];
  __shared__ __attribute__((aligned(16))) float xlds[2][TQ];       // -delta

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  // Key blocks ascending (for causal masks, the longest first).
  const int nrest = p.partial ? p.B * p.H : p.B * p.Hk;
  const int kb = blockIdx.x / nrest, rest = blockIdx.x % nrest;
  int b, hk, h0, nheads;
  if (p.partial) {
    b = rest / p.H;
    h0 = rest % p.H;
    hk = h0 / p.G;
    nheads = 1;
  } else {
    b = rest / p.Hk;
    hk = rest % p.Hk;
    h0 = hk * p.G;
    nheads = p.G;
  }
  const int key0 = kb * BK + 32 * wave;  // this wave's keys [key0, key0 + 32)

  // K and V (B operands of S = Q K^T and dP = dO V^T): lane holds row key0 + c,
  // head dims [16ks + 8g, +8).  Q arrives unchanged by DMA, so K carries the
  // sign of a negative sm_scale.
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + b * p.sv0 + hk * p.sv1, p.v_bytes);
  u32x4 kreg[KS], vreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kreg[ks] = buf_load16(rk, (uint32_t)(((key0 + c) * p.sk2 + 16 * ks + 8 * g) * 2)) ^ p.qneg;
    vreg[ks] = buf_load16(rv, (uint32_t)(((key0 + c) * p.sv2 + 16 * ks + 8 * g) * 2));
  }
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kreg[ks]), "+v"(vreg[ks]));

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  // Query rows that can see a key of the block.
  const int rstart = p.causal ? max(0, kb * BK - p.causal_off) : 0;
  const int t0 = rstart / TQ, t1 = (p.M + TQ - 1) / TQ;
  const float qk = p.qk_scale;
  const uint32_t q_base = lds_addr(&qlds[0][0]), g_base = lds_addr(&glds[0][0]);

  // With the forward's keep words (keep_keys) the mask is read, not
  // evaluated, and nothing is stored for the dQ kernel; otherwise the
  // decisions are evaluated and, with drop_bits, stored for it.
  constexpr bool from_keys = DROP == 2;
  const bool bits = DROP == 1 && p.drop_bits != nullptr;
  const int r32 = (p.M + 31) >> 5;
  for (int hh = 0; hh < nheads && t0 < t1; ++hh) {
    const int h = h0 + hh;
    const int64_t bh = (int64_t)b * p.H + h;
    __amdgpu_buffer_rsrc_t rbits = make_rsrc(p.drop_bits, 0), rkeys = rbits;
    if (bits)
      rbits = make_rsrc(p.drop_bits + bh * p.Mpad * p.n32,
                        __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)p.Mpad * p.n32 * 4)));
    if (from_keys)
      rkeys = make_rsrc(p.keep_keys + bh * r32 * p.N,
                        __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)r32 * p.N * 4)));
    // Keep words of tile t (from_keys): rows t*TQ + 32 qb .. +31 of key
    // key0 + c, loaded with the tile's Q and dO.
    uint32_t kcur[2] = {0u, 0u}, knext[2] = {0u, 0u};
    auto fetch_keys = [&](int t, uint32_t (&w)[2]) __attribute__((always_inline)) {
      if constexpr (from_keys) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const int key = key0 + c;
          const uint32_t rw = (uint32_t)((t * TQ + 32 * qb) >> 5);
          w[qb] = __builtin_amdgcn_raw_buffer_load_b32(
              rkeys, key < p.N ? (rw * (uint32_t)p.N + (uint32_t)key) * 4u : kOffNoneBwd, 0, 0);
        }
      }
    };
    const i32x4 wq = make_rsrc_words(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
    const i32x4 wg = make_rsrc_words(p.dout + b * p.sg0 + h * p.sg1, p.g_bytes);
    // dS blocks for bwd_dq_ds_kernel (p.ds): block (r0/32, key0/32) of this
    // head, lane l's 16 bytes of the first half (rows acc_row(0..7, g)) at
    // 16 l, of the second half (rows acc_row(8..15, g)) at 1024 + 16 l.
    // Non-temporal: the dS stream (about B*H*M*N bytes) would otherwise
    // evict the Q and dO tiles every key block re-reads from L2.
    const bool store_ds = p.ds != nullptr && key0 < p.N;
    const __amdgpu_buffer_rsrc_t rds =
        make_rsrc(p.ds + (store_ds ? bh * p.ds_head * 1024 : 0),
                  store_ds ? (uint32_t)(p.ds_head * 2048) : 0u);
    const float* nlg = p.nl + bh * p.Mpad;
    const float* xg = p.delta + bh * p.Mpad;
    float nst = 0.f, xst = 0.f;
    // Tile t into stage s: Q and dO rows by DMA, the row values by plain loads
    // (rows < Mpad always: Mpad is a multiple of the tile height).
    auto fetch = [&](int t, int s) __attribute__((always_inline)) {
      dma_tile<D, TQ, NW>(wq, p.sq2, t * TQ, q_base + (uint32_t)(s * TILE * 2), wave, lane);
      dma_tile<D, TQ, NW>(wg, p.sg2, t * TQ, g_base + (uint32_t)(s * TILE * 2), wave, lane);
      if (tid < TQ) {
        nst = nlg[t * TQ + tid];
        xst = xg[t * TQ + tid];
      }
    };
    auto stash = [&](int s) __attribute__((always_inline)) {
      if (tid < TQ) {
        nlds[s][tid] = nst;
        xlds[s][tid] = xst;
      }
    };
    fetch(t0, 0);
    fetch_keys(t0, kcur);
    vm_wait_all();
    stash(0);
    __syncthreads();
    auto step = [&](int t, auto stage_tag) __attribute__((always_inline)) {
      constexpr int stage = decltype(stage_tag)::value;
      const bool more = t + 1 < t1;
      if (more) {
        fetch(t + 1, stage ^ 1);
        fetch_keys(t + 1, knext);
      }
      const uint16_t* qt = qlds[stage];
      const uint16_t* gt = glds[stage];
      // One 32-row block.  The mask (diagonal blocks only) changes the
      // weights alone: the masked and unmasked copies of the elementwise
      // part join before the dV / dK products, so the 128 accumulator
      // registers stay on one code path (two copies of the whole block gave
      // them different registers, merged by 128 moves per block).
      auto body = [&](int qb, bool full) __attribute__((always_inline)) {
        const int r0 = t * TQ + 32 * qb;
        // Register r holds query row r0 + acc_row(r, g) and key key0 + c.
        f32x16 s = f32x16{}, dp;
        if constexpr (DROP) {
          dp = f32x16{};
        } else {
          load8(dp, &xlds[stage][32 * qb + 8 * g], 0, 0);
          load8(dp, &xlds[stage][32 * qb + 16 + 8 * g], 0, 1);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          s = E::mma(lds_row_chunk<D>(qt, 32 * qb + perm_row(c), ks, g), kreg[ks], s);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          dp = E::mma(lds_row_chunk<D>(gt, 32 * qb + perm_row(c), ks, g), vreg[ks], dp);
        f32x16 nl;
        load8(nl, &nlds[stage][32 * qb + 8 * g], 0, 0);
        load8(nl, &nlds[stage][32 * qb + 16 + 8 * g], 0, 1);
        f32x16 pr;
#pragma unroll
        for (int r = 0; r < 16; ++r) pr[r] = exp2f_fast(fmaf(s[r], qk, nl[r]));
        if (!full) {
          // Row r0 + acc_row(r, g) sees key key0 + c iff acc_row(r, g) >= lim;
          // keys past N see no row (lim 32).  Without that their weight
          // would be exp2(nl[row]) (s = 0 from the zero K rows), whose dS
          // can round to inf in the input type and turn the dQ product over
          // the stored blocks into inf * 0.
          const int lim = key0 + c >= p.N ? 32
                          : p.causal     ? key0 + c - p.causal_off - r0
                                         : -32;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row(r, g) < lim) pr[r] = 0.f;
        }
        if constexpr (DROP) {
          // Keep bits for the dQ kernel (p.drop_bits): the ballot of
          // register r's keep decisions is the block's keys for rows
          // acc_row(r, 0) (lanes 0-31) and acc_row(r, 1) (lanes 32-63);
          // lane L collects row r0 + L's word and lanes 0-31 store them.
          // The keep decisions come first, all 16 Philox evaluations free to
          // interleave; the lane writes (inline assembly, which the compiler
          // does not move instructions across) follow in their own pass.
          bool keep[16];
          if constexpr (from_keys) {
            // Bit acc_row(r, g) = 16 (r / 8) + 8 g + r % 8 of the block's word.
            const uint32_t wb = kcur[qb] >> (8 * g);
#pragma unroll
            for (int r = 0; r < 16; ++r) keep[r] = (wb >> (16 * (r >> 3) + (r & 7))) & 1u;
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const uint32_t idx =
                  ((uint32_t)bh * (uint32_t)p.M + (uint32_t)(r0 + acc_row(r, g))) *
                      (uint32_t)p.N + (uint32_t)(key0 + c);
              keep[r] = dropout_keep(p.drop, idx);
            }
          }
          f32x16 nd;  // -delta of row acc_row(r, g)
          load8(nd, &xlds[stage][32 * qb + 8 * g], 0, 0);
          load8(nd, &xlds[stage][32 * qb + 16 + 8 * g], 0, 1);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[r] = keep[r] ? pr[r] : 0.f;
            dp[r] = pr[r] * ((keep[r] ? p.drop.scale * dp[r] : 0.f) + nd[r]);
          }
          uint32_t word = 0;
          if (bits) {
            // Registers r .. r+3 (acc_row(r, 0) = 16 (r / 8) + r % 8) per
            // group of four ballots.
            static_for<4>([&](auto qi) __attribute__((always_inline)) {
              constexpr int r = 4 * decltype(qi)::value;
              constexpr int L = 16 * (r >> 3) + (r & 7);
              const uint64_t bk[4] = {__builtin_amdgcn_ballot_w64(keep[r]),
                                      __builtin_amdgcn_ballot_w64(keep[r + 1]),
                                      __builtin_amdgcn_ballot_w64(keep[r + 2]),
                                      __builtin_amdgcn_ballot_w64(keep[r + 3])};
              write_lanes8<L, L + 8, L + 1, L + 9, L + 2, L + 10, L + 3, L + 11>(word, bk);
            });
          }
          if (bits && key0 < p.N)
            __builtin_amdgcn_raw_buffer_store_b32(
                word, rbits,
                lane < 32 ? (uint32_t)((((r0 >> 5) * p.n32 + (key0 >> 5)) << 5) + lane) * 4u
                          : kOffNoneBwd,
                0, 0);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[r] = pr[r];
            dp[r] = pr[r] * dp[r];
          }
        }
        const u32x4 pb0 = pack_b<E>(s, 0), pb1 = pack_b<E>(s, 1);
        const u32x4 sb0 = pack_b<E>(dp, 0), sb1 = pack_b<E>(dp, 1);
        if (store_ds) {
          const uint32_t blk =
              (uint32_t)(ds_block_start32(r0 >> 5, p.ds_a, p.n32) + (key0 >> 5)) * 2048u;
          buf_store16_nt(sb0, rds, blk + 16u * (uint32_t)lane);
          buf_store16_nt(sb1, rds, blk + 1024u + 16u * (uint32_t)lane);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          dv[db] = E::mma(lds_vt_operand<D>(gt, db, 2 * qb, lane), pb0, dv[db]);
          dv[db] = E::mma(lds_vt_operand<D>(gt, db, 2 * qb + 1, lane), pb1, dv[db]);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          dk[db] = E::mma(lds_vt_operand<D>(qt, db, 2 * qb, lane), sb0, dk[db]);
          dk[db] = E::mma(lds_vt_operand<D>(qt, db, 2 * qb + 1, lane), sb1, dk[db]);
        }
      };
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int r0 = t * TQ + 32 * qb;
        // Live if the block's last row sees the wave's first key, full if its
        // first row sees the wave's last key and every key lies below N.
        const bool live = !p.causal || p.causal_off + r0 + 31 >= key0;
        const bool full = (!p.causal || p.causal_off + r0 >= key0 + 31) && key0 + 31 < p.N;
        if (live) body(qb, full);
      }
      if (more) {
        vm_wait_all();
        stash(stage ^ 1);
        kcur[0] = knext[0];
        kcur[1] = knext[1];
      }
      __syncthreads();
    };
    for (int t = t0; t < t1; t += 2) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < t1) step(t + 1, std::integral_constant<int, 1>{});
    }
  }

  // Lane (c, g), register r of block db: key key0 + c, head dim
  // 32db + acc_row(r, g); registers 8hf..8hf+7 are 8 consecutive dims.
  const int key = key0 + c;
  if (key >= p.N) return;
  const float ks_ = p.scale_signed;
  if constexpr (DROP) {
#pragma unroll
    for (int db = 0; db < DB; ++db) dv[db] *= p.drop.scale;
  }
  if (!p.partial) {
    uint16_t* dkr = p.dk + b * p.sdk0 + hk * p.sdk1 + (int64_t)key * p.sdk2;
    uint16_t* dvr = p.dv + b * p.sdv0 + hk * p.sdv1 + (int64_t)key * p.sdv2;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int d0 = 32 * db + 16 * hf + 8 * g;
        if (d0 < D) {
          f32x16 x = dk[db] * ks_;
          *reinterpret_cast<u32x4*>(dkr + d0) = pack_b<E>(x, hf);
          *reinterpret_cast<u32x4*>(dvr + d0) = pack_b<E>(dv[db], hf);
        }
      }
  } else {
    float* pr = p.part + (((int64_t)b * p.H + h0) * p.N + key) * (2 * D);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int d0 = 32 * db + 16 * hf + 8 * g;
        if (d0 < D) {
          const f32x16& x = dk[db];
          const f32x16& y = dv[db];
          const int r = 8 * hf;
          *reinterpret_cast<f32x4*>(pr + d0) =
              f32x4{x[r] * ks_, x[r + 1] * ks_, x[r + 2] * ks_, x[r + 3] * ks_};
          *reinterpret_cast<f32x4*>(pr + d0 + 4) =
              f32x4{x[r + 4] * ks_, x[r + 5] * ks_, x[r + 6] * ks_, x[r + 7] * ks_};
          *reinterpret_cast<f32x4*>(pr + D + d0) = f32x4{y[r], y[r + 1], y[r + 2], y[r + 3]};
          *reinterpret_cast<f32x4*>(pr + D + d0 + 4) =
              f32x4{y[r + 4], y[r + 5], y[r + 6], y[r + 7]};
        }
      }
  }
}

// dK, dV of KV head hk = sum over its G query heads of the fp32 partials, in
// head order; one thread per 8 elements.
template <class E, int D>
__global__ __launch_bounds__(256) void bwd_dkdv_reduce_kernel(const BwdParams p) {
  constexpr int CPR = D / 8;
  const int64_t total = (int64_t)p.B * p.Hk * p.N * CPR;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int ch = (int)(i % CPR);
    const int64_t r = i / CPR;
    const int key = (int)(r % p.N);
    const int64_t bhk = r / p.N;
    const int hk = (int)(bhk % p.Hk), b = (int)(bhk / p.Hk);
    float a[8] = {}, v[8] = {};
    for (int j = 0; j < p.G; ++j) {
      const float* src = p.part + (((int64_t)b * p.H + hk * p.G + j) * p.N + key) * (2 * D) + 8 * ch;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a[e] += src[e];
        v[e] += src[D + e];
      }
    }
    const int d0 = 8 * ch;
    *reinterpret_cast<u32x4*>(p.dk + b * p.sdk0 + hk * p.sdk1 + (int64_t)key * p.sdk2 + d0) =
        u32x4{E::pack(a[0], a[1]), E::pack(a[2], a[3]), E::pack(a[4], a[5]), E::pack(a[6], a[7])};
    *reinterpret_cast<u32x4*>(p.dv + b * p.sdv0 + hk * p.sdv1 + (int64_t)key * p.sdv2 + d0) =
        u32x4{E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]), E::pack(v[6], v[7])};
  }
}

// ---------------------------------------------------------------- dQ

// DROP: dS = P (r Z dP - delta) as in the dK/dV kernel (flash.py:885-895),
// Z by Philox (DROP 1) or from the keep bits in drop_bits (DROP 2).
template <class E, int D, int DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_dq_kernel(const BwdParams p) {
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int NW = 4;
  constexpr int BM = 32 * NW;  // query rows per workgroup
  constexpr int BN = 64;       // keys per tile
  constexpr int TILE = BN * D;

  __shared__ __attribute__((aligned(16))) uint16_t klds[2][TILE];
  __shared__ __attribute__((aligned(16))) uint16_t vlds[2][TILE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int nbh = p.B * p.H;
  int rb = blockIdx.x / nbh;
  const int bh = blockIdx.x % nbh;
  if (p.causal) rb = p.nrb - 1 - rb;  // longest row blocks first
  const int b = bh / p.H, h = bh % p.H, hk = h / p.G;
  const int row0 = rb * BM, wrow0 = row0 + 32 * wave, qrow = wrow0 + c;

  // Q and dO (B operands of S^T = K Q^T and dP^T = V dO^T): lane holds row
  // qrow, head dims [16ks + 8g, +8).
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(p.dout + b * p.sg0 + h * p.sg1, p.g_bytes);
  u32x4 qreg[KS], greg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qreg[ks] = buf_load16(rq, (uint32_t)((qrow * p.sq2 + 16 * ks + 8 * g) * 2)) ^ p.qneg;
    greg[ks] = buf_load16(rg, (uint32_t)((qrow * p.sg2 + 16 * ks + 8 * g) * 2));
  }
  // Rows past M read nl = -inf (padding), so their P is 0.
  const float nl = p.nl[(int64_t)bh * p.Mpad + qrow];
  const float xl = p.delta[(int64_t)bh * p.Mpad + qrow];
  const uint32_t drow = ((uint32_t)bh * (uint32_t)p.M + (uint32_t)qrow) * (uint32_t)p.N;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qreg[ks]), "+v"(greg[ks]));

  // Key tiles: [0, ntiles) for the workgroup, [0, wtiles) for this wave,
  // [0, tfull) without any mask.
  const int hi = p.causal ? min(p.N, max(0, p.causal_off + row0 + BM)) : p.N;
  const int ntiles = (hi + BN - 1) / BN;
  const int whi = p.causal ? min(p.N, max(0, p.causal_off + wrow0 + 32)) : p.N;
  const int wtiles = (whi + BN - 1) / BN;
  int tfull = p.N / BN;
  if (p.causal) tfull = min(tfull, max(0, p.causal_off + wrow0 + 1) / BN);

  const i32x4 wk = make_rsrc_words(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const i32x4 wv = make_rsrc_words(p.v + b * p.sv0 + hk * p.sv1, p.v_bytes);
  const uint32_t k_base = lds_addr(&klds[0][0]), v_base = lds_addr(&vlds[0][0]);
  auto fetch = [&](int t, int s) __attribute__((always_inline)) {
    dma_tile<D, BN, NW>(wk, p.sk2, t * BN, k_base + (uint32_t)(s * TILE * 2), wave, lane);
    dma_tile<D, BN, NW>(wv, p.sv2, t * BN, v_base + (uint32_t)(s * TILE * 2), wave, lane);
  };

  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = f32x16{};
  const float qk = p.qk_scale;
  const VtOff vto = vt_offsets<D>(lane);
  const uint32_t rco = row_chunk_offset<D>(perm_row(c), g);

  // Keep words of tile t (dropout with p.drop_bits): this row's keys
  // 64t .. 64t+31 and 64t+32 .. 64t+63, loaded with the tile's K and V.
  constexpr bool bits = DROP == 2;
  __amdgpu_buffer_rsrc_t rbits = make_rsrc(p.drop_bits, 0);
  if (bits)
    rbits = make_rsrc(p.drop_bits + (int64_t)bh * p.Mpad * p.n32,
                      __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)p.Mpad * p.n32 * 4)));
  uint32_t wcur[2] = {0u, 0u}, wnext[2] = {0u, 0u};
  auto fetch_bits = [&](int t, uint32_t (&w)[2]) __attribute__((always_inline)) {
    if constexpr (DROP) {
      if (bits) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int kw = 2 * t + j;
          w[j] = __builtin_amdgcn_raw_buffer_load_b32(
              rbits, kw < p.n32 ? (uint32_t)((((wrow0 >> 5) * p.n32 + kw) << 5) + c) * 4u
                                : kOffNoneBwd,
              0, 0);
        }
      }
    }
  };
  if (ntiles > 0) {
    fetch(0, 0);
    fetch_bits(0, wcur);
    vm_wait_all();
    __syncthreads();
  }
  auto step = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_tag)::value;
    const bool more = t + 1 < ntiles;
    if (more) {
      fetch(t + 1, stage ^ 1);
      fetch_bits(t + 1, wnext);
    }
    const uint16_t* kt = klds[stage];
    const uint16_t* vt = vlds[stage];
    // One 32-key sub-block.  The mask (tiles at the diagonal or the key
    // edge) only zeroes weights, and both cases join before the dQ
    // products, so the dQ accumulators stay on one code path.
    auto body = [&](int kb2, bool full) __attribute__((always_inline)) {
      const int kbase = t * BN + 32 * kb2;
      // Fenced per sub-block, operand fetches pinned two k-steps ahead of
      // their MFMAs: left free, the scheduler hoists every fetch of the tile
      // and the kernel needs more than 256 VGPRs.
      __builtin_amdgcn_sched_barrier(0);
      uint32_t ro = rco;
      opaque(ro);
      u32x4 ak[KS], av[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        ak[ks] = lds_row_chunk(kt + 32 * kb2 * D, ro, ks);
        av[ks] = lds_row_chunk(vt + 32 * kb2 * D, ro, ks);
      }
      // Register r holds key kbase + acc_row(r, g) for query row qrow.  S
      // starts from a zero accumulator (an inline constant of the first
      // MFMA), dP - delta from -delta.
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = DROP ? 0.f : xl;
      s = E::mma(ak[0], qreg[0], f32x16{});
      dp = E::mma(av[0], greg[0], dp);
#pragma unroll
      for (int ks = 1; ks < KS; ++ks) {
        s = E::mma(ak[ks], qreg[ks], s);
        dp = E::mma(av[ks], greg[ks], dp);
      }
      {
        constexpr int PD = KS < 2 ? KS : 2;
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * PD, 0);  // DS read
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
          if (i + PD < KS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
      }
      // Key kbase + acc_row(r, g) is admissible iff acc_row(r, g) < lim.
      const int lim = (p.causal ? min(p.N, p.causal_off + qrow + 1) : p.N) - kbase;
      float pr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pr[r] = exp2f_fast(fmaf(s[r], qk, nl));
        if (!full && acc_row(r, g) >= lim) pr[r] = 0.f;
      }
      if constexpr (DROP) {
        if constexpr (bits) {
          // The dK/dV kernel's keep bits: bit acc_row(r, g) of the word of
          // this row and sub-block.
          const uint32_t wb = wcur[kb2] >> (8 * g);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool keep = (wb >> (16 * (r >> 3) + (r & 7))) & 1u;
            dp[r] = pr[r] * ((keep ? p.drop.scale * dp[r] : 0.f) + xl);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const uint32_t idx = drow + (uint32_t)(kbase + acc_row(r, g));
            dp[r] = pr[r] * ((dropout_keep(p.drop, idx) ? p.drop.scale * dp[r] : 0.f) + xl);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] = pr[r] * dp[r];
      }
      const u32x4 sb0 = pack_b<E>(dp, 0), sb1 = pack_b<E>(dp, 1);
      __builtin_amdgcn_sched_barrier(0);
      VtOff o = vto;
      opaque(o);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dq[db] = E::mma(lds_vt_operand<D>(kt, o, db, 2 * kb2), sb0, dq[db]);
        dq[db] = E::mma(lds_vt_operand<D>(kt, o, db, 2 * kb2 + 1), sb1, dq[db]);
      }
      {
        // K^T fetches (two transposing reads each) one MFMA ahead.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 2 * DB; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i + 2 < 2 * DB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
      }
    };
    if (t < wtiles) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        // Sub-blocks past this wave's last visible key are skipped.
        if (t * BN + 32 * kb2 < whi) body(kb2, t < tfull);
      }
    }
    if (more) {
      vm_wait_all();
      wcur[0] = wnext[0];
      wcur[1] = wnext[1];
    }
    __syncthreads();
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
  }

  // Lane (c, g), register r of block db: row qrow, head dim 32db + acc_row(r, g).
  if (qrow >= p.M) return;
  uint16_t* dqr = p.dq + b * p.sdq0 + h * p.sdq1 + (int64_t)qrow * p.sdq2;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int d0 = 32 * db + 16 * hf + 8 * g;
      if (d0 < D) {
        const f32x16 x = dq[db] * p.scale_signed;
        *reinterpret_cast<u32x4*>(dqr + d0) = pack_b<E>(x, hf);
      }
    }
}

constexpr int kBwdDqDsWaves = 8;  // waves (32 rows each) per bwd_dq_ds_kernel workgroup

// dQ from the dS blocks the dK/dV kernel stored (p.ds): query-block outer, a
// wave owns 32 rows and streams 64-key tiles; per tile the workgroup's K rows
// and each wave's two dS blocks arrive in LDS by DMA, and
//   dQ^T += K^T dS^T
// takes both operands from LDS with the transposing read.  The dS blocks
// are stored as the dK/dV kernel's B-operand fragments (lane l of a 2 KiB
// block: key l % 32, eight consecutive rows per 16 bytes, at 16 l and
// 1024 + 16 l), so the DMA gathers them into a swizzled [64 keys][32 rows]
// tile, whose transposing
// read yields rows on lanes and eight consecutive keys per lane, the B
// operand; lane c then holds row perm_row(c) of the wave.  Blocks a causal
// mask hides were never stored and are not read.  No recomputation of S and
// dP, no dropout (dS already carries it), and the same dS values as dK.
//
// The kernel is bound by the dS stream from HBM and by the latency of the K
// tiles from L2, so both run two tiles ahead (three LDS stages each) for
// 256-row workgroups of eight waves: 144 KiB of LDS, one workgroup per CU.
// Every wave issues its K DMAs and then exactly four dS DMAs per tile
// (blocks outside the visible range read from an offset past the buffer:
// zeros, no memory traffic), so at the end of a step "vmcnt <= this wave's
// DMA count of one tile" means everything but the newest tile has landed
// (vector loads complete in issue order).
template <class E, int D>
__global__ __launch_bounds__(512) void bwd_dq_ds_kernel(const BwdParams p) {
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int NW = kBwdDqDsWaves;
  constexpr int BM = 32 * NW;     // query rows per workgroup
  constexpr int BN = 64;          // keys per tile
  constexpr int TILE = BN * D;
  constexpr int STILE = BN * 32;  // a wave's dS^T tile
  constexpr int KBLK = TILE / 512;  // 1 KiB K blocks per tile, dealt to the waves
  static_assert(KBLK % NW == 0 || NW % KBLK == 0, "K DMA blocks per wave");

  __shared__ __attribute__((aligned(16))) uint16_t klds[3][TILE];
  __shared__ __attribute__((aligned(16))) uint16_t slds[3][NW][STILE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  // Workgroup i runs on XCD i % 8: each XCD takes the row blocks of its own
  // B*H/8 heads (their K rows stay in its L2), row-block major and, under a
  // causal mask, longest first across those heads, so the CUs that finish
  // short blocks take the next-longest ones (heads one after another instead
  // left CUs that had finished mid-length blocks with full-length ones: 160
  // against 120 us at B1 H32 S4096 D128 causal).
  const int nrb = (p.Mpad + BM - 1) / BM;
  const int total = (int)gridDim.x;
  const int nbh = total / nrb;
  int bid = blockIdx.x;
  const bool xcd = total % 8 == 0 && nbh % 8 == 0;
  if (xcd) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  const int per = xcd ? nbh / 8 : nbh;  // heads per XCD
  const int run = bid / (per * nrb), idx = bid % (per * nrb);
  const int bh = run * per + idx % per;
  int rb = idx / per;
  if (p.causal) rb = nrb - 1 - rb;  // longest row blocks first
  const int b = bh / p.H, h = bh % p.H, hk = h / p.G;
  const int row0 = rb * BM, wrow0 = row0 + 32 * wave;

  // Key tiles of the workgroup; this wave's visible 32-key blocks [0, wblk).
  const int hi = p.causal ? min(p.N, max(0, p.causal_off + row0 + BM)) : p.N;
  const int ntiles = (hi + BN - 1) / BN;
  const int whi = wrow0 >= p.M ? 0
                  : p.causal ? min(p.N, max(0, p.causal_off + wrow0 + 32))
                             : p.N;
  const int wblk = (whi + 31) >> 5;
  const uint32_t sblk =
      wblk > 0 ? (uint32_t)ds_block_start32(wrow0 >> 5, p.ds_a, p.n32) * 2048u : 0u;

  const i32x4 wk = make_rsrc_words(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const i32x4 wd = make_rsrc_words(p.ds + (int64_t)bh * p.ds_head * 1024,
                                    (uint32_t)(p.ds_head * 2048));
  const uint32_t k_base = lds_addr(&klds[0][0]);
  const uint32_t s_base = lds_addr(&slds[0][wave][0]);
  // DMA lane l of step i fills tile key 16 i + l / 4, physical chunk l % 4,
  // i.e. rows 8 ch .. 8 ch + 7 with ch = (l % 4) ^ swz<32>(key): half ch / 2
  // of the stored block, lane (key % 32) + 32 (ch % 2).
  uint32_t goff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 16 * i + (lane >> 2);
    const int ch = (lane & 3) ^ swz<32>(key);
    goff[i] = (uint32_t)((key >> 5) * 2048 + (ch >> 1) * 1024 + ((key & 31) + 32 * (ch & 1)) * 16);
  }
  auto fetch = [&](int t) __attribute__((always_inline)) {
    const int st = t % 3;
    dma_tile<D, BN, NW>(wk, p.sk2, t * BN, k_base + (uint32_t)(st * TILE * 2), wave, lane);
    const uint32_t lb = s_base + (uint32_t)(st * NW * STILE * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool vis = 2 * t + (i >> 1) < wblk;
      dma16_nt(wd, vis ? sblk + (uint32_t)(2 * t) * 2048u + goff[i] : kOffNoneBwd,
               lb + 1024u * (uint32_t)i);
    }
  };
  // Wait for everything but the newest tile's DMAs (ahead) or for all.
  auto wait_ahead = [&](bool ahead) __attribute__((always_inline)) {
    if (!ahead) {
      vm_wait_all();
    } else if constexpr (KBLK >= NW) {
      static_assert(KBLK % NW == 0 && KBLK / NW <= 2, "K DMA count per wave");
      if constexpr (KBLK / NW == 2)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    } else {
      if (wave < KBLK)
        asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    }
  };

  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = f32x16{};
  const VtOff vto = vt_offsets<D>(lane);
  const VtOff vts = vt_offsets<32>(lane);

  if (ntiles > 0) {
    fetch(0);
    if (ntiles > 1) fetch(1);
    wait_ahead(ntiles > 1);
    __syncthreads();
  }
  for (int t = 0; t < ntiles; ++t) {
    if (t + 2 < ntiles) fetch(t + 2);
    const uint16_t* kt = klds[t % 3];
    const uint16_t* st = slds[t % 3][wave];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      if (2 * t + kb2 < wblk) {
        VtOff o = vto, os = vts;
        opaque(o);
        opaque(os);
        const u32x4 sb0 = lds_vt_operand<32>(st, os, 0, 2 * kb2);
        const u32x4 sb1 = lds_vt_operand<32>(st, os, 0, 2 * kb2 + 1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          dq[db] = E::mma(lds_vt_operand<D>(kt, o, db, 2 * kb2), sb0, dq[db]);
          dq[db] = E::mma(lds_vt_operand<D>(kt, o, db, 2 * kb2 + 1), sb1, dq[db]);
        }
      }
    }
    if (t + 1 < ntiles) {
      wait_ahead(t + 2 < ntiles);
      __syncthreads();
    }
  }

  // Lane (c, g), register r of block db: row wrow0 + perm_row(c), head dim
  // 32db + acc_row(r, g).
  const int qrow = wrow0 + perm_row(c);
  if (qrow >= p.M) return;
  uint16_t* dqr = p.dq + b * p.sdq0 + h * p.sdq1 + (int64_t)qrow * p.sdq2;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int d0 = 32 * db + 16 * hf + 8 * g;
      if (d0 < D) {
        const f32x16 x = dq[db] * p.scale_signed;
        *reinterpret_cast<u32x4*>(dqr + d0) = pack_b<E>(x, hf);
      }
    }
}

}  // namespace fas
