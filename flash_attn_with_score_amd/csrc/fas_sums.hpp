// gfx950 kernels for the column-type side products.
//
// Softmax-weight column sums (attention_with_col_softmax_sum.py:195-270,
// attention_cross_token_softmax_sum.py:203-268 and the buffered :568-627)
// are computed after the forward pass, key-block outer: a workgroup owns two
// blocks of 256 keys of one (batch, query head), keeps them in VGPRs and
// streams the query rows that can see them (colsm64_kernel).  S = Q K^T puts keys on lanes and
// queries in the accumulator registers, so P = exp2(s*qk_scale - lse2[row])
// (the forward pass's final base-2 log-sum-exp) is summed over queries
// in-lane.  Every column is owned by one workgroup: no atomics, the result is
// deterministic.
// GQA groups are folded inside the pass: a workgroup walks the query heads
// of its KV head with its keys resident, or, when that would leave CUs idle,
// shares them with other workgroups and the last one to finish adds their
// column sums in a fixed order.
//
// Raw-score column sums (attention_with_col_sum.py:186-191,
// attention_with_col_sum_sequential.py:177-182,
// attention_cross_token_qk_sum.py:169-216) are linear in q:
//   sum_{i admissible for j} (q_i . k_j) * sm_scale = (sum_i q_i) . k_j * sm_scale
// so they need per-64-row block sums of q (qsum_blocks_kernel) and one dot
// product per key (colraw_kernel, which also forms the exclusive suffix over
// blocks and the in-block suffix): O(N*D) work and one read of Q and K
// instead of a reduction over the N*N score matrix.
#pragma once
#include "fas_device.hpp"
#include "fas_params.hpp"

#include <type_traits>

namespace fas {

// Byte offset past every buffer extent: the load returns 0.
constexpr uint32_t kOffNoneSums = 0x80000000u;

// ---------------------------------------------------------------- softmax

// Workgroup bid runs on XCD bid % 8.  Work items [0, T) are dealt to the
// XCDs in contiguous runs: XCD x takes ceil((T - x) / 8) of them, so items
// that read the same rows of q or k (neighbours in item order) share an L2.
__device__ __forceinline__ int xcd_item(int bid, int T) {
  const int x = bid & 7, s = bid >> 3;
  return x * (T >> 3) + min(x, T & 7) + s;
}

// Column-pass work item: unit u of the nunits per output group (a key block
// or a mirror pair of them), head split sp, output group og; item order
// (og, sp, u), u fastest, so the units reading one split's q rows are
// neighbours.
struct ColItem {
  int unit, sp, og;
};
__device__ __forceinline__ ColItem col_item(int bid, int nunits, int nsplit, int nog) {
  const int item = xcd_item(bid, nunits * nsplit * nog);
  ColItem c;
  c.unit = item % nunits;
  const int rest = item / nunits;
  c.sp = rest % nsplit;
  c.og = rest / nsplit;
  return c;
}

// With a head split (p.nsplit > 1) the splits of a unit run on other XCDs,
// whose L2 caches are not coherent with this one's, so their column sums
// meet at device scope: each split stores them with device-scope (relaxed
// atomic) stores, which write through to the device's coherent level, and
// waits for them to complete; one thread then takes the unit's ticket (a
// device-scope atomic), and the workgroup that takes the last one reads the
// nsplit partials of keys [kA0, kA1) and [kB0, kB1) with device-scope loads
// and adds them in split order.  Fences would write back and invalidate the
// whole L2 at every workgroup's end instead (measured: config-3 column pass
// 75 -> 108 us).
__device__ __forceinline__ void store_part(const ColsmParams& p, const ColItem& it, int key,
                                           float v) {
  __hip_atomic_store(&p.part[((int64_t)it.og * p.nsplit + it.sp) * p.ncols + key], v,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void col_fold_splits(const ColsmParams& p, const ColItem& it,
                                                int nunits, int kA0, int kA1, int kB0, int kB1,
                                                bool* last_flag) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    *last_flag = __hip_atomic_fetch_add(&p.ticket[(int64_t)it.og * nunits + it.unit], 1u,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(p.nsplit - 1);
  __syncthreads();
  if (!*last_flag) return;
  const int hout = p.H / p.fold;
  const int b = it.og / hout, ho = it.og - b * hout;
  float* src = p.part + (int64_t)it.og * p.nsplit * p.ncols;
  auto fold_range = [&](int k0, int k1) {
    for (int key = k0 + (int)threadIdx.x; key < k1; key += (int)blockDim.x) {
      // Eight loads in flight at a time (they miss the L2), added in split
      // order; splits past nsplit add 0.
      float acc = 0.f;
      for (int s0 = 0; s0 < p.nsplit; s0 += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = s0 + i < p.nsplit
                     ? __hip_atomic_load(&src[(int64_t)(s0 + i) * p.ncols + key],
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += v[i];
      }
      p.out[b * p.so0 + ho * p.so1 + (int64_t)key * p.so2] = acc;
    }
  };
  fold_range(kA0, kA1);
  fold_range(kB0, kB1);
}

// The column pass with 64 keys per wave.  Each 32x16 Q operand fetched from
// LDS feeds two MFMAs (the wave's two 32-key sets), so a CU reads half the
// LDS bytes per MFMA of a wave holding 32 keys (one 1 KiB fetch per
// v_mfma_32x32x16, which at full MFMA rate on four SIMDs is the whole LDS
// bandwidth).  Workgroup: 8 waves = 4 key groups (64 keys each, a
// 256-key block) x 2 row groups; a step stages 128 query rows, row group rg
// taking rows [64 rg, 64 rg + 64).  The two row groups' column sums of a key
// are added through LDS at the end of the block, in a fixed order.
// Key blocks of 256 are dealt in mirror pairs (pb, nkb-1-pb): under a
// causal mask block kb sees (M - 256 kb) query rows, so a pair always sums
// to the same amount of work and every workgroup finishes together.  Keys
// sit on lanes and queries in the accumulator registers; the row's
// -lse2/qk_scale is the accumulator's starting value, so P = exp2(acc *
// qk_scale) is summed over queries in-lane.  Per 32 x 32 block a wave
// issues 8 MFMAs against 16 exp, 16 multiply and 16 add instructions
// (measured: 81.8 us with 32 keys per wave, 76.9 us with 64, at B1 H32
// S4096 D128 fp16 causal).  Interleaving a block's exponentials with the
// next block's MFMAs, or streaming Q by LDS DMA in 256-row steps, left the
// time unchanged: at the board's power limit the energy of this work, not
// its issue order, bounds the pass.
// GQA (attention_with_col_softmax_sum.py:61-67, 264-270 add every query
// head of a KV head into one column): the workgroup walks the query heads
// of its split one after the other with its keys resident in VGPRs, the
// column sums accumulating over all of them in registers; the row steps of
// consecutive heads form one pipeline (the next head's first rows are
// fetched during the current head's last step).  K is therefore read once
// per workgroup, not once per query head.
// LN: the row offsets come from a natural-log normalizer (p.lse_ln,
// total_attention) instead of the forward's base-2 LSE; a template flag so
// the default copy carries no conversion code in its loop.
// DROP: the weights pass through the dropout mask before the sum, as the
// reference's column pass does (attention_with_col_softmax_sum.py:237-244):
// 1 evaluates the mask's Philox stream again, 2 reads the keep bits the
// forward pass stored (one word per key and 32-row block, prefetched with
// the next step's Q rows).
// The sign of a negative sm_scale is applied to K once per block.
// The Philox instances (DROP 1, used only when the keep bits do not fit) are
// too large for the compiler to unroll the two-block loop below; it stays a
// loop there, and the warning saying so is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <class E, int D, bool LN, int DROP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void colsm64_kernel(const ColsmParams p) {
  constexpr int KS = D / 16;
  constexpr int NT = 512;
  constexpr int BK = 256;           // keys per block (4 key groups x 64)
  constexpr int TQ = 128;           // query rows per step (2 row groups x 64)
  constexpr int CPR = D / 8;
  constexpr int CHUNKS = TQ * CPR;
  constexpr int CPT = (CHUNKS + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) uint16_t qlds[2][TQ * D];
  __shared__ __attribute__((aligned(16))) float llds[2][TQ];
  __shared__ float red[4][64];
  __shared__ bool last_flag;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lane = tid & 63, c = lane & 31, g = lane >> 5;
  const int kg = wave & 3, rg = wave >> 2;
  const int npairs = (p.nkb + 1) / 2;
  const int hout = p.H / p.fold;
  const ColItem item = col_item(blockIdx.x, npairs, p.nsplit, p.B * hout);
  const int pb = item.unit;
  const int b = item.og / hout, ho = item.og - b * hout;
  const int hfirst = ho * p.fold;   // first query head of the output group
  const int hk = hfirst / p.G;
  // Heads of this split: hfirst + j, j = sp, sp + nsplit, ... < fold.
  const int nheads = (p.fold - item.sp + p.nsplit - 1) / p.nsplit;
  const int kbb = p.nkb - 1 - pb;

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + b * p.sk0 + hk * p.sk1, p.k_bytes);
  const int t1 = (p.M + TQ - 1) / TQ;
  const int r32 = (p.M + 31) >> 5;

  u32x4 qst[CPT];
  float lst = 0.f;
  // Q rows and row offsets of step t of head h.
  auto fetch = [&](int h, int t) {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q + b * p.sq0 + h * p.sq1, p.q_bytes);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + i * NT;
      const int row = id / CPR, ch = id % CPR;
      qst[i] = buf_load16(rq, (uint32_t)(((t * TQ + row) * p.sq2 + ch * 8) * 2));
    }
    if (tid < TQ) {
      const int row = t * TQ + tid;
      if (row < p.row_lo || row >= p.M) {
        lst = pos_inf();
      } else if constexpr (!LN) {
        lst = p.lse2[(int64_t)(b * p.H + h) * p.M + row];
      } else {
        // total_attention(): the caller's natural-log normalizer, -inf for
        // rows that see no key (total.py:125-128).
        const float L = p.lse_ln[b * p.sl0 + h * p.sl1 + (int64_t)row * p.sl2];
        lst = L == neg_inf() ? pos_inf() : L * 1.44269504088896341f;
      }
    }
  };
  // LDS gets -lse2 / qk_scale, the starting value of the row's accumulator
  // (-inf for rows that do not contribute).
  const float inv_scale = 1.f / p.qk_scale;
  auto stash = [&](int stage) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = tid + i * NT;
      if (CHUNKS % NT == 0 || id < CHUNKS) {
        const int row = id / CPR, ch = id % CPR;
        *reinterpret_cast<u32x4*>(&qlds[stage][tile_off<D>(row, ch)]) = qst[i];
      }
    }
    if (tid < TQ) llds[stage][tid] = -lst * inv_scale;
  };

  int kA0 = 0, kA1 = 0, kB0 = 0, kB1 = 0;  // key ranges of the two blocks
  for (int blk = 0; blk < 2; ++blk) {
    const int kb = blk == 0 ? pb : kbb;
    if (blk == 1 && kbb == pb) break;
    if (blk == 0) {
      kA0 = kb * BK;
      kA1 = min(p.ncols, kA0 + BK);
    } else {
      kB0 = kb * BK;
      kB1 = min(p.ncols, kB0 + BK);
    }
    // Keys of this wave: [key0, key0 + 64), set j = keys key0 + 32 j + c.
    const int key0 = kb * BK + 64 * kg;
    u32x4 kreg[2][KS];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kreg[j][ks] =
            buf_load16(rk, (uint32_t)(((key0 + 32 * j + c) * p.sk2 + 16 * ks + 8 * g) * 2)) ^ p.qneg;
    // Settle the K loads here: left pending, the compiler's wait counters for
    // them would also hold back (vmcnt N) on the Q prefetch inside the loop.
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kreg[j][ks]));

    // Query steps that can see any key of the block.
    int rstart = p.row_lo;
    if (p.causal) rstart = max(rstart, kb * BK - p.causal_off);
    const int t0 = max(0, rstart) / TQ;
    const int nt = t1 > t0 ? t1 - t0 : 0;
    const int nsteps = nheads * nt;  // (head, step) pairs, head-major

    float colacc[2] = {0.f, 0.f};
    // Keep words of step t of head h (DROP == 2): block (qb, j) is rows
    // t*TQ + 64 rg + 32 qb .. +31 of key key0 + 32 j + c.
    uint32_t bcur[4] = {0u, 0u, 0u, 0u}, bnext[4] = {0u, 0u, 0u, 0u};
    auto fetch_bits = [&](int h, int t, uint32_t (&w)[4]) __attribute__((always_inline)) {
      if constexpr (DROP == 2) {
        const __amdgpu_buffer_rsrc_t rbits =
            make_rsrc(p.drop_bits + (int64_t)(b * p.H + h) * r32 * p.N,
                      __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)r32 * p.N * 4)));
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int key = key0 + 32 * j + c;
            const uint32_t rw = (uint32_t)((t * TQ + 64 * rg + 32 * qb) >> 5);
            w[2 * qb + j] = __builtin_amdgcn_raw_buffer_load_b32(
                rbits, key < p.N ? (rw * (uint32_t)p.N + (uint32_t)key) * 4u : kOffNoneSums, 0, 0);
          }
      }
    };
    // The step being computed (head ch, row step ct) and the one after it.
    int ch = hfirst + item.sp, ct = t0;
    auto advance = [&](int& h, int& t) __attribute__((always_inline)) {
      if (++t == t1) {
        t = t0;
        h += p.nsplit;
      }
    };
    if (nsteps > 0) {
      fetch(ch, ct);
      fetch_bits(ch, ct, bcur);
      stash(0);
    }
    __syncthreads();
    auto step = [&](int i, auto stage_tag) __attribute__((always_inline)) {
      constexpr int stage = decltype(stage_tag)::value;
      const bool more = i + 1 < nsteps;
      int nh = ch, ntt = ct;
      advance(nh, ntt);
      if (more) {
        fetch(nh, ntt);
        fetch_bits(nh, ntt, bnext);
      }
      const int t = ct;
      const uint32_t bh = (uint32_t)(b * p.H + ch);
      const int r0 = t * TQ + 64 * rg;  // this row group's first row
      const uint16_t* qt = qlds[stage];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int rq0 = r0 + 32 * qb;
        // Live if some row of the block sees the wave's first key, full if
        // every row sees its last.
        const bool live = !p.causal || p.causal_off + rq0 + 31 >= key0;
        const bool full = !p.causal || p.causal_off + rq0 >= key0 + 63;
        auto body = [&](auto mask_tag) __attribute__((always_inline)) {
          constexpr bool MASK = decltype(mask_tag)::value;
          // Fenced per query block: the scheduler would otherwise fetch the
          // next block's operands early and run out of registers.
          __builtin_amdgcn_sched_barrier(0);
          u32x4 a[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            a[ks] = lds_row_chunk<D>(qt, 64 * rg + 32 * qb + perm_row(c), ks, g);
          // Register r holds query row rq0 + acc_row(r, g); it starts at
          // -lse2[row] / qk_scale, so P = exp2(acc * qk_scale).
          f32x16 s[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const float* lp = &llds[stage][64 * rg + 32 * qb + 16 * hf + 8 * g];
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(lp);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(lp + 4);
            s[0][8 * hf + 0] = x0.x; s[0][8 * hf + 1] = x0.y;
            s[0][8 * hf + 2] = x0.z; s[0][8 * hf + 3] = x0.w;
            s[0][8 * hf + 4] = x1.x; s[0][8 * hf + 5] = x1.y;
            s[0][8 * hf + 6] = x1.z; s[0][8 * hf + 7] = x1.w;
          }
          s[1] = s[0];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            s[0] = E::mma(a[ks], kreg[0][ks], s[0]);
            s[1] = E::mma(a[ks], kreg[1][ks], s[1]);
          }
          {
            constexpr int PD = KS < 2 ? KS : 2;
            __builtin_amdgcn_sched_group_barrier(0x100, PD + 4, 0);  // DS read: 4 of -lse, PD of Q
#pragma unroll
            for (int i2 = 0; i2 < KS; ++i2) {
              __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
              if (i2 + PD < KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              s[j][r] = exp2f_fast(s[j][r] * p.qk_scale);
              if constexpr (MASK) {
                const int row = rq0 + acc_row(r, g);
                if (p.causal_off + row < key0 + 32 * j + c) s[j][r] = 0.f;
              }
              if constexpr (DROP == 1) {
                const uint32_t row = (uint32_t)(rq0 + acc_row(r, g));
                const uint32_t idx = (bh * (uint32_t)p.M + row) * (uint32_t)p.drop.n +
                                     (uint32_t)(key0 + 32 * j + c);
                if (!dropout_keep(p.drop, idx)) s[j][r] = 0.f;
              }
              if constexpr (DROP == 2) {
                // Bit acc_row(r, g) = 16 (r / 8) + 8 g + r % 8 of the block's
                // word, sign-extended to a mask (0 or all ones) for the weight.
                // (Through a float local: bit_cast of a vector element itself
                // read element 0 in this compiler.)
                const int m = __builtin_amdgcn_sbfe((int)(bcur[2 * qb + j] >> (8 * g)),
                                                    16 * (r >> 3) + (r & 7), 1);
                const float w = s[j][r];
                s[j][r] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w) & (uint32_t)m);
              }
            }
#pragma unroll
            for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
              for (int r = 0; r < w; ++r) s[j][r] += s[j][r + w];
            colacc[j] += s[j][0];
          }
        };
        if (live) {
          if (full) body(std::false_type{});
          else body(std::true_type{});
        }
      }
      if (more) {
        stash(stage ^ 1);
#pragma unroll
        for (int k = 0; k < 4; ++k) bcur[k] = bnext[k];
      }
      ch = nh;
      ct = ntt;
      __syncthreads();
    };
    for (int i = 0; i < nsteps; i += 2) {
      step(i, std::integral_constant<int, 0>{});
      if (i + 1 < nsteps) step(i + 1, std::integral_constant<int, 1>{});
    }
    // Fold the half-waves, then row group 1 into row group 0 (fixed order).
    float tot[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) tot[j] = xor32_add(colacc[j]);
    if (rg == 1 && g == 0) {
      red[kg][c] = tot[0];
      red[kg][32 + c] = tot[1];
    }
    __syncthreads();
    if (rg == 0 && g == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int key = key0 + 32 * j + c;
        if (key < p.ncols) {
          const float v = tot[j] + red[kg][32 * j + c];
          if (p.nsplit == 1)
            p.out[b * p.so0 + ho * p.so1 + (int64_t)key * p.so2] = v;
          else
            store_part(p, item, key, v);
        }
      }
    }
    __syncthreads();
  }
  if (p.nsplit > 1) col_fold_splits(p, item, npairs, kA0, kA1, kB0, kB1, &last_flag);
}
#pragma clang diagnostic pop

// Buffered source: pass 1 left the region (rows >= split, keys < split) as
// fp16 base-2 exponents y = (s - t) * qk_scale in p.region and t * qk_scale,
// t the row's maximum over the region keys of each 64-key tile, in
// p.region_m, so a weight is exp2(y + t * qk_scale - lse2).  A workgroup of
// 4 waves owns 256 keys of one output group and walks the query heads of its
// split one after the other: lane l of every wave holds keys 4 l .. 4 l + 3
// (one 64-key tile) and reads them as one 8-byte load per row, so a wave
// reads 512 bytes contiguous per row; the waves take every fourth row (the
// row and its lse2 are wave-uniform, the latter a scalar load), several rows
// in flight, and their sums meet in LDS in a fixed order.  Entries above a
// key's first admissible row were never written and are excluded by a
// select.  VEC: split % 4 == 0 (8-byte aligned lane groups); otherwise one
// key per lane.
template <bool VEC>
__global__ __launch_bounds__(256) void colsm_buffered_kernel(const ColsmParams p) {
  constexpr int KPL = VEC ? 4 : 1;  // keys per lane
  constexpr int BKB = 64 * KPL;     // keys per workgroup
  __shared__ float red[4][256];
  __shared__ bool last_flag;
  const int hout = p.H / p.fold;
  const ColItem item = col_item(blockIdx.x, p.nkb, p.nsplit, p.B * hout);
  const int kb = item.unit;
  const int b = item.og / hout, ho = item.og - b * hout;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int key0 = kb * BKB + KPL * lane;
  const int tile = key0 / 64;  // the lane's keys lie in one 64-key tile
  const int rows = max(0, p.M - p.split);
  // First admissible row of each key, and of the workgroup's first key.
  int rs[KPL];
#pragma unroll
  for (int e = 0; e < KPL; ++e) rs[e] = p.causal ? max(p.split, key0 + e - p.causal_off) : p.split;
  const int r_lo = p.causal ? max(p.split, kb * BKB - p.causal_off) : p.split;
  const bool live = key0 < p.ncols;
  float acc[KPL];
#pragma unroll
  for (int e = 0; e < KPL; ++e) acc[e] = 0.f;
  for (int h = ho * p.fold + item.sp; h < (ho + 1) * p.fold; h += p.nsplit) {
    const int64_t bh = (int64_t)b * p.H + h;
    const uint16_t* reg = p.region + bh * rows * p.split;
    const float* rm = p.region_m + tile * p.region_rows + bh * rows;
    const float* lse = p.lse2 + bh * p.M;
    auto row_step = [&](int row) __attribute__((always_inline)) {
      const float l = lse[row];
      const int64_t rr = row - p.split;
      const uint16_t* rp = reg + rr * p.split + key0;
      const float off = (live ? rm[rr] : 0.f) - l;
      float v[KPL];
      if constexpr (VEC) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 x = live ? __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(rp))
                             : u32x2{0u, 0u};
        v[0] = F16::to_f32((uint16_t)(x.x & 0xffffu));
        v[1] = F16::to_f32((uint16_t)(x.x >> 16));
        v[2] = F16::to_f32((uint16_t)(x.y & 0xffffu));
        v[3] = F16::to_f32((uint16_t)(x.y >> 16));
      } else {
        v[0] = live ? F16::to_f32(rp[0]) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < KPL; ++e) {
        const float w = exp2f_fast(v[e] + off);
        acc[e] += row >= rs[e] ? w : 0.f;
      }
    };
    // Eight rows in flight per wave: the pass is bound by load latency
    // where a workgroup has few rows (metric shape, split 3072: 71.1 us at
    // four rows in flight).
    int row = __builtin_amdgcn_readfirstlane(r_lo + wave);
#pragma unroll 1
    for (; row + 28 < p.M; row += 32) {
#pragma unroll
      for (int u = 0; u < 8; ++u) row_step(row + 4 * u);
    }
    for (; row < p.M; row += 4) row_step(row);
  }
#pragma unroll
  for (int e = 0; e < KPL; ++e) red[wave][KPL * lane + e] = acc[e];
  __syncthreads();
  const int t = threadIdx.x;
  const int key = kb * BKB + t;
  if (t < BKB && key < p.ncols) {
    const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    if (p.nsplit == 1)
      p.out[b * p.so0 + ho * p.so1 + (int64_t)key * p.so2] = v;
    else
      store_part(p, item, key, v);
  }
  if (p.nsplit > 1)
    col_fold_splits(p, item, p.nkb, kb * BKB, min(p.ncols, kb * BKB + BKB), 0, 0, &last_flag);
}

// ---------------------------------------------------------------- raw sums

// bsum[bhk][blk][:] = sum over the group's query heads and the rows
// [row_lo + 64*blk, +64) of q (fp32).
template <class E, int D>
__global__ __launch_bounds__(256) void qsum_blocks_kernel(const RawParams p) {
  constexpr int CPR = D / 8;          // threads per row
  constexpr int RPI = 256 / CPR;      // rows in flight
  __shared__ float red[RPI][D];
  const int blk = blockIdx.x, bhk = blockIdx.y;
  const int hk = bhk % p.Hk, b = bhk / p.Hk;
  const int ch = threadIdx.x % CPR, rg = threadIdx.x / CPR;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int r0 = p.row_lo + 64 * blk;
  const int r1 = min(p.M, r0 + 64);
  // Items (head gg, row r0 + rg + RPI j) in head-major order, four loads in
  // flight (a GQA group's G heads are G times the rows of one workgroup),
  // added in item order.
  constexpr int ITER = (64 + RPI - 1) / RPI;
  const int nitems = p.G * ITER;
  const uint16_t* qb = p.q + b * p.sq0 + (int64_t)(hk * p.G) * p.sq1 + ch * 8;
  auto load_item = [&](int i) __attribute__((always_inline)) {
    const int gg = i / ITER, row = r0 + rg + RPI * (i - gg * ITER);
    return i < nitems && row < r1
               ? *reinterpret_cast<const u32x4*>(qb + (int64_t)gg * p.sq1 + (int64_t)row * p.sq2)
               : u32x4{0u, 0u, 0u, 0u};
  };
  for (int i = 0; i < nitems; i += 4) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = load_item(i + u);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float x[8];
      unpack8<E>(v[u], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += x[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[rg][ch * 8 + e] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    float s = 0.f;
    for (int r = 0; r < RPI; ++r) s += red[r][d];
    p.bsum[((int64_t)bhk * (p.nblk + 1) + blk) * D + d] = s;
  }
}

// out[d] = sum of the block sums bs[blk][d] for blk in [lo, hi), by all 256
// threads of the workgroup (256/D per dimension, blocks strided between
// them, then a fixed-order combine), so the loads are independent and in
// flight together.  Call from every thread; ends with a barrier.
template <int D>
__device__ __forceinline__ void block_range_sum(const float* bs, int lo, int hi, float* out,
                                                float* scratch) {
  constexpr int TP = 256 / D;
  const int d = threadIdx.x % D, part = threadIdx.x / D;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int blk = lo + part;
  for (; blk + 3 * TP < hi; blk += 4 * TP) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += bs[(int64_t)(blk + u * TP) * D + d];
  }
  for (; blk < hi; blk += TP) acc[0] += bs[(int64_t)blk * D + d];
  scratch[threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (part == 0) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < TP; ++j) t += scratch[d + j * D];
    out[d] = t;
  }
  __syncthreads();
}

// One dot product per key with a per-key fp32 vector held in LDS rows.
template <class E, int D>
__device__ __forceinline__ float key_dot(const RawParams& p, const uint16_t* kbase, int key,
                                         const float* vec, int part) {
  constexpr int DP = D / 4;  // dims per thread (4 threads per key)
  const uint16_t* kr = kbase + (int64_t)key * p.sk2 + part * DP;
  float acc = 0.f;
#pragma unroll
  for (int d8 = 0; d8 < DP; d8 += 8) {
    float x[8];
    if constexpr (DP >= 8) {
      unpack8<E>(*reinterpret_cast<const u32x4*>(kr + d8), x);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = e < DP ? E::to_f32(kr[d8 + e]) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (d8 + e < DP) acc = fmaf(x[e], vec[part * DP + d8 + e], acc);
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  return acc;
}

// Causal column sums: workgroup w < nextra handles keys [64w, 64w+64) below
// causal_off (every row admissible); the others own one 64-row block rb and
// the keys j = row + causal_off of its rows.  Non-causal / cross: every
// workgroup owns p.kgroups groups of 64 keys and uses the total, which it
// sums from the head's block sums once for all of them (one group per
// workgroup re-read the whole block-sum table per 64 keys: at B2 H32 S8192
// four times the bytes of K from the L2).
template <class E, int D, bool SUFFIX>
__global__ __launch_bounds__(256) void colraw_kernel(const RawParams p) {
  __shared__ float vec[64][D];
  __shared__ float seed[D];
  __shared__ float scratch[256];
  const int bhk = blockIdx.y;
  const int hk = bhk % p.Hk, b = bhk / p.Hk;
  const float* bs = p.bsum + (int64_t)bhk * (p.nblk + 1) * D;
  const uint16_t* kbase = p.k + b * p.sk0 + hk * p.sk1;
  const int w = blockIdx.x;
  const int kslot = threadIdx.x >> 2, part = threadIdx.x & 3;

  if (!SUFFIX || w < p.nextra) {
    // Keys every query row sees: the sum over all row blocks.
    block_range_sum<D>(bs, 0, p.nblk, vec[0], scratch);
    const int lim = SUFFIX ? min(p.ncols, p.causal_off) : p.ncols;
    const int ng = SUFFIX ? 1 : p.kgroups;
    for (int kg = 0; kg < ng; ++kg) {
      const int key = 64 * (w * ng + kg) + kslot;
      if (key < lim) {
        const float dot = key_dot<E, D>(p, kbase, key, vec[0], part);
        if (part == 0) p.out[b * p.so0 + hk * p.so1 + (int64_t)key * p.so2] = dot * p.sm_scale;
      }
    }
    return;
  }
  // In-block suffix sums over rows [64rb, 64rb + 64) of the group's heads.
  const int rb = w - p.nextra;
  const int r0 = 64 * rb;
  // Rows of the later row blocks: the exclusive suffix over blocks.
  block_range_sum<D>(bs, rb + 1, p.nblk, seed, scratch);
  for (int i = threadIdx.x; i < 64 * D; i += 256) (&vec[0][0])[i] = 0.f;
  __syncthreads();
  {
    constexpr int CPR = D / 8;
    constexpr int RPI = 256 / CPR;
    const int ch = threadIdx.x % CPR, rg = threadIdx.x / CPR;
    for (int gg = 0; gg < p.G; ++gg) {
      const uint16_t* qh = p.q + b * p.sq0 + (int64_t)(hk * p.G + gg) * p.sq1 + ch * 8;
      for (int rr = rg; rr < 64; rr += RPI) {
        const int row = r0 + rr;
        if (row >= p.M) break;
        float x[8];
        unpack8<E>(*reinterpret_cast<const u32x4*>(qh + (int64_t)row * p.sq2), x);
#pragma unroll
        for (int e = 0; e < 8; ++e) vec[rr][ch * 8 + e] += x[e];
      }
    }
  }
  __syncthreads();
  {
    // In-block suffix scan, 256/D threads per dimension: each scans a
    // segment of 64*D/256 rows seeded with the later segments' totals.
    constexpr int TP = 256 / D, SEG = 64 / TP;
    const int d = threadIdx.x % D, part = threadIdx.x / D;
    float tot = 0.f;
#pragma unroll
    for (int rr = 0; rr < SEG; ++rr) tot += vec[part * SEG + rr][d];
    scratch[threadIdx.x] = tot;
    __syncthreads();
    float acc = seed[d];
    for (int j = TP - 1; j > part; --j) acc += scratch[d + j * D];
#pragma unroll
    for (int rr = SEG - 1; rr >= 0; --rr) {
      acc += vec[part * SEG + rr][d];
      vec[part * SEG + rr][d] = acc;
    }
  }
  __syncthreads();
  const int row = r0 + kslot;
  const int key = row + p.causal_off;
  if (row < p.M && key >= 0 && key < p.ncols) {
    const float dot = key_dot<E, D>(p, kbase, key, vec[kslot], part);
    if (part == 0) p.out[b * p.so0 + hk * p.so1 + (int64_t)key * p.so2] = dot * p.sm_scale;
  }
}

}  // namespace fas
