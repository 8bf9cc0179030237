// gfx950 (CDNA4) fused flash-attention-forward kernels with side products.
//
// One kernel template covers every variant of the reference's Triton family
// (attention_with_scores.py:23-211, attention_with_row_sum.py:22-202,
// attention_with_col_sum.py:22-294, attention_with_col_sum_sequential.py:23-211,
// attention_with_col_softmax_sum.py:23-270, attention_cross_token_qk_sum.py:17-252,
// attention_cross_token_softmax_sum.py:24-268 and :434-636).  The design is
// MI355X-first rather than a translation of those kernels:
//
//  * A workgroup is 4 wave64s and owns 128 query rows of one (batch, head);
//    each wave owns 32 rows.  Key/value tiles of 64 keys are staged in LDS
//    once per workgroup (K row-major, V transposed to [dim][key]) and
//    prefetched into registers one tile ahead.
//  * Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_{f16,bf16}; K comes from LDS, Q stays in VGPRs.
//    In the 32x32 accumulator layout lane l then holds one query row
//    (l % 32) and 16 keys per 32-key sub-block, so row max / row sum of the
//    online softmax are in-lane reductions plus one exchange with lane l^32.
//  * The output is accumulated transposed too, O^T = V^T P^T: P never leaves
//    the registers it was produced in (it is already in the B-operand
//    layout), and the per-row rescale alpha is a per-lane scalar.
//  * LDS rows are read through a permutation (bits 2 and 3 of the row index
//    swapped) so that each lane's accumulator values cover 8 consecutive
//    keys / dims: score and output stores are 16-byte vector stores.
//  * Column sums (over queries) use a 5-step butterfly across the 32 lanes
//    of a half-wave (31 exchanges for 32 values), then the 4 waves fold in
//    LDS, then one fp32 atomic per key per tile per workgroup.
//  * The score-materialising variant writes every element of its rows,
//    including the causal upper triangle as zeros, so the caller needs no
//    memset of the (B,H,M,N) matrix.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fas_launch.hpp"
#include "fas_params.hpp"

namespace fas {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = kBMHost;  // query rows per workgroup
constexpr int kBN = 64;       // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// fp16 element ops.
struct F16 {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even conversion of two floats, packed lo | hi << 16.
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    f16x2 h = __builtin_convertvector((f32x2){lo, hi}, f16x2);
    return __builtin_bit_cast(uint32_t, h);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
};

// bf16 element ops.
struct BF16 {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    bf16x2 h = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, h);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
};

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS row read by lane c of a half-wave: bits 2 and 3 swapped.  With it the
// 16 accumulator values of lane l (group g = l/32) of a 32x32 MFMA cover
// rows {16*(r/8) + 8*g + r%8 : r = 0..15}.
__device__ __forceinline__ int perm_row(int c) {
  return (c & 0x13) | ((c & 4) << 1) | ((c & 8) >> 1);
}

// Key (within a 64-key tile) of value idx = 16*kb + r (kb = 32-key
// sub-block, r = accumulator register) held by lane group g.
__device__ __forceinline__ int key_of(int idx, int g) {
  return 16 * (idx >> 3) + 8 * g + (idx & 7);
}

// Column sum of x[0..31] over the 32 lanes of each half-wave.  Each step
// halves the live values: a lane keeps the half its partner does not and
// adds the partner's copy.  Afterwards lane c of the half-wave holds the
// total of value index c.
__device__ __forceinline__ float col_butterfly(float (&x)[32], int c) {
#pragma unroll
  for (int step = 0; step < 5; ++step) {
    const int m = 16 >> step;
    const bool up = (c & m) != 0;
#pragma unroll
    for (int i = 0; i < m; ++i) {
      const float keep = up ? x[i + m] : x[i];
      const float send = up ? x[i] : x[i + m];
      x[i] = keep + __shfl_xor(send, m);
    }
  }
  return x[0];
}

// Register staging of one K/V tile (global -> VGPR -> LDS).
template <int D>
struct TileRegs {
  static constexpr int kChunksK = kBN * D / 8;                 // 16-byte chunks
  static constexpr int kItersK = (kChunksK + kThreads - 1) / kThreads;
  static constexpr int kItemsV = (kBN / 4) * (D / 8);          // 4 keys x 8 dims
  static constexpr int kItersV = (kItemsV + kThreads - 1) / kThreads;
  u32x4 k[kItersK];
  u32x4 v[kItersV][4];
};

template <int D>
__device__ __forceinline__ void load_k(TileRegs<D>& t, const uint16_t* __restrict__ K,
                                       int64_t stride, int k0, int n, int tid) {
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kItersK; ++i) {
    const int id = tid + i * kThreads;
    const int row = id / (D / 8), col = (id % (D / 8)) * 8;
    const int key = k0 + row;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (id < TileRegs<D>::kChunksK && key < n)
      val = *reinterpret_cast<const u32x4*>(K + (int64_t)key * stride + col);
    t.k[i] = val;
  }
}

template <int D>
__device__ __forceinline__ void load_v(TileRegs<D>& t, const uint16_t* __restrict__ V,
                                       int64_t stride, int k0, int n, int tid) {
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kItersV; ++i) {
    const int id = tid + i * kThreads;
    const int kg = id % (kBN / 4), dg = id / (kBN / 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = k0 + 4 * kg + r;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (id < TileRegs<D>::kItemsV && key < n)
        val = *reinterpret_cast<const u32x4*>(V + (int64_t)key * stride + dg * 8);
      t.v[i][r] = val;
    }
  }
}

template <int D, int KROW>
__device__ __forceinline__ void store_k(const TileRegs<D>& t, uint16_t* klds, int tid) {
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kItersK; ++i) {
    const int id = tid + i * kThreads;
    if (id < TileRegs<D>::kChunksK) {
      const int row = id / (D / 8), col = (id % (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(klds + row * KROW + col) = t.k[i];
    }
  }
}

// Writes V^T: element (key, dim) of the tile goes to vlds[dim * VROW + key].
// Each item packs the same dim of 4 consecutive keys into one 8-byte store.
template <int D, int VROW>
__device__ __forceinline__ void store_v(const TileRegs<D>& t, uint16_t* vlds, int tid) {
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kItersV; ++i) {
    const int id = tid + i * kThreads;
    if (id < TileRegs<D>::kItemsV) {
      const int kg = id % (kBN / 4), dg = id / (kBN / 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        uint32_t x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          x[r] = (e & 1) ? (t.v[i][r][w] >> 16) : (t.v[i][r][w] & 0xffffu);
        const u32x2 packed = {x[0] | (x[1] << 16), x[2] | (x[3] << 16)};
        *reinterpret_cast<u32x2*>(vlds + (dg * 8 + e) * VROW + kg * 4) = packed;
      }
    }
  }
}

__device__ __forceinline__ int tile_at(int it, int n, int order, int rb) {
  if (order == kOrderReverse) return n - 1 - it;
  if (order == kOrderRoundRobin) return (rb % n + it) % n;
  return it;
}

template <class E, int D, int MODE>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(const KParams p) {
  constexpr int KS = D / 16;            // MFMA k-steps over the head dim
  constexpr int DB = (D + 31) / 32;     // 32-row blocks of O^T
  constexpr int KROW = D + 8;           // LDS K row pitch (elements)
  constexpr int VROW = kBN + 8;         // LDS V^T row pitch (elements)
  constexpr bool kTwoPass = MODE == kModeColSoftmax || MODE == kModeCrossSoftmax ||
                            MODE == kModeCrossSoftmaxBuf;
  constexpr bool kRed1 = MODE == kModeColSum || MODE == kModeCrossQk;
  constexpr bool kRed2 = MODE == kModeColSoftmax || MODE == kModeCrossSoftmax;
  constexpr bool kCross = MODE == kModeCrossQk || MODE == kModeCrossSoftmax ||
                          MODE == kModeCrossSoftmaxBuf;

  __shared__ __attribute__((aligned(16))) uint16_t klds[kBN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vlds[DB * 32 * VROW];
  __shared__ float cred[(kRed1 || kRed2) ? kWaves * kBN : 1];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, c = lane & 31;

  // Block -> (row block, head, batch).  Causal row blocks run longest first.
  const int bh_count = p.B * p.H;
  const int bh = blockIdx.x % bh_count;
  int rb = blockIdx.x / bh_count;
  if (p.causal) rb = p.nrb - 1 - rb;
  const int h = bh % p.H, b = bh / p.H, hk = h / p.G;

  const int row0 = rb * kBM;
  const int wrow0 = row0 + wave * 32;
  const int qrow = wrow0 + c;
  const bool row_ok = qrow < p.M;

  const uint16_t* __restrict__ Q = p.q + b * p.sq0 + h * p.sq1;
  const uint16_t* __restrict__ K = p.k + b * p.sk0 + hk * p.sk1;
  const uint16_t* __restrict__ V = p.v + b * p.sv0 + hk * p.sv1;

  // Key range of the workgroup (hi) and of this wave (whi), tile-rounded.
  int hi = p.N, whi = p.N;
  if (p.causal) {
    hi = min(p.N, max(0, p.causal_off + row0 + kBM));
    whi = min(p.N, max(0, p.causal_off + wrow0 + 32));
  }
  const int ntiles = (hi + kBN - 1) / kBN;
  const int wtiles = (whi + kBN - 1) / kBN;
  const bool wave_partial_rows = wrow0 + 32 > p.M;

  // Cross-token region: rows in [split, M) (and keys < split).
  const bool wg_cross = kCross && max(row0, p.split) < min(row0 + kBM, p.M);
  const bool wave_cross = kCross && max(wrow0, p.split) < min(wrow0 + 32, p.M);

  // Q operand (B of S^T = K Q^T): lane holds Q[qrow][16*ks + 8*g .. +7].
  u32x4 qreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 val = {0u, 0u, 0u, 0u};
    if (row_ok) val = *reinterpret_cast<const u32x4*>(Q + (int64_t)qrow * p.sq2 + ks * 16 + 8 * g);
    qreg[ks] = val;
  }
  if constexpr (D < 32) {  // V^T rows past the head dim feed unused O^T rows
    for (int i = tid; i < (32 - D) * VROW; i += kThreads) vlds[D * VROW + i] = 0;
  }

  // Admissibility of (qrow, key) for the softmax.
  auto admissible = [&](int key) -> bool {
    return row_ok && key < p.N && (!p.causal || p.causal_off + qrow >= key);
  };

  // S^T for the current LDS tile: s[0] keys 0..31, s[1] keys 32..63.
  auto compute_s = [&](f32x16 (&s)[2]) {
    s[0] = f32x16{};
    s[1] = f32x16{};
    const uint16_t* kb = klds + perm_row(c) * KROW + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(kb + ks * 16);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(kb + 32 * KROW + ks * 16);
      s[0] = E::mma(a0, qreg[ks], s[0]);
      s[1] = E::mma(a1, qreg[ks], s[1]);
    }
  };

  float m_i = neg_inf(), l_i = 0.f, rsum = 0.f;
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};

  TileRegs<D> tr;
  // ------------------------------------------------------------- pass 1
  if (ntiles > 0) {
    const int t0 = tile_at(0, ntiles, p.order, rb);
    load_k<D>(tr, K, p.sk2, t0 * kBN, p.N, tid);
    load_v<D>(tr, V, p.sv2, t0 * kBN, p.N, tid);
    store_k<D, KROW>(tr, klds, tid);
    store_v<D, VROW>(tr, vlds, tid);
    __syncthreads();
  }
  for (int it = 0; it < ntiles; ++it) {
    const int t = tile_at(it, ntiles, p.order, rb);
    const int k0 = t * kBN;
    const bool has_next = it + 1 < ntiles;
    if (has_next) {
      const int tn = tile_at(it + 1, ntiles, p.order, rb);
      load_k<D>(tr, K, p.sk2, tn * kBN, p.N, tid);
      load_v<D>(tr, V, p.sv2, tn * kBN, p.N, tid);
    }
    const bool red_tile = kRed1 && (MODE == kModeColSum || (wg_cross && k0 < p.split));

    if (t < wtiles) {
      f32x16 s[2];
      compute_s(s);
      float sv[32];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sv[i] = s[0][i];
        sv[16 + i] = s[1][i];
      }
      const bool full = !(k0 + kBN > p.N || (p.causal && k0 + kBN - 1 > p.causal_off + wrow0) ||
                          wave_partial_rows);
      bool ok[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) ok[i] = full || admissible(k0 + key_of(i, g));

      if constexpr (MODE == kModeScores) {
        if (row_ok) {
          uint16_t* srow = p.scores + b * p.ss0 + h * p.ss1 + (int64_t)qrow * p.ss2;
#pragma unroll
          for (int j8 = 0; j8 < 4; ++j8) {
            const int key0 = k0 + 16 * j8 + 8 * g;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = ok[8 * j8 + e] ? sv[8 * j8 + e] * p.sm_scale : 0.f;
            if (p.vec_scores && key0 + 8 <= p.N) {
              const u32x4 w = {E::pack(v[0], v[1]), E::pack(v[2], v[3]), E::pack(v[4], v[5]),
                               E::pack(v[6], v[7])};
              __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(srow + key0));
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (key0 + e < p.N) srow[key0 + e] = E::cvt(v[e]);
            }
          }
        }
      }
      if constexpr (MODE == kModeRowSum) {
#pragma unroll
        for (int i = 0; i < 32; ++i) rsum += ok[i] ? sv[i] * p.sm_scale : 0.f;
      }
      if constexpr (kRed1) {
        if (red_tile) {
          float x[32];
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            bool use = ok[i];
            if constexpr (MODE == kModeCrossQk)
              use = use && row_ok && qrow >= p.split && k0 + key_of(i, g) < p.split;
            x[i] = use ? sv[i] * p.sm_scale : 0.f;
          }
          const float tot = col_butterfly(x, c);
          cred[wave * kBN + key_of(c, g)] = tot;
        }
      }
      if constexpr (MODE == kModeCrossSoftmaxBuf) {
        if (wave_cross && k0 < p.split && row_ok && qrow >= p.split) {
          float* brow = p.buf + b * p.sb0 + h * p.sb1 + (int64_t)(qrow - p.split) * p.sb2;
          const bool vec = (p.split & 3) == 0;
#pragma unroll
          for (int j8 = 0; j8 < 4; ++j8) {
            const int key0 = k0 + 16 * j8 + 8 * g;
            if (vec && key0 + 8 <= p.split) {
              const f32x4 lo = {sv[8 * j8 + 0], sv[8 * j8 + 1], sv[8 * j8 + 2], sv[8 * j8 + 3]};
              const f32x4 hi4 = {sv[8 * j8 + 4], sv[8 * j8 + 5], sv[8 * j8 + 6], sv[8 * j8 + 7]};
              *reinterpret_cast<f32x4*>(brow + key0) = lo;
              *reinterpret_cast<f32x4*>(brow + key0 + 4) = hi4;
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (key0 + e < p.split) brow[key0 + e] = sv[8 * j8 + e];
            }
          }
        }
      }

      // Online softmax (base 2 on raw scores) and O^T += V^T P^T.
      float mx = neg_inf();
#pragma unroll
      for (int i = 0; i < 32; ++i) mx = fmaxf(mx, ok[i] ? sv[i] : neg_inf());
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_i, mx);
      const float m_use = (m_new == neg_inf()) ? 0.f : m_new;
      const float alpha = fast_exp2((m_i - m_use) * p.qk_scale);
      const float nb = m_use * p.qk_scale;
      float psum = 0.f;
      u32x4 pb[4];
#pragma unroll
      for (int j8 = 0; j8 < 4; ++j8) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * j8 + e;
          pv[e] = ok[i] ? fast_exp2(fmaf(sv[i], p.qk_scale, -nb)) : 0.f;
          psum += pv[e];
        }
        pb[j8] = u32x4{E::pack(pv[0], pv[1]), E::pack(pv[2], pv[3]), E::pack(pv[4], pv[5]),
                       E::pack(pv[6], pv[7])};
      }
      l_i = l_i * alpha + psum;
      m_i = m_new;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        oacc[db] *= alpha;
        const uint16_t* vb = vlds + (32 * db + perm_row(c)) * VROW + 8 * g;
#pragma unroll
        for (int cs = 0; cs < 4; ++cs) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(vb + 16 * cs);
          oacc[db] = E::mma(a, pb[cs], oacc[db]);
        }
      }
    } else if (red_tile) {
      cred[wave * kBN + lane] = 0.f;
    }

    __syncthreads();
    if constexpr (kRed1) {
      if (red_tile && tid < kBN) {
        const float tot = cred[tid] + cred[kBN + tid] + cred[2 * kBN + tid] + cred[3 * kBN + tid];
        const int key = k0 + tid;
        const int lim = (MODE == kModeCrossQk) ? p.split : p.N;
        if (key < lim) unsafeAtomicAdd(p.aux + b * p.sa0 + hk * p.sa1 + (int64_t)key * p.sa2, tot);
      }
    }
    if (has_next) {
      store_k<D, KROW>(tr, klds, tid);
      store_v<D, VROW>(tr, vlds, tid);
    }
    __syncthreads();
  }

  // ------------------------------------------------------- pass 1 epilogue
  const float l_tot = l_i + __shfl_xor(l_i, 32);
  if (row_ok) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = p.o + b * p.so0 + h * p.so1 + (int64_t)qrow * p.so2;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int t8 = 0; t8 < 2; ++t8) {
        const int d0 = 32 * db + 16 * t8 + 8 * g;
        if (d0 < D) {
          const f32x16& o = oacc[db];
          const u32x4 w = {E::pack(o[8 * t8 + 0] * inv, o[8 * t8 + 1] * inv),
                           E::pack(o[8 * t8 + 2] * inv, o[8 * t8 + 3] * inv),
                           E::pack(o[8 * t8 + 4] * inv, o[8 * t8 + 5] * inv),
                           E::pack(o[8 * t8 + 6] * inv, o[8 * t8 + 7] * inv)};
          *reinterpret_cast<u32x4*>(orow + d0) = w;
        }
      }
    }
    if (p.lse != nullptr && g == 0)
      p.lse[b * p.sl0 + h * p.sl1 + (int64_t)qrow * p.sl2] =
          l_tot > 0.f ? m_i * p.sm_scale + __logf(l_tot) : neg_inf();
  }
  if constexpr (MODE == kModeRowSum) {
    const float r = rsum + __shfl_xor(rsum, 32);
    if (row_ok && g == 0) p.aux[b * p.sa0 + h * p.sa1 + (int64_t)qrow * p.sa2] = r;
  }

  // Causal score rows: keys past this wave's last computed tile are zero.
  if constexpr (MODE == kModeScores) {
    const int z0 = wtiles * kBN;
    if (z0 < p.N) {
      for (int rr = 0; rr < 32; ++rr) {
        const int row = wrow0 + rr;
        if (row >= p.M) break;
        uint16_t* srow = p.scores + b * p.ss0 + h * p.ss1 + (int64_t)row * p.ss2;
        if (p.vec_scores) {
          for (int key = z0 + lane * 8; key < p.N; key += 64 * 8) {
            if (key + 8 <= p.N) {
              __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, reinterpret_cast<u32x4*>(srow + key));
            } else {
              for (int e = key; e < p.N; ++e) srow[e] = 0;
            }
          }
        } else {
          for (int key = z0 + lane; key < p.N; key += 64) srow[key] = 0;
        }
      }
    }
  }

  // ------------------------------------------------------------- pass 2
  if constexpr (kTwoPass) {
    const float m_fin = (m_i == neg_inf()) ? 0.f : m_i;
    const float nb = m_fin * p.qk_scale;
    const float inv = (MODE == kModeColSoftmax) ? (l_tot > 0.f ? 1.f / l_tot : 0.f)
                                                : 1.f / (l_tot + 1e-12f);
    int ntiles2 = ntiles, wtiles2 = wtiles;
    bool wave_active = true;
    if constexpr (kCross) {
      ntiles2 = wg_cross ? (min(hi, p.split) + kBN - 1) / kBN : 0;
      wtiles2 = min(wtiles, ntiles2);
      wave_active = wave_cross;
    }
    auto weight = [&](float s, int key) -> float {
      bool use = admissible(key);
      if constexpr (kCross) use = use && qrow >= p.split && key < p.split;
      return use ? fast_exp2(fmaf(s, p.qk_scale, -nb)) * inv : 0.f;
    };

    if constexpr (MODE == kModeCrossSoftmaxBuf) {
      __threadfence();
      // Every lane re-reads exactly the scores it stored in pass 1.
      for (int it = 0; it < ntiles2; ++it) {
        const int t = tile_at(it, ntiles2, p.order2, rb);
        const int k0 = t * kBN;
        if (!(wave_active && t < wtiles2)) continue;
        float x[32];
        const bool rin = row_ok && qrow >= p.split;
        const float* brow = p.buf + b * p.sb0 + h * p.sb1 + (int64_t)(rin ? qrow - p.split : 0) * p.sb2;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int key = k0 + key_of(i, g);
          x[i] = (rin && key < p.split) ? weight(brow[key], key) : 0.f;
        }
        const float tot = col_butterfly(x, c);
        const int key = k0 + key_of(c, g);
        if (key < p.split) unsafeAtomicAdd(p.aux + b * p.sa0 + hk * p.sa1 + (int64_t)key * p.sa2, tot);
      }
    } else {
      if (ntiles2 > 0) {
        const int t0 = tile_at(0, ntiles2, p.order2, rb);
        load_k<D>(tr, K, p.sk2, t0 * kBN, p.N, tid);
        store_k<D, KROW>(tr, klds, tid);
        __syncthreads();
      }
      for (int it = 0; it < ntiles2; ++it) {
        const int t = tile_at(it, ntiles2, p.order2, rb);
        const int k0 = t * kBN;
        const bool has_next = it + 1 < ntiles2;
        if (has_next) {
          const int tn = tile_at(it + 1, ntiles2, p.order2, rb);
          load_k<D>(tr, K, p.sk2, tn * kBN, p.N, tid);
        }
        if (wave_active && t < wtiles2) {
          f32x16 s[2];
          compute_s(s);
          float x[32];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            x[i] = weight(s[0][i], k0 + key_of(i, g));
            x[16 + i] = weight(s[1][i], k0 + key_of(16 + i, g));
          }
          const float tot = col_butterfly(x, c);
          cred[wave * kBN + key_of(c, g)] = tot;
        } else {
          cred[wave * kBN + lane] = 0.f;
        }
        __syncthreads();
        if (tid < kBN) {
          const float tot = cred[tid] + cred[kBN + tid] + cred[2 * kBN + tid] + cred[3 * kBN + tid];
          const int key = k0 + tid;
          const int lim = kCross ? p.split : p.N;
          if (key < lim) unsafeAtomicAdd(p.aux + b * p.sa0 + hk * p.sa1 + (int64_t)key * p.sa2, tot);
        }
        if (has_next) store_k<D, KROW>(tr, klds, tid);
        __syncthreads();
      }
    }
  }
}

// Zero-fill of a strided (n0, n1, n2) fp32 accumulator, used instead of a
// memset so the whole launch sequence stays capturable in a HIP graph.
__global__ void fill_zero_3d(float* p, int64_t s0, int64_t s1, int64_t s2, int64_t n0, int64_t n1,
                             int64_t n2);

template <int MODE>
hipError_t launch_mode(const KParams& p, int dtype, int d, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)p.nrb * p.B * p.H)), block(kThreads);
  void* args[] = {const_cast<KParams*>(&p)};
  const void* fn = nullptr;
  if (dtype == 0) {
    switch (d) {
      case 16: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<F16, 16, MODE>); break;
      case 32: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<F16, 32, MODE>); break;
      case 64: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<F16, 64, MODE>); break;
      case 128: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<F16, 128, MODE>); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (d) {
      case 16: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<BF16, 16, MODE>); break;
      case 32: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<BF16, 32, MODE>); break;
      case 64: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<BF16, 64, MODE>); break;
      case 128: fn = reinterpret_cast<const void*>(&attn_fwd_kernel<BF16, 128, MODE>); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipLaunchKernel(fn, grid, block, args, 0, stream);
}

}  // namespace fas
