// Device-side building blocks shared by the gfx950 kernels: element traits
// (fp16 / bf16 MFMA and packing), buffer descriptors, the LDS tile layout and
// the MFMA operand fetches from it.
//
// MFMA used throughout: v_mfma_f32_32x32x16_{f16,bf16}.  Operand layout for
// lane l (c = l % 32, g = l / 32): A supplies row c, contraction indices
// 8g..8g+7; B supplies column c, the same contraction indices; the 32x32
// fp32 accumulator gives lane l column c and rows 8*(r/4) + 4g + r%4 for
// register r = 0..15.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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
typedef __fp16 fp16x4_lds __attribute__((__vector_size__(4 * sizeof(__fp16))));

#define FAS_LDS __attribute__((address_space(3)))

// Buffer descriptor word 3 for gfx9-family raw buffers.
constexpr int kRsrcWord3 = 0x00020000;
// Buffer access flags of the streaming score stores: nt (bit 1, non-temporal)
// with sc1 (bit 4, device scope).  Measured against nt alone at B1 H32 S4096
// D128 fp16: score writer 0.2323 -> 0.2293 ms, scores alone 0.2106 ->
// 0.2062 ms (averages of four alternating runs on one box).
constexpr int kAuxNT = 2 | 16;

struct F16 {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // acc + both halves of a packed pair (one v_dot2 against (1, 1)).  Row sums
  // of fp16-rounded softmax weights stay within a half-ulp (2^-12) of the
  // fp32 sum; bf16 (2^-9) would not, so only F16 sums packed weights.
  static constexpr bool kPackedRowSum = true;
  static __device__ __forceinline__ float sum2(uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), f16x2{(_Float16)1.f, (_Float16)1.f},
                                  acc, false);
  }
  // Round-to-nearest-even conversion of two floats packed lo | hi << 16.
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2));
  }
  static __device__ __forceinline__ uint16_t cvt(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
};

struct BF16 {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static constexpr bool kPackedRowSum = false;
  static __device__ __forceinline__ float sum2(uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x),
                                           bf16x2{(__bf16)1.f, (__bf16)1.f}, acc, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
  }
  static __device__ __forceinline__ uint16_t cvt(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __builtin_bit_cast(float, (uint32_t)x << 16);
  }
};

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }
__device__ __forceinline__ float pos_inf() { return __builtin_inff(); }
__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }
// The values of lanes l % 32 and l % 32 + 32, in every lane l: one
// v_permlane32_swap of x with itself (a VALU lane swap on gfx950, not an
// LDS-routed shuffle).  Both results pass through an empty asm: this
// compiler's InstCombine folds the intrinsic's second result into its first
// (it then adds or compares a register with itself).
__device__ __forceinline__ void lane_halves(float x, float& lo, float& hi) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  unsigned a = r[0], b = r[1];
  asm volatile("" : "+v"(a), "+v"(b));
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
// x combined with x of lane l ^ 32.
// (A select, not fmaxf: the asm outputs would otherwise be canonicalised
// first.)
__device__ __forceinline__ float xor32_max(float x) {
  float lo, hi;
  lane_halves(x, lo, hi);
  return lo > hi ? lo : hi;
}
__device__ __forceinline__ float xor32_add(float x) {
  float lo, hi;
  lane_halves(x, lo, hi);
  return lo + hi;
}
__device__ __forceinline__ float log2f_fast(float x) { return __builtin_amdgcn_logf(x); }

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Eight 16-bit elements of a 16-byte vector as floats.
template <class E>
__device__ __forceinline__ void unpack8(u32x4 v, float (&x)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    x[2 * w] = E::to_f32((uint16_t)(v[w] & 0xffffu));
    x[2 * w + 1] = E::to_f32((uint16_t)(v[w] >> 16));
  }
}

// Buffer descriptor as four SGPR words for inline assembly.
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes, kRsrcWord3};
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const FAS_LDS void*)p);
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Direct global -> LDS copy of 16 bytes per lane: lane l's bytes land at
// LDS byte address lds_base + 16*l (lds_base wave-uniform); out-of-range
// offsets write zeros.  Issued from inline assembly so the compiler neither
// tracks it nor inserts waits for it: the caller waits with vm_wait_all().
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
// dma16 with the non-temporal policy, for streams read once.
__device__ __forceinline__ void dma16_nt(i32x4 rsrc, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ void vm_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Lanes L0 and L1 of w take the wave-uniform values x0 and x1
// (v_writelane_b32).  x0 and x1 are typically a ballot just written by a
// vector compare; the compiler's hazard checks do not look into inline
// assembly, so the s_nop supplies the wait states between that write and
// the lane writes (without it a lane was measured to receive a stale
// register).
template <int L0, int L1>
__device__ __forceinline__ void write_lanes(uint32_t& w, uint32_t x0, uint32_t x1) {
  static_assert(L0 >= 0 && L0 < 64 && L1 >= 0 && L1 < 64, "lane out of range");
  asm volatile("s_nop 4\n\tv_writelane_b32 %0, %1, %3\n\tv_writelane_b32 %0, %2, %4"
               : "+v"(w)
               : "s"(x0), "s"(x1), "n"(L0), "n"(L1));
}
// Eight lanes at once, behind one s_nop: the 32-bit halves of four ballots
// b[0..3] go to lanes L[2i] (low half) and L[2i + 1] (high half).
template <int L0, int L1, int L2, int L3, int L4, int L5, int L6, int L7>
__device__ __forceinline__ void write_lanes8(uint32_t& w, const uint64_t (&b)[4]) {
  asm volatile(
      "s_nop 4\n\t"
      "v_writelane_b32 %0, %1, %9\n\tv_writelane_b32 %0, %2, %10\n\t"
      "v_writelane_b32 %0, %3, %11\n\tv_writelane_b32 %0, %4, %12\n\t"
      "v_writelane_b32 %0, %5, %13\n\tv_writelane_b32 %0, %6, %14\n\t"
      "v_writelane_b32 %0, %7, %15\n\tv_writelane_b32 %0, %8, %16"
      : "+v"(w)
      : "s"((uint32_t)b[0]), "s"((uint32_t)(b[0] >> 32)), "s"((uint32_t)b[1]),
        "s"((uint32_t)(b[1] >> 32)), "s"((uint32_t)b[2]), "s"((uint32_t)(b[2] >> 32)),
        "s"((uint32_t)b[3]), "s"((uint32_t)(b[3] >> 32)), "n"(L0), "n"(L1), "n"(L2), "n"(L3),
        "n"(L4), "n"(L5), "n"(L6), "n"(L7));
}

// Workgroup barrier ordering LDS only.  __syncthreads() is also a release
// fence for global memory, which makes every wave drain its outstanding
// global stores at each barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Raw buffer over [base, base + bytes): loads past the end return 0, stores
// past the end are dropped.  Offsets are 32-bit byte offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ void buf_store16(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store16_nt(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kAuxNT);
}
// The same with a wave-uniform scalar byte offset soff added to off.
__device__ __forceinline__ void buf_store16_nt(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off,
                                               uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, soff, kAuxNT);
}

// a ^ b ^ c in one instruction (v_bitop3_b32; 0x96 is the truth table of the
// three-way exclusive or over operand bytes 0xF0, 0xCC, 0xAA).
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

// Dropout keep decision for element index idx (mod 2^32): the first word of
// Philox4x32-6 on counter (x0, w1, 0, 0) under key (k0, k1), i.e. Triton's
// randint(seed, offset + idx, n_rounds=6) (triton/language/random.py:
// philox_impl, randint4x), which follows the Random123 Philox round
// (Salmon et al., SC'11): with products pa = A c0, pb = B c2,
//   (c0, c1, c2, c3) <- (hi(pb) ^ c1 ^ k0, lo(pb), hi(pa) ^ c3 ^ k1, lo(pa)),
// then the key advances by the Weyl increments.  Round 0's word-2 product is
// zero and round 1's word-0 product is wave-uniform (DropParams), so a
// weight costs 8 of the 12 products; each 32x32 product is one 64-bit
// multiply giving both halves, and the parts the last rounds do not use fold
// away.  The carry picks round 1's product through a select against zero of
// the host-made difference (one instruction per half; the uniform low half
// joins round 2's key).  Triton keeps the weight iff
// float(y) * 4.6566127342e-10 > p with y = x for x >= 0 (x the word as
// int32), -x - 1 otherwise; the host turns that into an interval of
// x mod 2^32.
template <class DP>
__device__ __forceinline__ bool dropout_keep(const DP& d, uint32_t idx) {
  const uint32_t x0 = d.off_lo + idx;
  const bool carry = x0 < d.carry_lim;
  const uint64_t p0 = (uint64_t)kPhiloxMulA * x0;                                  // round 0
  const uint64_t p1 = (uint64_t)kPhiloxMulB * ((uint32_t)(p0 >> 32) ^ d.k1);       // round 1
  uint32_t c0 = (uint32_t)(p1 >> 32) ^ (d.k0 + kPhiloxWeylA);
  uint32_t c1 = (uint32_t)p1;
  uint32_t c2 = xor3(d.r1_hi, (uint32_t)p0, carry ? d.r1_hi_carry : 0u);
  uint32_t c3 = carry ? d.r1_lo_carry : 0u;  // round 1's low half without d.r1_lo
  uint32_t k0 = d.k0 + 2u * kPhiloxWeylA, k1 = d.k1 + 2u * kPhiloxWeylB;
  {  // round 2, taking d.r1_lo with its key
    const uint64_t pa = (uint64_t)kPhiloxMulA * c0;
    const uint64_t pb = (uint64_t)kPhiloxMulB * c2;
    c0 = xor3((uint32_t)(pb >> 32), c1, k0);
    c2 = xor3((uint32_t)(pa >> 32), c3, k1 ^ d.r1_lo);
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    k0 += kPhiloxWeylA;
    k1 += kPhiloxWeylB;
  }
#pragma unroll
  for (int r = 3; r < 6; ++r) {
    const uint64_t pa = (uint64_t)kPhiloxMulA * c0;
    const uint64_t pb = (uint64_t)kPhiloxMulB * c2;
    c0 = xor3((uint32_t)(pb >> 32), c1, k0);
    c2 = xor3((uint32_t)(pa >> 32), c3, k1);
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    k0 += kPhiloxWeylA;
    k1 += kPhiloxWeylB;
  }
  return c0 - d.keep_lo < d.keep_span;
}

// Row permutation applied to MFMA operand rows (bits 2 and 3 swapped).  With
// it the 16 accumulator registers of lane l (g = l / 32) cover rows
// {16*(r/8) + 8g + r%8}: two runs of 8 consecutive rows, so a lane's values
// can leave as 16-byte vectors.
__device__ __forceinline__ int perm_row(int c) {
  return (c & 0x13) | ((c & 4) << 1) | ((c & 8) >> 1);
}
// Row index (within a 32-row block) of accumulator register r of lane group g.
__device__ __forceinline__ int acc_row(int r, int g) { return 16 * (r >> 3) + 8 * g + (r & 7); }

// LDS tile of 16-bit elements, `rows` x D, row-major with the 16-byte chunks
// of each row XOR-permuted by swz(row).  The permutation keeps both operand
// fetches below free of bank conflicts: 16 lanes reading one logical chunk
// from 16 consecutive rows (ds_read_b128), and 32 lanes reading 4 rows x 64
// bytes with the transposing ds_read_b64_tr_b16.
template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (D == 128) {
    return ((row & 3) << 2) | ((row >> 2) & 3);
  } else if constexpr (D == 64) {
    const int t = (row >> 1) & 7;
    return ((t & 1) << 2) | ((t >> 1) & 3);
  } else if constexpr (D == 32) {
    return (row >> 2) & 3;
  } else {
    return (row >> 3) & 1;
  }
}
// Element offset of (row, logical 16-byte chunk ch) in a swizzled tile.
template <int D>
__device__ __forceinline__ int tile_off(int row, int ch) {
  return row * D + ((ch ^ swz<D>(row)) << 3);
}

// LDS DMA of rows [r0, r0 + R) of a row-major (., D) 16-bit matrix into a
// swizzled R x D LDS tile at byte address lds: 1 KiB blocks dealt to the NW
// waves; lane l fills physical chunk l % (D/8) of its row, i.e. logical
// chunk (l % (D/8)) ^ swz(row).  Rows outside the buffer read as zeros.
template <int D, int R, int NW>
__device__ __forceinline__ void dma_tile(i32x4 rsrc, int64_t stride, int r0, uint32_t lds,
                                         int wave, int lane) {
  constexpr int BLOCKS = R * D / 512;
  constexpr int RPB = 512 / D;
  constexpr int CPR = D / 8;
  constexpr int PER = (BLOCKS + NW - 1) / NW;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int q = wave + i * NW;
    if (BLOCKS % NW == 0 || q < BLOCKS) {
      const int row = q * RPB + lane / CPR;
      const int ch = (lane % CPR) ^ swz<D>(row);
      dma16(rsrc, (uint32_t)(((r0 + row) * stride + ch * 8) * 2),
            __builtin_amdgcn_readfirstlane(lds + (uint32_t)(q * 1024)));
    }
  }
}

// A/B operand fetch for a contraction over the head dim: lane (c, g) gets
// elements [16*ks + 8g, +8) of tile row `row`.
template <int D>
__device__ __forceinline__ u32x4 lds_row_chunk(const uint16_t* tile, int row, int ks, int g) {
  return *reinterpret_cast<const u32x4*>(tile + tile_off<D>(row, 2 * ks + g));
}

// Transposing fetch of the A operand V^T for O^T += V^T P^T: rows of the
// MFMA are head dims (block db: dims 32db + perm_row(c)), contraction index
// 8g + e is key 16*cs + 8g + e of the tile.  ds_read_b64_tr_b16 hands lane i
// of each 16-lane group element i%4 of the 8-byte rows fetched by lanes
// i/4 + 4e; the fetch addresses below make that the column of 4 keys of one
// head dim.
template <int D>
__device__ __forceinline__ u32x4 lds_vt_operand(const uint16_t* vtile, int db, int cs, int lane) {
  const int g = lane >> 5, half = (lane >> 4) & 1, j = lane & 15;
  const int jj = j & 3;
  const int sw = ((jj & 1) << 1) | (jj >> 1);  // swap the two bits of j % 4
  int dim = 32 * db + 16 * half + 4 * sw;
  if constexpr (D < 32) dim &= D - 1;  // rows past the head dim duplicate (never stored)
  const int key = 16 * cs + 8 * g + (j >> 2);
  const int ch = dim >> 3, sub = dim & 7;
  const uint16_t* p0 = vtile + tile_off<D>(key, ch) + sub;
  const uint16_t* p1 = vtile + tile_off<D>(key + 4, ch) + sub;
  const fp16x4_lds r0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((FAS_LDS fp16x4_lds*)(p0));
  const fp16x4_lds r1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((FAS_LDS fp16x4_lds*)(p1));
  const u32x2 a = __builtin_bit_cast(u32x2, r0), b = __builtin_bit_cast(u32x2, r1);
  return u32x4{a.x, a.y, b.x, b.y};
}

// lds_vt_operand with its per-lane addressing reduced to two registers.  For
// every head dim the two byte offsets of block db, contraction step cs are
// those of (0, 0) XOR 64*db, plus 32*D*cs (checked exhaustively over lanes,
// blocks and steps): one v_xor per fetch instead of 2*DB offset registers
// held across the loop.  Callers pass the offsets through an empty asm per
// use region so the XORs are not hoisted back into registers.
struct VtOff {
  uint32_t o0, o1;
};
template <int D>
__device__ __forceinline__ VtOff vt_offsets(int lane) {
  const int g = lane >> 5, half = (lane >> 4) & 1, j = lane & 15;
  const int jj = j & 3;
  const int sw = ((jj & 1) << 1) | (jj >> 1);
  int dim = 16 * half + 4 * sw;
  if constexpr (D < 32) dim &= D - 1;
  const int key = 8 * g + (j >> 2);
  const int ch = dim >> 3, sub = dim & 7;
  return VtOff{(uint32_t)(2 * (tile_off<D>(key, ch) + sub)),
               (uint32_t)(2 * (tile_off<D>(key + 4, ch) + sub))};
}
template <int D>
__device__ __forceinline__ u32x4 lds_vt_operand(const uint16_t* vtile, VtOff o, int db, int cs) {
  const char* t = reinterpret_cast<const char*>(vtile) + 32 * D * cs;
  const uint32_t m = 64u * (uint32_t)db;
  const fp16x4_lds r0 =
      __builtin_amdgcn_ds_read_tr16_b64_v4f16((FAS_LDS fp16x4_lds*)(t + (o.o0 ^ m)));
  const fp16x4_lds r1 =
      __builtin_amdgcn_ds_read_tr16_b64_v4f16((FAS_LDS fp16x4_lds*)(t + (o.o1 ^ m)));
  const u32x2 a = __builtin_bit_cast(u32x2, r0), b = __builtin_bit_cast(u32x2, r1);
  return u32x4{a.x, a.y, b.x, b.y};
}
__device__ __forceinline__ void opaque(VtOff& o) { asm volatile("" : "+v"(o.o0), "+v"(o.o1)); }
// lds_row_chunk likewise: the byte offset of k-step ks is that of k-step 0
// XOR 32*ks (also checked exhaustively), and rows 16 apart differ by an
// immediate because swz depends on row bits 0-3 only.
template <int D>
__device__ __forceinline__ uint32_t row_chunk_offset(int row, int g) {
  return (uint32_t)(2 * tile_off<D>(row, g));
}
__device__ __forceinline__ u32x4 lds_row_chunk(const uint16_t* tile, uint32_t off, int ks) {
  return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(tile) +
                                         (off ^ (32u * (uint32_t)ks)));
}
__device__ __forceinline__ void opaque(uint32_t& o) { asm volatile("" : "+v"(o)); }

}  // namespace fas
