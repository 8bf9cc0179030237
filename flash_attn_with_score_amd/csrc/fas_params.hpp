// Kernel-side parameter block shared by the host dispatcher (fas_api.cpp)
// and the gfx950 kernels (fas_kernel.hpp).  Plain data only.
#pragma once
#include <stdint.h>

namespace fas {

// Query rows per workgroup; the host sizes the grid with it.
constexpr int kBMHost = 128;

// Side product a launch computes besides the attention output.
enum Mode : int {
  kModeScores = 0,         // full (B,Hq,M,N) score matrix, masked -> 0
  kModeRowSum = 1,         // (B,Hq,M) sum of scaled raw scores
  kModeColSum = 2,         // (B,Hk,N) sum of scaled raw scores
  kModeCrossQk = 3,        // (B,Hk,split) raw sum, rows >= split, keys < split
  kModeColSoftmax = 4,     // (B,Hk,N) sum of final softmax weights (2 passes)
  kModeCrossSoftmax = 5,   // (B,Hk,split) softmax-weight sum (2 passes)
  kModeCrossSoftmaxBuf = 6 // as 5, pass 2 reloads fp32 scores from scratch
};

// Order in which a workgroup visits its key tiles.  Only the fp32 summation
// order of the side products depends on it.
enum Order : int { kOrderForward = 0, kOrderReverse = 1, kOrderRoundRobin = 2 };

struct KParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;        // optional
  uint16_t* scores;  // kModeScores
  float* aux;        // row / column / cross sums
  float* buf;        // kModeCrossSoftmaxBuf scratch
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t sv0, sv1, sv2;
  int64_t so0, so1, so2;
  int64_t ss0, ss1, ss2;  // scores
  int64_t sa0, sa1, sa2;  // aux
  int64_t sl0, sl1, sl2;  // lse
  int64_t sb0, sb1, sb2;  // buf: (B, Hq, M - split, split)
  int B, H, G, M, N, split;
  int causal;      // 0/1
  int causal_off;  // key j admissible for query i iff causal_off + i >= j
  int order;       // pass-1 tile order (Order)
  int order2;      // pass-2 tile order (Order)
  int nrb;         // number of 128-row query blocks
  int vec_scores;  // 1 when every score row start is 16-byte aligned
  float sm_scale;
  float qk_scale;  // sm_scale * log2(e)
};

}  // namespace fas
