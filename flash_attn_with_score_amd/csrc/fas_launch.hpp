// Host-side launchers of the gfx950 kernels.  Each family is instantiated in
// its own translation unit so the template instances compile in parallel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fas_params.hpp"

namespace fas {

// Forward pass (fas_fwd.hpp); mode is a FwdMode, dtype 0 = fp16, 1 = bf16.
hipError_t launch_fwd(const FwdParams& p, int mode, int dtype, int d, hipStream_t s);
// Query rows per forward workgroup (8 wave64s x 32 rows).
constexpr int kFwdRows = 256;

// Softmax-weight column sums after a forward pass that wrote lse2.
hipError_t launch_colsm(const ColsmParams& p, int dtype, int d, bool buffered, hipStream_t s);
// Raw-score column sums: block sums of q, suffix scan, per-key dot products.
hipError_t launch_rawsum(const RawParams& p, int dtype, bool suffix, hipStream_t s);

// Backward pass of attention(): prep, dK/dV (+ group reduction), dQ.
hipError_t launch_bwd(const BwdParams& p, int dtype, int d, hipStream_t s);
// Rows per dK/dV key block and per dQ row block of the backward kernels.
constexpr int kBwdBlock = 128;

// Scores alone, (q . k) * sm_scale, optionally masked (fas_scores.hpp).
hipError_t launch_scores(const ScoresParams& p, int dtype, int d, hipStream_t s);
// Keys per scores-only workgroup (4 key groups x 64 keys).
constexpr int kScoresKeysPerBlock = 256;
// Most query rows, and keys per block, of the resident-Q scores kernel
// (ScoresParams::ngrp > 0).
constexpr int kScoresResidentRows = 512;
constexpr int kScoresResidentKeys = 512;
// Bound on the resident-Q kernel's q and score offsets within a head group.
constexpr int64_t kScoresResidentBytes = 0x7ffffff0;

hipError_t launch_fill_zero(float* p, int64_t s0, int64_t s1, int64_t s2, int64_t n0, int64_t n1,
                            int64_t n2, hipStream_t s);

}  // namespace fas
