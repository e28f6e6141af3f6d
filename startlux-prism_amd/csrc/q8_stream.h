// Host side of the balanced-grid Q8_0 decode kernel (w8a8_q8_stream.hip), called by the packed Q8_0 entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// At most one workgroup per CU of the MI355X (256 CUs), and never more workgroups than 16-row weight tiles.
constexpr int kQ8StreamMaxWG = 256;

int q8_stream_workgroups(int64_t N, int64_t K);
// Workspace the kernel needs for N x K weights: one 64-bit handoff word per (workgroup, output of a 16 x 16 tile).
int64_t q8_stream_workspace_bytes(int64_t N, int64_t K);
// M in 1..16; hand: a zero-initialised workspace of at least q8_stream_workspace_bytes (left zeroed by every launch).
int q8_stream_launch(const int8_t* a, const float* a_s, int64_t as_sm, const int8_t* qt, const uint16_t* dt,
                     void* out, int64_t ldo, const int32_t* n_rows, int64_t M, int64_t N, int64_t K, int epi,
                     void* hand, int64_t hand_bytes, hipStream_t st);

}  // namespace prism
