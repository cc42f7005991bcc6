// tbh_wave.h -- cross-lane reductions of a 64-lane wave on gfx950.
//
// Inside a 16-lane row the partners come from DPP lane permutations, which
// run in the VALU; the four row results are then read with v_readlane and
// combined as uniform values.  A chain of __shfl_xor steps would instead go
// through ds_bpermute, an LDS round trip per step.
#pragma once

#include <hip/hip_runtime.h>

namespace tbh {
namespace wave {

// gfx9 dpp_ctrl codes
enum : int {
    kXor1 = 0xB1,         // quad_perm [1,0,3,2]
    kXor2 = 0x4E,         // quad_perm [2,3,0,1]
    kHalfMirror = 0x141,  // lane l <- 7 - l within each 8-lane half row
    kRowMirror = 0x140,   // lane l <- 15 - l within the row
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                 false));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over each aligned group of 4 lanes, in every lane of the group.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<kXor1>(v);
    return v + dpp<kXor2>(v);
}

// Row total in every lane of each 16-lane row.
__device__ __forceinline__ float row_sum(float v) {
    v = quad_sum(v);
    v += dpp<kHalfMirror>(v);  // quads already reduced
    return v + dpp<kRowMirror>(v);  // halves already reduced
}

__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp<kXor1>(v));
    v = fmaxf(v, dpp<kXor2>(v));
    v = fmaxf(v, dpp<kHalfMirror>(v));
    return fmaxf(v, dpp<kRowMirror>(v));
}

// Wave total / maximum, the same value in every lane.
__device__ __forceinline__ float sum(float v) {
    v = row_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float max(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

}  // namespace wave
}  // namespace tbh
